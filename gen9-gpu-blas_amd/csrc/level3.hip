// Level 3 beyond GEMM: SYMM, SYRK, SYR2K, TRMM, TRSM, all on the MFMA GEMM kernels.
//
// Semantics follow the reference (reference: lib/src/level3.c, declarations lib/gen9blas.h:98-112; row-major, the
// uplo triangle of a symmetric or triangular A is the one read, diag = 1 means a unit diagonal that is not read):
// - SYMM: C = alpha·A·B + beta·C (left, A M×M) or alpha·B·A + beta·C (right, A N×N). As the reference (level3.c:
//   13-60), the symmetric matrix is first made explicit from its triangle (here into a device work buffer), then one
//   GEMM runs;
// - TRMM: B = alpha·op(A)·B (left) or alpha·B·op(A) (right). op(A) is made explicit with zeros outside its triangle;
//   one product then runs with each tile over only the k range where op(A) is non-zero (about half of the full work;
//   the reference uses 4 row or column bands, level3.c:28-49: 62 %), into a work buffer copied back to B;
// - SYRK / SYR2K: only the uplo triangle of C changes. One launch of the GEMM kernel in triangle mode covers the
//   tiles that meet the triangle and writes alpha·product + beta·C there (C not read when beta = 0), each element
//   rounded once; the reference runs row bands over the columns the triangle needs (level3.c:76-97) into a work
//   buffer that is merged afterwards. SYR2K joins X = [op(A) | op(B)] and Y = [op(B) | op(A)] so that
//   X·Yᵀ = op(A)·op(B)ᵀ + op(B)·op(A)ᵀ is one accumulation (level3.c:109-125);
// - TRSM: op(A)·X = alpha·B (left) or X·op(A) = alpha·B (right), X overwrites B. As the reference (level3.c:127-215)
//   the problem is brought to L·Y = alpha·R with L lower triangular (an upper matrix by reversing the index order,
//   the right side by transposition) and the diagonal blocks of L are inverted in FP64; the substitution then runs on
//   the GEMM kernels by recursive halving (the reference's per-block-row updates Y_i -= L[i, <i]·X[<i] grouped into a
//   few large products), each 128-row block finished by X_i = inv(L_ii)·Y_i.
// Products of the element type round as a GEMM does; the TRMM copy pass and SYMM's explicit matrix add no rounding
// (they copy elements of the element type).
#include "internal.h"
#include <algorithm>
#include <type_traits>

namespace g9 {
namespace l3 {

typedef long long ll;
typedef _Float16 f16;

template <class T> struct Acc { using S = float; };
template <> struct Acc<double> { using S = double; };

template <class F> static int by_es(int es, F f) {
    if (es == 2) return f((f16 *)nullptr);
    if (es == 4) return f((float *)nullptr);
    return f((double *)nullptr);
}

static unsigned grid_for(ll n) {
    const ll g = (n + 255) / 256, cap = (ll)(num_cus > 0 ? num_cus : 256) * 16;
    return (unsigned)(g < 1 ? 1 : g > cap ? cap : g);
}

// F (n×n, row stride n) = the full matrix G built from the uplo triangle of A (tr: F = Gᵀ). sym: G mirrored from the
// triangle; otherwise triangular with zeros outside it and, with unit, ones on the diagonal.
template <class T>
__global__ void __launch_bounds__(256) expand_kernel(const T *A, ll lda, T *F, int n, int lower, int sym, int unit, int tr) {
    const ll nn = (ll)n * n;
    for (ll e = blockIdx.x * 256ll + threadIdx.x; e < nn; e += (ll)gridDim.x * 256) {
        const int i = (int)(e / n), j = (int)(e % n);
        const int p = tr ? j : i, q = tr ? i : j;   // F[i][j] = G[p][q]
        const bool in = lower ? q <= p : q >= p;
        T v;
        if (sym) v = in ? A[(ll)p * lda + q] : A[(ll)q * lda + p];
        else v = in ? ((p == q && unit) ? T(1) : A[(ll)p * lda + q]) : T(0);
        F[e] = v;
    }
}

// C = P + beta·C on the lower (or upper) triangle of the N×N matrix C (C not read when beta = 0; P null: zero).
template <class T>
__global__ void __launch_bounds__(256) merge_kernel(const T *P, ll ldp, T *C, ll ldc, int N, int lower,
                                                    typename Acc<T>::S beta) {
    using S = typename Acc<T>::S;
    const ll nn = (ll)N * N;
    for (ll e = blockIdx.x * 256ll + threadIdx.x; e < nn; e += (ll)gridDim.x * 256) {
        const int i = (int)(e / N), j = (int)(e % N);
        if (lower ? j > i : j < i) continue;
        S v = P ? (S)P[(ll)i * ldp + j] : S(0);
        T *c = C + (ll)i * ldc + j;
        if (beta != S(0)) v += beta * (S)*c;
        *c = (T)v;
    }
}

// X = [op(A) | op(B)], Y = [op(B) | op(A)], both N×2K with row stride 2K (op: A stored K×N when trans).
template <class T>
__global__ void __launch_bounds__(256) join_kernel(const T *A, ll lda, const T *B, ll ldb, T *X, T *Y, int N, int K, int trans) {
    const ll k2 = 2ll * K, tot = (ll)N * k2;
    for (ll e = blockIdx.x * 256ll + threadIdx.x; e < tot; e += (ll)gridDim.x * 256) {
        const int i = (int)(e / k2), c = (int)(e % k2), k = c < K ? c : c - K;
        const T a = trans ? A[(ll)k * lda + i] : A[(ll)i * lda + k];
        const T b = trans ? B[(ll)k * ldb + i] : B[(ll)i * ldb + k];
        X[e] = c < K ? a : b;
        Y[e] = c < K ? b : a;
    }
}

// TRSM set-up: L (n×n lower) from op'(A) = (tr ? Aᵀ : A) restricted to the triangle of A (uplo), reversed in both
// indices when rev; unit: ones on the diagonal.
template <class T>
__global__ void __launch_bounds__(256) trsm_l_kernel(const T *A, ll lda, T *L, int n, int lower, int tr, int unit, int rev) {
    const ll nn = (ll)n * n;
    for (ll e = blockIdx.x * 256ll + threadIdx.x; e < nn; e += (ll)gridDim.x * 256) {
        const int i = (int)(e / n), j = (int)(e % n);
        const int p = rev ? n - 1 - i : i, q = rev ? n - 1 - j : j;   // element (p, q) of op'(A)
        const int r = tr ? q : p, c = tr ? p : q;                      // = A[r][c]
        const bool in = lower ? c <= r : c >= r;
        L[e] = in ? ((r == c && unit) ? T(1) : A[(ll)r * lda + c]) : T(0);
    }
}
// Y (n×m, row stride m) = alpha·R with R = B (left, M×N = n×m) or Bᵀ (right), rows reversed when rev.
template <class T>
__global__ void __launch_bounds__(256) trsm_y_kernel(const T *B, ll ldb, T *Y, int n, int m, int left, int rev,
                                                     typename Acc<T>::S alpha) {
    using S = typename Acc<T>::S;
    const ll nm = (ll)n * m;
    for (ll e = blockIdx.x * 256ll + threadIdx.x; e < nm; e += (ll)gridDim.x * 256) {
        const int i = (int)(e / m), j = (int)(e % m), p = rev ? n - 1 - i : i;
        const T b = left ? B[(ll)p * ldb + j] : B[(ll)j * ldb + p];
        Y[e] = (T)(alpha * (S)b);
    }
}
// B rows (byte stride ldb_bytes) = the rows of Z (n rows of cpr 16-byte chunks, contiguous): the solution of a left
// solve in its own order, 16 bytes per lane (both row strides and both pointers 16-byte aligned; the caller checks).
__global__ void __launch_bounds__(256) trsm_store_rows16_kernel(const uint4 *Z, char *B, ll ldb_bytes, int n, int cpr) {
    const ll tot = (ll)n * cpr;
    for (ll e = blockIdx.x * 256ll + threadIdx.x; e < tot; e += (ll)gridDim.x * 256) {
        const ll i = e / cpr, c = e - i * cpr;
        *(uint4 *)(B + i * ldb_bytes + c * 16) = Z[e];
    }
}
// B = X from Y (inverse of trsm_y_kernel's index map, without alpha).
template <class T>
__global__ void __launch_bounds__(256) trsm_store_kernel(const T *Y, T *B, ll ldb, int n, int m, int left, int rev) {
    const ll nm = (ll)n * m;
    for (ll e = blockIdx.x * 256ll + threadIdx.x; e < nm; e += (ll)gridDim.x * 256) {
        const int i = (int)(e / m), j = (int)(e % m), p = rev ? n - 1 - i : i;
        if (left) B[(ll)p * ldb + j] = Y[e];
        else B[(ll)j * ldb + p] = Y[e];
    }
}

constexpr int TRSM_NB = 128;
// rows of a leaf (an inverted diagonal block applied by one product) of the FP32 and the FP64 solve: one more
// composition level and half the leaves for FP64 (n = 4096 left lower, MI355X: 1.427 -> 1.412 ms with 1024 rows
// against 512; FP32 stays at 512: 0.729 against 0.823 ms when measured)
constexpr int TRSM_LEAF_S = 512, TRSM_LEAF_D = 1024;
// Inverse of the diagonal block bi of L (rows and columns r0 .. r0+b-1, b ≤ TRSM_NB, in the leaf p = r0 / lb of lb
// rows whose element (i, j) is at L[p·bstride + i·ld + j]; the block's entries above the diagonal are read as zeros,
// and its diagonal as ones when unit),
// in FP64, stored in the element type into the inverted diagonal block of lb rows (lb a multiple of TRSM_NB) that
// holds it: leaf p = r0 / lb at Inv + p·istride, row stride lb, at row and column offset o = r0 − p·lb. Each block
// also writes zeros right of itself up to the end of its leaf (or column n), so that everything above the leaf's
// diagonal is zero once the parts below its diagonal blocks are composed. The block is split into 32×32 sub-blocks: the four diagonal sub-blocks are inverted first, thread j
// forming column j of its sub-block by substitution (X[j][j] = 1 / L[j][j], X[i][j] = −(Σ_{k=j}^{i-1}
// L[i][k]·X[k][j]) / L[i][i]) from copies of those sub-blocks in LDS (placed, with one round of loads, in regions of
// X that are filled only later); the off-diagonal sub-blocks then follow by distance d from the diagonal,
// X_ij = −inv(L_ii)·Σ_{k=j}^{i-1} L_ik·X_kj (i − j = d), both products on the FP64 matrix cores (below). No thread runs
// a column chain of the whole block (8128 FMAs); the sums differ from plain column substitution in FP64 rounding
// only. X lives in LDS (132 KiB).
template <class T>
__global__ void __launch_bounds__(256) trsm_inv_kernel(const T *L, ll ld, ll bstride, int n, T *Inv, int lb, ll istride,
                                                        int unit) {
    constexpr int S = 32, NSB = TRSM_NB / S;
    static_assert(NSB == 4, "four diagonal sub-blocks, staged in the lower regions (1,0), (2,0), (3,0), (3,1)");
    __shared__ double X[TRSM_NB][TRSM_NB + 1];
    const int bi = blockIdx.x, r0 = bi * TRSM_NB, b = min(TRSM_NB, n - r0), t = threadIdx.x;
    const T *Lb = L + (ll)(r0 / lb) * bstride + (ll)(r0 % lb) * (ld + 1);   // element (i, j) of the block at Lb[i·ld + j]
    // region of X holding the copy of diagonal sub-block s of L until a level d ≥ 1 below overwrites it
    const auto stage_row = [](int s) { return S * (s < 3 ? s + 1 : 3); };
    const auto stage_col = [](int s) { return S * (s < 3 ? 0 : 1); };
    // The off-diagonal levels below are tasks (j, J) of wave wv: task = wv + 4·round, j = task / 2, J = task % 2, and
    // their operands from L are rows i·32 + 16h + lane % 16, columns j·32 + 4q + lane / 16 (i = j + d; addresses
    // clamped into the block, values outside it not used). Level 1's are loaded here with the gather's, level d + 1's
    // before level d runs, so that their latency is hidden (all three levels' at once need 256 registers and slow the
    // diagonal inverses down).
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6), lr = t & 15, lg = (t & 63) >> 4;
    const auto load_task = [&](auto dc, int task, auto &lv) {
        constexpr int d = decltype(dc)::value, KS4 = d * S / 4;
        const int j = task >> 1, i = j + d;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const T *li = Lb + (ll)min(i * S + 16 * h + lr, b - 1) * ld;
#pragma unroll
            for (int q = 0; q < KS4; q++) lv[h][q] = li[min(j * S + 4 * q + lg, b - 1)];
        }
    };
    using D1 = std::integral_constant<int, 1>;
    using D2 = std::integral_constant<int, 2>;
    using D3 = std::integral_constant<int, 3>;
    T l1[2][2][S / 4], l2[2][2 * S / 4], l3[2][3 * S / 4];   // level 1: a second task for waves 0, 1; level 3: waves 0, 1
    load_task(D1(), wv, l1[0]);
    if (wv + 4 < 2 * (NSB - 1)) load_task(D1(), wv + 4, l1[1]);
    {
        constexpr int PER = NSB * S * S / 256;
        T v[PER];   // every load in flight, from addresses clamped into the block
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const int e = u * 256 + t, sb = e / (S * S), i = sb * S + (e / S) % S, k = sb * S + e % S;
            v[u] = Lb[(ll)min(i, b - 1) * ld + min(k, b - 1)];
        }
        for (int e = t; e < TRSM_NB * TRSM_NB; e += 256) X[e / TRSM_NB][e % TRSM_NB] = 0.0;
        __syncthreads();
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const int e = u * 256 + t, sb = e / (S * S), ii = (e / S) % S, kk = e % S;
            const int i = sb * S + ii, k = sb * S + kk;
            // entries above the diagonal read as zero and, with a unit diagonal, the diagonal as one, so L may be the
            // caller's matrix itself (whose other triangle and diagonal are not referenced)
            const double lv = kk > ii ? 0.0 : (kk == ii && unit) ? 1.0 : (double)v[u];
            X[stage_row(sb) + ii][stage_col(sb) + kk] = i < b && k < b ? lv : 0.0;
        }
    }
    __syncthreads();
    if (t < TRSM_NB && t < b) {
        // column j of diagonal sub-block sb in registers, rows i (local) at compile-time indices: x_i = 0 above the
        // diagonal (i < jj), 1 / L(i, i) on it, −(Σ_{k<i} L(i, k)·x_k) / L(i, i) below, for rows inside the block
        const int j = t, sb = j / S, jj = j % S, nrow = min(b - sb * S, S);
        const double *Ls = &X[stage_row(sb)][stage_col(sb)];   // L(sb·32 + i, sb·32 + k) at Ls[i·(TRSM_NB + 1) + k]
        double x[S];
#pragma unroll
        for (int i = 0; i < S; i++) {
            const double *li = Ls + i * (TRSM_NB + 1);
            double s = 0.0;
#pragma unroll
            for (int k = 0; k < i; k++) s = __builtin_fma(li[k], x[k], s);
            const double v = i == jj ? 1.0 / li[i] : -s / li[i];
            x[i] = i < jj || i >= nrow ? 0.0 : v;
        }
#pragma unroll
        for (int i = 0; i < S; i++) X[sb * S + i][j] = x[i];
    }
    __syncthreads();
    // Off-diagonal sub-blocks by distance d from the diagonal, on the matrix cores (v_mfma_f64_16x16x4f64: lane l
    // supplies A[l % 16][k = l / 16] and B[k = l / 16][l % 16]; accumulator r of lane l holds D[4r + l / 16][l % 16]).
    // Task (j, J) of level d forms columns j·32 + 16J .. + 15 of X_(i, j), i = j + d, as two 16-row halves:
    // S = Σ_k L_(i, k)·X_(k, j) over the d·32 columns k of blocks j .. i − 1 (d·8 steps; L from the registers loaded
    // above, zero outside the block, X from LDS), then X_(i, j) = −inv(L_(i, i))·S with S taken straight from the accumulators:
    // accumulator r of half kh holds rows 16kh + 4r + l / 16 of S, which is the second operand's k of that step. A
    // level's tasks read only blocks of earlier levels and write distinct blocks.
    typedef double f64x4 __attribute__((ext_vector_type(4)));
    const auto task_run = [&](auto dc, int task, const auto &lv) {
        constexpr int d = decltype(dc)::value, KS4 = d * S / 4;
        const int j = task >> 1, J = task & 1, i = j + d, c0 = j * S + 16 * J;
        f64x4 sacc[2] = {{0.0, 0.0, 0.0, 0.0}, {0.0, 0.0, 0.0, 0.0}};
#pragma unroll
        for (int q = 0; q < KS4; q++) {
            const int k = j * S + 4 * q + lg;
            const double xb = X[k][c0 + lr];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const double a = i * S + 16 * h + lr < b && k < b ? (double)lv[h][q] : 0.0;
                sacc[h] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, xb, sacc[h], 0, 0, 0);
            }
        }
        f64x4 pacc[2] = {{0.0, 0.0, 0.0, 0.0}, {0.0, 0.0, 0.0, 0.0}};
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int kh = 0; kh < 2; kh++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const double a = X[i * S + 16 * h + lr][i * S + 16 * kh + 4 * r + lg];
                    pacc[h] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, sacc[kh][r], pacc[h], 0, 0, 0);
                }
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = i * S + 16 * h + 4 * r + lg, col = c0 + lr;
                if (row < b && col < b) X[row][col] = -pacc[h][r];
            }
    };
    load_task(D2(), wv, l2);
    task_run(D1(), wv, l1[0]);
    if (wv + 4 < 2 * (NSB - 1)) task_run(D1(), wv + 4, l1[1]);
    __syncthreads();
    if (wv < 2 * (NSB - 3)) load_task(D3(), wv, l3);
    task_run(D2(), wv, l2);
    __syncthreads();
    if (wv < 2 * (NSB - 3)) task_run(D3(), wv, l3);
    __syncthreads();
    // the block's rows from its diagonal to the end of its leaf: the inverse, then zeros (w ≤ lb columns)
    const int p = r0 / lb, o = r0 - p * lb, w = min(lb, n - p * lb) - o;
    T *out = Inv + (ll)p * istride + (ll)o * lb + o;
    // thread t writes columns t, t + 256, ... of the block's rows, 8 rows' LDS reads at a time
    for (int c = t; c < w; c += 256) {
        const int jc = min(c, TRSM_NB - 1);
        for (int i0 = 0; i0 < b; i0 += 8) {
            double v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = X[min(i0 + u, TRSM_NB - 1)][jc];
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (i0 + u < b) out[(ll)(i0 + u) * lb + c] = c < b ? (T)v[u] : T(0);
        }
    }
}

// count GEMMs on device operands (no staging, no wait): C_z = alpha·op(A_z)·op(B_z) + beta·C_z, X_z = X + z·sX.
static int dgemm_dev_batched(int type, int tA, int tB, int M, int N, int K, double alpha, const void *A, ll lda, ll sA,
                             const void *B, ll ldb, ll sB, double beta, void *C, ll ldc, ll sC, int count) {
    if (M <= 0 || N <= 0 || K <= 0 || count <= 0) return 0;
    GemmCall g;
    g.type = type;
    g.tA = tA; g.tB = tB;
    g.M = M; g.N = N; g.K = K;
    g.count = count;
    g.alpha = alpha; g.beta = beta;
    g.A = A; g.lda = lda; g.sA = sA;
    g.B = B; g.ldb = ldb; g.sB = sB;
    g.C = C; g.ldc = ldc; g.sC = sC;
    return launch_gemm(g);
}
static int dgemm_dev(int type, int tA, int tB, int M, int N, int K, double alpha, const void *A, ll lda, const void *B,
                     ll ldb, double beta, void *C, ll ldc) {
    return dgemm_dev_batched(type, tA, tB, M, N, K, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0, 1);
}

// Blocked forward substitution L·X = alpha·Y (L n×n lower, Y and X n×m, row strides ldl, ldy and m; alpha is applied
// by the first product that touches each block of rows of Y, or is 1 when Y already holds alpha·R) over diagonal blocks of lb
// rows (TRSM_LEAF_S / TRSM_LEAF_D for FP32 / FP64, 128 for FP16), by recursive halving: the first half of a block range is solved, one
// GEMM then subtracts its contribution from the right-hand side of the second half, Y[i1..i2) -= L[i1..i2, i0..i1)·
// X[i0..i1), and the second half is solved. A single block is X_i = inv(L_ii)·Y_i with the block's inverse (128-row
// inverses computed in FP64, larger ones composed from them; element (i, j) of the inverses at Iv[i·lb + j]), a product
// whose tiles take only the k range where the lower-triangular inverse is non-zero. The reference updates one block row at a time,
// Y_i -= L[i, <i]·X[<i] (level3.c:127-215): the same products, grouped so that most of the flops run in a few large
// GEMMs instead of n/128 products of 128 rows; the sums differ only in rounding (each GEMM rounds once).
struct TrsmSolve {
    int type, n, m, es, lb;   // lb: rows of an inverted diagonal block (leaf)
    const char *L, *Iv;
    char *Y, *X;
    ll ldl, ldy;              // row strides of L and Y (X: m)
    double alpha;             // applied by the first product that touches a row block of Y (1 when Y holds alpha·R)
    int solve(int b0, int nb) const {   // leaves [b0, b0 + nb)
        if (nb == 1) {
            const int i0 = b0 * lb, b = n - i0 < lb ? n - i0 : lb;
            // only leaf 0's rows of Y are still unscaled when it is solved
            GemmCall g;
            g.type = type;
            g.tA = g.tB = 0;
            g.M = b; g.N = m; g.K = b;
            g.count = 1;
            g.alpha = b0 == 0 ? alpha : 1.0; g.beta = 0.0;
            g.A = Iv + (ll)i0 * (lb + 1) * es; g.lda = lb; g.sA = 0;
            g.B = Y + (ll)i0 * ldy * es; g.ldb = ldy; g.sB = 0;
            g.C = X + (ll)i0 * m * es; g.ldc = m; g.sC = 0;
            return lb > TRSM_NB ? launch_gemm_klim(g, 1) : launch_gemm(g);
        }
        const int h = nb / 2;
        G9_TRY(solve(b0, h));
        const int i0 = b0 * lb, i1 = (b0 + h) * lb, i2 = n < (b0 + nb) * lb ? n : (b0 + nb) * lb;
        // rows i1 .. i2 are first touched here when the range starts at row 0 (an enclosing range updates its second
        // half only after solving its first): Y = alpha·Y − L·X then, Y −= L·X after
        G9_TRY(dgemm_dev(type, 0, 0, i2 - i1, m, i1 - i0, -1.0, L + ((ll)i1 * ldl + i0) * es, ldl, X + (ll)i0 * m * es, m,
                         b0 == 0 ? alpha : 1.0, Y + (ll)i1 * ldy * es, ldy));
        return solve(b0 + h, nb - h);
    }
};

static int check_type(int type) {
    if (type < 0 || type > 3) G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "type %d unavailable", type);
    return 0;
}

// Triangle (lower / upper) of C = alpha·X·Yᵀ + beta·C for device X, Y (N×K, or stored K×N when trans) and resolved C.
static int tri_product(int type, int lower, int trans, int N, int K, double alpha, const void *X, ll ldx, const void *Y,
                       ll ldy, double beta, void *C, ll ldc) {
    const int es = elem_size(type);
    if (K > 0 && alpha != 0.0) {
        // one launch over the tiles of the triangle: C = alpha·op(X)·op(Y)ᵀ + beta·C there, rounded once
        GemmCall g;
        g.type = type;
        g.tA = trans; g.tB = !trans;
        g.M = N; g.N = N; g.K = K;
        g.count = 1;
        g.alpha = alpha; g.beta = beta;
        g.A = X; g.lda = ldx; g.sA = 0;
        g.B = Y; g.ldb = ldy; g.sB = 0;
        g.C = C; g.ldc = ldc; g.sC = 0;
        return launch_gemm_tri(g, lower != 0);
    }
    return by_es(es, [&](auto *tag) -> int {
        using T = std::remove_pointer_t<decltype(tag)>;
        using S = typename Acc<T>::S;
        hipLaunchKernelGGL((merge_kernel<T>), dim3(grid_for((ll)N * N)), dim3(256), 0, stream, (const T *)nullptr, (ll)N,
                           (T *)C, ldc, N, lower, (S)beta);
        G9_HIP(hipGetLastError());
        return 0;
    });
}

}  // namespace l3

// The 128-row diagonal blocks of `count` / (lb / 128) lower-triangular leaves of lb rows for the level-2 solves: leaf
// p's element (i, j) at L[p·bstride + i·ld + j] (es 4: float, 8: double); inverses into Inv as trsm_inv_kernel
// places them (leaf p at Inv + p·istride, row stride lb, zeros right of each block's inverse to the end of its leaf).
int launch_tri_inverse(int es, const void *L, long long ld, long long bstride, int count, void *Inv, int lb,
                       long long istride, int unit) {
    using namespace l3;
    const int n = count * TRSM_NB;
    if (es == 8)
        hipLaunchKernelGGL((trsm_inv_kernel<double>), dim3(count), dim3(256), 0, stream, (const double *)L, (ll)ld,
                           (ll)bstride, n, (double *)Inv, lb, (ll)istride, unit);
    else
        hipLaunchKernelGGL((trsm_inv_kernel<float>), dim3(count), dim3(256), 0, stream, (const float *)L, (ll)ld,
                           (ll)bstride, n, (float *)Inv, lb, (ll)istride, unit);
    G9_HIP(hipGetLastError());
    return 0;
}

}  // namespace g9

using namespace g9;
using namespace g9::l3;

extern "C" {

int gen9blas_symm(int type, int side, int uplo, int M, int N, double alpha, const void *A, int lda, const void *B, int ldb,
                  double beta, void *C, int ldc) {
    G9_TRY(begin());
    G9_TRY(check_type(type));
    if (M <= 0 || N <= 0) return 0;
    const int left = side == GEN9BLAS_LEFT, n = left ? M : N, es = elem_size(type);
    if (!A || !B || !C) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "symm: NULL matrix pointer");
    if (lda < n || ldb < N || ldc < N)
        G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "symm: leading dimension too small (lda %d, ldb %d, ldc %d)", lda, ldb, ldc);
    Operand oa;
    oa.host = A; oa.es = es; oa.rows = n; oa.cols = n; oa.caller_ld = lda;
    G9_TRY(resolve(oa, SLOT_A, true, false, true));
    void *F;
    G9_TRY(scratch(SLOT_T, (size_t)n * n * es, &F));
    G9_TRY(by_es(es, [&](auto *tag) -> int {
        using T = std::remove_pointer_t<decltype(tag)>;
        hipLaunchKernelGGL((expand_kernel<T>), dim3(grid_for((ll)n * n)), dim3(256), 0, stream, (const T *)oa.dev, oa.ld,
                           (T *)F, n, uplo == GEN9BLAS_LOWER, 1, 0, 0);
        G9_HIP(hipGetLastError());
        return 0;
    }));
    if (left) return gemm_impl(type, 0, 0, M, N, M, alpha, F, n, 0, B, ldb, 0, beta, C, ldc, 0, 1);
    return gemm_impl(type, 0, 0, M, N, N, alpha, B, ldb, 0, F, n, 0, beta, C, ldc, 0, 1);
}

int gen9blas_trmm(int type, int side, int uplo, int transA, int diag, int M, int N, double alpha, const void *A, int lda,
                  void *B, int ldb) {
    G9_TRY(begin());
    G9_TRY(check_type(type));
    if (M <= 0 || N <= 0) return 0;
    const int left = side == GEN9BLAS_LEFT, n = left ? M : N, es = elem_size(type);
    if (!A || !B) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "trmm: NULL matrix pointer");
    if (lda < n || ldb < N) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "trmm: leading dimension too small (lda %d, ldb %d)", lda, ldb);
    Operand ops[2];
    ops[0].host = A; ops[0].es = es; ops[0].rows = n; ops[0].cols = n; ops[0].caller_ld = lda;
    ops[1].host = B; ops[1].es = es; ops[1].rows = M; ops[1].cols = N; ops[1].caller_ld = ldb;
    G9_TRY(resolve(ops[0], SLOT_A, true, false, true));
    G9_TRY(resolve(ops[1], SLOT_B, true, true, true));
    last_zc = (ops[0].zc ? 1 : 0) | (ops[1].zc ? 2 | 4 : 0);
    void *F, *Z;
    G9_TRY(scratch(SLOT_T, (size_t)n * n * es, &F));
    G9_TRY(scratch(SLOT_X, (size_t)M * N * es, &Z));
    const int tr = transA != 0, lower = (uplo == GEN9BLAS_LOWER) != tr;   // F = op(A) is lower triangular?
    G9_TRY(by_es(es, [&](auto *tag) -> int {
        using T = std::remove_pointer_t<decltype(tag)>;
        hipLaunchKernelGGL((expand_kernel<T>), dim3(grid_for((ll)n * n)), dim3(256), 0, stream, (const T *)ops[0].dev,
                           ops[0].ld, (T *)F, n, uplo == GEN9BLAS_LOWER, 0, diag != 0, tr);
        G9_HIP(hipGetLastError());
        return 0;
    }));
    const ll ldB = ops[1].ld;
    // Z = alpha·F·B (left) or alpha·B·F (right) in one launch, each tile over the k range where F is non-zero
    GemmCall g;
    g.type = type;
    g.tA = g.tB = 0;
    g.M = M; g.N = N; g.K = n;
    g.count = 1;
    g.alpha = alpha; g.beta = 0.0;
    g.A = left ? F : ops[1].dev; g.lda = left ? n : ldB; g.sA = 0;
    g.B = left ? ops[1].dev : F; g.ldb = left ? ldB : n; g.sB = 0;
    g.C = Z; g.ldc = N; g.sC = 0;
    G9_TRY(launch_gemm_klim(g, left ? (lower ? 1 : 2) : (lower ? 3 : 4)));
    G9_HIP(hipMemcpy2DAsync(ops[1].dev, (size_t)ldB * es, Z, (size_t)N * es, (size_t)N * es, (size_t)M,
                            hipMemcpyDeviceToDevice, stream));
    return finish(ops, 2);
}

static int syrk_common(int type, int uplo, int trans, int N, int K, double alpha, const void *A, int lda, const void *B,
                       int ldb, double beta, void *C, int ldc, bool two) {
    G9_TRY(begin());
    G9_TRY(check_type(type));
    if (N <= 0) return 0;
    if (K < 0) K = 0;
    const int es = elem_size(type);
    if (!C || (K > 0 && (!A || (two && !B)))) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "%s: NULL matrix pointer", two ? "syr2k" : "syrk");
    const int need = trans ? N : K;
    if ((K > 0 && (lda < need || (two && ldb < need))) || ldc < N)
        G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "%s: leading dimension too small (lda %d, ldb %d, ldc %d)", two ? "syr2k" : "syrk",
                lda, ldb, ldc);
    Operand ops[3];
    int nops = 0;
    if (K > 0) {
        ops[0].host = A; ops[0].es = es; ops[0].rows = trans ? K : N; ops[0].cols = trans ? N : K; ops[0].caller_ld = lda;
        G9_TRY(resolve(ops[0], SLOT_A, true, false, true));
        nops = 1;
        if (two) {
            ops[1].host = B; ops[1].es = es; ops[1].rows = trans ? K : N; ops[1].cols = trans ? N : K; ops[1].caller_ld = ldb;
            G9_TRY(resolve(ops[1], SLOT_B, true, false, true));
            nops = 2;
        }
    }
    Operand &oc = ops[nops];
    oc.host = C; oc.es = es; oc.rows = N; oc.cols = N; oc.caller_ld = ldc;
    G9_TRY(resolve(oc, SLOT_C, true, true, true));   // the other triangle is kept: C always comes in
    const int lower = uplo == GEN9BLAS_LOWER;
    if (K == 0) {
        G9_TRY(tri_product(type, lower, 0, N, 0, alpha, nullptr, 0, nullptr, 0, beta, oc.dev, oc.ld));
    } else if (!two) {
        G9_TRY(tri_product(type, lower, trans, N, K, alpha, ops[0].dev, ops[0].ld, ops[0].dev, ops[0].ld, beta, oc.dev, oc.ld));
    } else {
        void *X, *Y;
        G9_TRY(scratch(SLOT_X, (size_t)N * 2 * K * es, &X));
        G9_TRY(scratch(SLOT_Y, (size_t)N * 2 * K * es, &Y));
        G9_TRY(by_es(es, [&](auto *tag) -> int {
            using T = std::remove_pointer_t<decltype(tag)>;
            hipLaunchKernelGGL((join_kernel<T>), dim3(grid_for((ll)N * 2 * K)), dim3(256), 0, stream, (const T *)ops[0].dev,
                               ops[0].ld, (const T *)ops[1].dev, ops[1].ld, (T *)X, (T *)Y, N, K, trans);
            G9_HIP(hipGetLastError());
            return 0;
        }));
        G9_TRY(tri_product(type, lower, 0, N, 2 * K, alpha, X, 2ll * K, Y, 2ll * K, beta, oc.dev, oc.ld));
    }
    last_zc = (nops > 0 && ops[0].zc ? 1 : 0) | (nops > 1 && ops[1].zc ? 2 : 0) | (oc.zc ? 4 : 0);
    return finish(ops, nops + 1);
}

int gen9blas_syrk(int type, int uplo, int trans, int N, int K, double alpha, const void *A, int lda, double beta, void *C,
                  int ldc) {
    return syrk_common(type, uplo, trans != 0, N, K, alpha, A, lda, nullptr, 0, beta, C, ldc, false);
}

int gen9blas_syr2k(int type, int uplo, int trans, int N, int K, double alpha, const void *A, int lda, const void *B, int ldb,
                   double beta, void *C, int ldc) {
    return syrk_common(type, uplo, trans != 0, N, K, alpha, A, lda, B, ldb, beta, C, ldc, true);
}

int gen9blas_trsm(int type, int side, int uplo, int transA, int diag, int M, int N, double alpha, const void *A, int lda,
                  void *B, int ldb) {
    G9_TRY(begin());
    G9_TRY(check_type(type));
    if (M <= 0 || N <= 0) return 0;
    const int left = side == GEN9BLAS_LEFT, n = left ? M : N, m = left ? N : M, es = elem_size(type);
    if (!A || !B) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "trsm: NULL matrix pointer");
    if (lda < n || ldb < N) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "trsm: leading dimension too small (lda %d, ldb %d)", lda, ldb);
    Operand ops[2];
    ops[0].host = A; ops[0].es = es; ops[0].rows = n; ops[0].cols = n; ops[0].caller_ld = lda;
    ops[1].host = B; ops[1].es = es; ops[1].rows = M; ops[1].cols = N; ops[1].caller_ld = ldb;
    G9_TRY(resolve(ops[0], SLOT_A, true, false, true));
    G9_TRY(resolve(ops[1], SLOT_B, true, true, true));
    last_zc = (ops[0].zc ? 1 : 0) | (ops[1].zc ? 2 | 4 : 0);
    // L·Y = alpha·R: op'(A) = left ? op(A) : op(A)ᵀ; lower when the triangle of A, transposed or not, is lower
    const int tr = left ? transA != 0 : transA == 0;
    const int lower = (uplo == GEN9BLAS_LOWER) != (tr != 0), rev = !lower;
    // Leaves of TRSM_LEAF_S / _D rows for FP32 / FP64: each leaf inverse is composed from the 128-row FP64 inverses (below);
    // FP16 keeps 128-row leaves (the composition would round once more in FP16)
    const int nbl = (n + TRSM_NB - 1) / TRSM_NB, lb = es == 8 ? TRSM_LEAF_D : es == 4 ? TRSM_LEAF_S : TRSM_NB, nleaf = (n + lb - 1) / lb;
    // A left solve with A lower and not transposed reads both operands where they lie: every product below reads L
    // strictly below its diagonal blocks, the block inversion masks the rest of A itself, B is the right-hand side
    // updated in place (alpha applied by the first product that touches each block of rows), and only the solution
    // is copied back. Every other case first writes L and alpha·R out in the solve's order (reversed for an upper
    // triangle, transposed for the right side).
    const bool direct = left && !tr && !rev;
    void *Ld, *Yd, *Iv, *Zd;
    ll ldl = n, ldy = m;
    if (direct) {
        Ld = ops[0].dev;
        ldl = ops[0].ld;
        Yd = ops[1].dev;
        ldy = ops[1].ld;
    } else {
        G9_TRY(scratch(SLOT_T, (size_t)n * n * es, &Ld));
        G9_TRY(scratch(SLOT_X, (size_t)n * m * es, &Yd));
    }
    // the leaf inverses (leaf p at Iv + p·lb·(lb + 1), row stride lb: element (i, j) of a leaf's rows and columns at
    // Iv[i·lb + j], and a sub-leaf at row s starts at Iv + s·(lb + 1) whatever leaf holds it), then (lb > TRSM_NB)
    // the products C·inv(J1) of the compositions, at most (n / 2h)·h² for a level of h-row halves, h < lb
    const size_t inv_bytes = ((size_t)n * (lb + 1) * es + 255) & ~(size_t)255;
    size_t tm_elems = 0;
    for (ll h = TRSM_NB; h < lb; h *= 2) tm_elems = std::max<size_t>(tm_elems, (size_t)(std::max<ll>(n / (2 * h), 1) * h * h));
    G9_TRY(scratch(SLOT_Y, inv_bytes + tm_elems * es, &Iv));
    G9_TRY(scratch(SLOT_W, (size_t)n * m * es, &Zd));
    G9_TRY(by_es(es, [&](auto *tag) -> int {
        using T = std::remove_pointer_t<decltype(tag)>;
        using S = typename Acc<T>::S;
        if (!direct) {
            hipLaunchKernelGGL((trsm_l_kernel<T>), dim3(grid_for((ll)n * n)), dim3(256), 0, stream, (const T *)ops[0].dev,
                               ops[0].ld, (T *)Ld, n, uplo == GEN9BLAS_LOWER, tr, diag != 0, rev);
            hipLaunchKernelGGL((trsm_y_kernel<T>), dim3(grid_for((ll)n * m)), dim3(256), 0, stream, (const T *)ops[1].dev,
                               ops[1].ld, (T *)Yd, n, m, left, rev, (S)alpha);
        }
        hipLaunchKernelGGL((trsm_inv_kernel<T>), dim3(nbl), dim3(256), 0, stream, (const T *)Ld, ldl, (ll)lb * (ldl + 1),
                           n, (T *)Iv, lb, (ll)lb * (lb + 1), diag != 0);
        G9_HIP(hipGetLastError());
        return 0;
    }));
    // A block [J1 0; C J2]⁻¹ = [inv(J1) 0; −inv(J2)·C·inv(J1) inv(J2)], level by level from halves of h = 128 rows up
    // to halves of lb / 2: the kernel above left the 128-row inverses and the zeros above the diagonal, each level's
    // two GEMMs form the lower-left quadrants, batched over the whole blocks of 2h rows (block at row s: C at
    // L + (s + h)·ldl + s, inv(J1) at Iv + s·(lb + 1), inv(J2) at Iv + (s + h)·(lb + 1), the quadrant at
    // Iv + (s + h)·lb + s), then once for a last block whose second half has b2 < h rows.
    for (ll h = TRSM_NB; h < lb; h *= 2) {
        const char *L0 = (const char *)Ld;
        char *I0 = (char *)Iv, *Tm = I0 + inv_bytes;
        const ll st = 2 * h, ils = ldl + 1, iis = (ll)lb + 1;
        const int full = (int)(n / st);
        G9_TRY(dgemm_dev_batched(type, 0, 0, (int)h, (int)h, (int)h, 1.0, L0 + h * ldl * es, ldl, st * ils, I0, lb,
                                 st * iis, 0.0, Tm, h, h * h, full));
        G9_TRY(dgemm_dev_batched(type, 0, 0, (int)h, (int)h, (int)h, -1.0, I0 + h * iis * es, lb, st * iis, Tm, h, h * h,
                                 0.0, I0 + h * lb * es, lb, st * iis, full));
        const ll s0 = (ll)full * st;
        const int b2 = n - (int)(s0 + h);
        if (b2 > 0) {
            G9_TRY(dgemm_dev(type, 0, 0, b2, (int)h, (int)h, 1.0, L0 + ((s0 + h) * ldl + s0) * es, ldl, I0 + s0 * iis * es,
                             lb, 0.0, Tm, h));
            G9_TRY(dgemm_dev(type, 0, 0, b2, (int)h, b2, -1.0, I0 + (s0 + h) * iis * es, lb, Tm, h, 0.0,
                             I0 + ((s0 + h) * lb + s0) * es, lb));
        }
    }
    TrsmSolve rec{type, n, m, es, lb, (const char *)Ld, (const char *)Iv, (char *)Yd, (char *)Zd, ldl, ldy,
                  direct ? alpha : 1.0};
    G9_TRY(rec.solve(0, nleaf));
    const ll row_bytes = (ll)m * es, ldb_bytes = ops[1].ld * es;
    if (left && !rev && row_bytes % 16 == 0 && ldb_bytes % 16 == 0 && (uintptr_t)ops[1].dev % 16 == 0) {
        const int cpr = (int)(row_bytes / 16);
        hipLaunchKernelGGL(trsm_store_rows16_kernel, dim3(grid_for((ll)n * cpr)), dim3(256), 0, stream,
                           (const uint4 *)Zd, (char *)ops[1].dev, ldb_bytes, n, cpr);
        G9_HIP(hipGetLastError());
        return finish(ops, 2);
    }
    G9_TRY(by_es(es, [&](auto *tag) -> int {
        using T = std::remove_pointer_t<decltype(tag)>;
        hipLaunchKernelGGL((trsm_store_kernel<T>), dim3(grid_for((ll)n * m)), dim3(256), 0, stream, (const T *)Zd,
                           (T *)ops[1].dev, ops[1].ld, n, m, left, rev);
        G9_HIP(hipGetLastError());
        return 0;
    }));
    return finish(ops, 2);
}

}  // extern "C"
