// MFMA GEMM kernels for gfx950: C = alpha·op(A)·op(B) + beta·C in FP16 (FP32 accumulation), FP32 and FP64.
//
// Semantics follow the reference's main kernels and epilogues (reference: lib/kernels/hgemm.cl:838-898 hgemm_v /
// hgemm_kc_v, lib/kernels/sgemm.cl:192-230 sgemm_v + gen9blas_epilog_fb, lib/kernels/dgemm_core.cl:61-94 dgemm_v,
// lib/kernels/hgemm.cl:558-564 gen9blas_epilog_b): every C element is the sum over k of A·B products, then
// alpha·sum + beta·C (C not read when beta = 0), rounded once to the element type. The design is MI355X-native:
// - no packing pass and no separate epilogue kernel: the kernel reads op(A) and op(B) in any of the four transpose
//   layouts straight from memory and applies alpha/beta in registers before its only store of C;
// - block tiles are staged through double-buffered LDS with one barrier per k-step; the next k-step's global loads
//   are in flight while the current one runs on the matrix cores;
// - LDS rows hold 128 bytes of k (64 FP16 / 32 FP32 / 16 FP64) plus 16 bytes of padding, so the fragment reads of
//   16 consecutive rows hit 16 distinct 4-bank groups;
// - an operand stored with its m (or n) index contiguous is transposed in registers, V×V elements per thread
//   (V = 16 bytes / element size), so LDS always holds k-contiguous rows and every fragment read is 16 bytes;
// - accumulation is on MFMA: v_mfma_f32_32x32x16_f16, v_mfma_f32_32x32x2_f32, v_mfma_f64_16x16x4_f64. Operands are
//   swapped (the MFMA "A" input is the B tile) so each lane ends up with 4 consecutive n of one row of C, which gives
//   vector stores of C;
// - the k index inside a block tile is permuted per lane group: lane group g of an MFMA consumes the k-run
//   [g·BK/G, (g+1)·BK/G). A and B use the same permutation, so every product A[m][k]·B[k][n] is summed exactly once;
// - workgroup → tile mapping: consecutive dispatch slots go to different XCDs, so tile indices are re-mapped to give
//   each XCD a contiguous range, and tiles are ordered in groups of GM tile rows so an XCD's L2 shares A and B panels.
#pragma once
#include "internal.h"

namespace g9 {

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// ---------------- MFMA traits ----------------
// D is MI × MI; G = 64 / MI lane groups; E elements of one operand per lane per instruction. Accumulator r of lane l
// holds D[row(r, l)][l % MI]. In the 32×32 layouts rows come in runs of 4 consecutive values (r = 4q .. 4q+3); in
// the FP64 16×16 layout accumulator r of lane group g holds row 4r + g.
// SWAP: the B tile is the MFMA's first operand, so D rows are n (consecutive n per lane → vector stores of C).
// BLOCKED: each block tile (BK values of k) is summed into a fresh accumulator that is then added to the running
// one, so the FP32 rounding error grows with K/BK + BK instead of K.
template <class T> struct Mma;
template <> struct Mma<f16> {
    static constexpr int MI = 32, G = 2, E = 8, NACC = 16;
    static constexpr bool SWAP = true, BLOCKED = false;
    using Acc = f32x16;
    using Sum = float;
    static __device__ __forceinline__ Acc mma(u32x4 a, u32x4 b, Acc c, int) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
    static __device__ __forceinline__ int row(int r, int l) { return 8 * (r >> 2) + 4 * (l >> 5) + (r & 3); }
};
template <> struct Mma<float> {
    static constexpr int MI = 32, G = 2, E = 1, NACC = 16;
    static constexpr bool SWAP = true, BLOCKED = true;
    using Acc = f32x16;
    using Sum = float;
    // ss selects the element of the 16-byte group (4 FP32 values = 4 consecutive k-steps). Elements are copied to
    // scalars before __builtin_bit_cast (hipcc evaluates a bit_cast of a vector element as element 0).
    static __device__ __forceinline__ Acc mma(u32x4 a, u32x4 b, Acc c, int ss) {
        const unsigned as = a[ss], bs = b[ss];
        return __builtin_amdgcn_mfma_f32_32x32x2f32(__builtin_bit_cast(float, as), __builtin_bit_cast(float, bs), c, 0, 0, 0);
    }
    static __device__ __forceinline__ int row(int r, int l) { return 8 * (r >> 2) + 4 * (l >> 5) + (r & 3); }
};
template <> struct Mma<double> {
    static constexpr int MI = 16, G = 4, E = 1, NACC = 4;
    static constexpr bool SWAP = false, BLOCKED = false;
    using Acc = f64x4;
    using Sum = double;
    static __device__ __forceinline__ Acc mma(u32x4 a, u32x4 b, Acc c, int ss) {
        const unsigned a0 = a[2 * ss], a1 = a[2 * ss + 1], b0 = b[2 * ss], b1 = b[2 * ss + 1];
        const u32x2 pa = {a0, a1}, pb = {b0, b1};
        return __builtin_amdgcn_mfma_f64_16x16x4f64(__builtin_bit_cast(double, pa), __builtin_bit_cast(double, pb), c, 0, 0, 0);
    }
    static __device__ __forceinline__ int row(int r, int l) { return 4 * r + (l >> 4); }
};

template <class S> struct GemmParams {
    const void *A, *B;
    void *C;
    long long lda, ldb, ldc, sA, sB, sC;
    int M, N, K, tiles_m, tiles_n, vec_c;
    S alpha, beta;
    // split K (count = 1 only): slice z = blockIdx.y covers k = z·kper .. +kper and writes its unscaled partial sums
    // to P + z·M·N (row stride N, accumulator type S); a reduction kernel then forms alpha·Σ + beta·C
    S *P;
    int kper, vec_p;
    int kpair = 0;   // KLIM: the second half of the dispatch order reversed (see the tile mapping)
};

// 16 bytes (V elements) of row r, columns c .. c+V-1 of a row-major matrix X (R valid rows, Cc valid columns, row
// stride ld); zero outside the valid region. VEC: X and ld are 16-byte aligned, so whole chunks load as one vector.
template <class T, bool VEC>
__device__ __forceinline__ u32x4 load16(const T *__restrict__ X, long long ld, int r, int c, int R, int Cc) {
    constexpr int V = 16 / sizeof(T);
    if (VEC && r < R && c + V <= Cc) return *reinterpret_cast<const u32x4 *>(X + (long long)r * ld + c);
    union { u32x4 v; T e[V]; } u;
#pragma unroll
    for (int e = 0; e < V; e++) u.e[e] = (r < R && c + e < Cc) ? X[(long long)r * ld + c + e] : T(0);
    return u.v;
}

// Transpose of a V×V block held as V rows of 16 bytes: out[j] element i = in[i] element j.
template <class T> __device__ __forceinline__ void transpose(const u32x4 *in, u32x4 *out);
template <> __device__ __forceinline__ void transpose<f16>(const u32x4 *in, u32x4 *out) {
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const unsigned lo = in[2 * w][j >> 1], hi = in[2 * w + 1][j >> 1];
            out[j][w] = (j & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
        }
}
template <> __device__ __forceinline__ void transpose<float>(const u32x4 *in, u32x4 *out) {
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) out[j][i] = in[i][j];
}
template <> __device__ __forceinline__ void transpose<double>(const u32x4 *in, u32x4 *out) {
    out[0] = u32x4{in[0][0], in[0][1], in[1][0], in[1][1]};
    out[1] = u32x4{in[0][2], in[0][3], in[1][2], in[1][3]};
}

// Global → register → LDS staging of one operand tile: RT rows (m or n) × BK (k), 128 bytes of k per row.
// KC: the operand is stored k-contiguous (element (mn, k) at X[mn·ld + k]); otherwise mn-contiguous
// (element (mn, k) at X[k·ld + mn]) and transposed in registers on the way to LDS.
constexpr int ROWB = 144;   // LDS bytes per tile row: 128 of data + 16 of padding
template <class T, int RT, int NT, bool KC, bool VEC>
struct Stage {
    static constexpr int V = 16 / (int)sizeof(T);
    // k-contiguous: N16 chunks per thread. Transposed: NB V×V blocks per thread; when the tile has fewer blocks than
    // the workgroup has threads, threads tid < RT·8/V take one block each (ACT) and the others idle.
    static constexpr int NBLK = RT * 8 / V;
    static constexpr int NB = KC ? 0 : (NBLK >= NT ? NBLK / NT : 1);
    static constexpr bool PART = !KC && NBLK < NT;
    static constexpr int N16 = KC ? RT * 8 / NT : NB * V;
    static_assert(!KC || RT * 8 % NT == 0, "tile rows × 8 chunks must divide over the threads");
    static_assert(KC || NBLK % NT == 0 || NT % NBLK == 0, "transposed blocks must divide over the threads");
    u32x4 r[N16];

    // CHECK = false: the whole tile lies inside the matrix (interior tile, full k-step) and X is 16-byte aligned,
    // so every chunk is one unconditional vector load.
    template <bool CHECK>
    __device__ __forceinline__ void load(const T *__restrict__ X, long long ld, int MN, int K, int mn0, int k0, int tid) {
        if constexpr (KC) {
#pragma unroll
            for (int i = 0; i < N16; i++) {
                const int id = i * NT + tid, row = mn0 + (id >> 3), col = k0 + (id & 7) * V;
                if constexpr (CHECK) r[i] = load16<T, VEC>(X, ld, row, col, MN, K);
                else r[i] = *reinterpret_cast<const u32x4 *>(X + (long long)row * ld + col);
            }
        } else {
            if (PART && tid >= NBLK) return;
#pragma unroll
            for (int b = 0; b < NB; b++) {
                const int id = b * NT + tid, lo = id & 31;
                const int mb = (lo & 3) + 4 * (id >> 5), kb = lo >> 2;
#pragma unroll
                for (int i = 0; i < V; i++) {
                    const int row = k0 + kb * V + i, col = mn0 + mb * V;
                    if constexpr (CHECK) r[b * V + i] = load16<T, VEC>(X, ld, row, col, K, MN);
                    else r[b * V + i] = *reinterpret_cast<const u32x4 *>(X + (long long)row * ld + col);
                }
            }
        }
    }
    __device__ __forceinline__ void store(unsigned char *rows, int tid) const {
        if constexpr (KC) {
#pragma unroll
            for (int i = 0; i < N16; i++) {
                const int id = i * NT + tid;
                *reinterpret_cast<u32x4 *>(rows + (id >> 3) * ROWB + (id & 7) * 16) = r[i];
            }
        } else {
            if (PART && tid >= NBLK) return;
#pragma unroll
            for (int b = 0; b < NB; b++) {
                const int id = b * NT + tid, lo = id & 31;
                const int mb = (lo & 3) + 4 * (id >> 5), kb = lo >> 2;
                u32x4 t[V];
                transpose<T>(r + b * V, t);
#pragma unroll
                for (int j = 0; j < V; j++) *reinterpret_cast<u32x4 *>(rows + (mb * V + j) * ROWB + kb * 16) = t[j];
            }
        }
    }
};

__device__ __forceinline__ float fma_s(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double fma_s(double a, double b, double c) { return __builtin_fma(a, b, c); }
template <class T, class S> __device__ __forceinline__ void store4(T *c, const S *v, S alpha, S beta, bool vec, int valid);

// Instruction-group masks of __builtin_amdgcn_sched_group_barrier.
constexpr int SG_MFMA = 0x008, SG_VMEM_READ = 0x020, SG_DS_READ = 0x100, SG_DS_WRITE = 0x200;

// TRI (1: lower, 2: upper): C is square and only its lower (upper) triangle is written, alpha·sum + beta·C as
// elsewhere; the grid holds only the tiles that meet the triangle (square tiles, one product, no split).
// KLIM: the k range of a tile is cut to where a triangular operand is non-zero (one product, no split):
//   1: op(A) lower, k < m0 + BM; 2: op(A) upper, k ≥ m0; 3: op(B) lower, k ≥ n0; 4: op(B) upper, k < n0 + BN.
//   Tiles are dispatched longest range first, spread over the XCDs.
template <class T, int BM, int BN, int WM, int WN, bool AK, bool BKC, bool VEC, bool SCHED = true, bool SPLIT = false,
          int TRI = 0, int KLIM = 0, int KG = 1>
__global__ void __launch_bounds__(WM *WN * 64 * KG) gemm_kernel(GemmParams<typename Mma<T>::Sum> p) {
    using MM = Mma<T>;
    using S = typename MM::Sum;
    constexpr int NT = WM * WN * 64;
    constexpr int BK = 128 / (int)sizeof(T);
    constexpr int MI = MM::MI, G = MM::G;
    constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / MI, TN = WTN / MI;
    constexpr int KRB = BK / G * (int)sizeof(T);   // bytes of k per lane group and row
    constexpr int QG = KRB / 16;                    // 16-byte groups per lane group and row
    constexpr int SPG = 16 / ((int)sizeof(T) * MM::E);   // MFMA steps per 16-byte group
    static_assert(TM * MI == WTM && TN * MI == WTN, "wave tile must be a multiple of the MFMA tile");
    static_assert(TRI == 0 || (BM == BN && !SPLIT), "triangle mode: square tiles, no split");
    static_assert(KLIM == 0 || (!SPLIT && TRI == 0), "k-limited tiles: one product, no split");
    static_assert(KG == 1 || (!SPLIT && TRI == 0 && KLIM == 0), "k groups: plain tiles only");
    __shared__ __attribute__((aligned(16))) unsigned char lds[2 * KG][(BM + BN) * ROWB];

    // KG > 1: the workgroup holds KG groups of WM × WN waves; group kh takes the block tiles kh, kh + KG, ... of the
    // k range into LDS buffers of its own, and the groups' sums are added in group order at the end
    const int kh = KG > 1 ? (int)threadIdx.x / NT : 0;
    const int tid = KG > 1 ? (int)threadIdx.x % NT : (int)threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid % WM, wn = wid / WM;
    const int g = lane / MI, lr = lane % MI;

    // tile of this workgroup
    int bid = blockIdx.x;
    const int nt = TRI ? p.tiles_m * (p.tiles_m + 1) / 2 : p.tiles_m * p.tiles_n, nt8 = nt & ~7;
    if (bid < nt8) bid = (bid & 7) * (nt8 >> 3) + (bid >> 3);
    int m0, n0;
    if constexpr (TRI != 0) {
        // tile bid of the lower triangle of tiles, row by row: (tr, tc) with tc ≤ tr; the upper triangle transposes it
        int tr = (int)((__builtin_sqrtf(8.f * (float)bid + 1.f) - 1.f) * 0.5f);
        while ((tr + 1) * (tr + 2) / 2 <= bid) tr++;
        while (tr * (tr + 1) / 2 > bid) tr--;
        const int tc = bid - tr * (tr + 1) / 2;
        m0 = (TRI == 1 ? tr : tc) * BM;
        n0 = (TRI == 1 ? tc : tr) * BN;
    } else if constexpr (KLIM != 0) {
        // Tiles in dispatch order, longest k range first, without the XCD remap: consecutive workgroups go to
        // different XCDs, so every XCD gets long and short tiles alike (a contiguous range per XCD would give one XCD
        // all the longest tiles). kpair (all tiles resident at once, two per CU): workgroups i and i + T/2 share a
        // CU, and the second half takes the ranks in reverse, so that each CU pairs a long range with a short one
        int b = blockIdx.x;
        if (p.kpair) {
            const int nt = p.tiles_m * p.tiles_n, h = nt / 2;
            if (b >= h) b = nt - 1 - (b - h);
        }
        if constexpr (KLIM <= 2) {   // the range depends on the tile row
            const int tr = b / p.tiles_n;
            m0 = (KLIM == 1 ? p.tiles_m - 1 - tr : tr) * BM;
            n0 = (b % p.tiles_n) * BN;
        } else {                     // on the tile column
            const int tc = b / p.tiles_m;
            n0 = (KLIM == 4 ? p.tiles_n - 1 - tc : tc) * BN;
            m0 = (b % p.tiles_m) * BM;
        }
    } else {
        constexpr int GM = 4;
        const int group = bid / (GM * p.tiles_n), first_m = group * GM;
        const int gsz = min(p.tiles_m - first_m, GM);
        const int in_group = bid % (GM * p.tiles_n);
        m0 = (first_m + in_group % gsz) * BM;
        n0 = (in_group / gsz) * BN;
    }
    // elements of a tile on the diagonal are written only inside the triangle
    const bool diag = TRI != 0 && m0 == n0;
    const auto in_tri = [&](int m, int n) { return TRI == 1 ? n <= m : n >= m; };

    const long long z = blockIdx.y;
    const T *A = reinterpret_cast<const T *>(p.A);
    const T *B = reinterpret_cast<const T *>(p.B);
    T *C = reinterpret_cast<T *>(p.C);
    int K = p.K;
    if constexpr (SPLIT || KLIM != 0) {
        int k0, k1;
        if constexpr (SPLIT) {
            k0 = (int)z * p.kper;
            k1 = min(p.K, k0 + p.kper);
        } else {
            k0 = KLIM == 2 ? m0 : KLIM == 3 ? n0 : 0;
            k1 = KLIM == 1 ? min(p.K, m0 + BM) : KLIM == 4 ? min(p.K, n0 + BN) : p.K;
        }
        K = max(k1 - k0, 0);
        A += AK ? k0 : (long long)k0 * p.lda;
        B += BKC ? k0 : (long long)k0 * p.ldb;
        if constexpr (!SPLIT) {   // k-limited tiles of a batch: product z
            A += z * p.sA;
            B += z * p.sB;
            C += z * p.sC;
        }
    } else {
        A += z * p.sA;
        B += z * p.sB;
        C += z * p.sC;
    }

    Stage<T, BM, NT, AK, VEC> sa;
    Stage<T, BN, NT, BKC, VEC> sb;
    constexpr int TI = MM::SWAP ? TN : TM, TJ = MM::SWAP ? TM : TN;   // acc[i][j]: D tile of (first, second) operand
    typename MM::Acc acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < TJ; j++)
#pragma unroll
            for (int r = 0; r < MM::NACC; r++) acc[i][j][r] = 0;

    // MFMAs of one block tile held in LDS buffer `cur`. Fragments live in two register sets: group q+1 is read from
    // LDS while the MFMAs of group q run.
    auto compute = [&](int cur) {
        const unsigned char *As = lds[cur * KG + kh] + (wm * WTM + lr) * ROWB + g * KRB;
        const unsigned char *Bs = lds[cur * KG + kh] + BM * ROWB + (wn * WTN + lr) * ROWB + g * KRB;
        typename MM::Acc part[MM::BLOCKED ? TI : 1][MM::BLOCKED ? TJ : 1];
        if constexpr (MM::BLOCKED) {
#pragma unroll
            for (int i = 0; i < TI; i++)
#pragma unroll
                for (int j = 0; j < TJ; j++)
#pragma unroll
                    for (int r = 0; r < MM::NACC; r++) part[i][j][r] = 0;
        }
        u32x4 ra[2][TM], rb[2][TN];
        auto read_frags = [&](int q, int set) {
#pragma unroll
            for (int i = 0; i < TM; i++) ra[set][i] = *reinterpret_cast<const u32x4 *>(As + i * MI * ROWB + q * 16);
#pragma unroll
            for (int i = 0; i < TN; i++) rb[set][i] = *reinterpret_cast<const u32x4 *>(Bs + i * MI * ROWB + q * 16);
        };
        read_frags(0, 0);
#pragma unroll
        for (int q = 0; q < QG; q++) {
            if (q + 1 < QG) read_frags(q + 1, (q + 1) & 1);
#pragma unroll
            for (int ss = 0; ss < SPG; ss++)
#pragma unroll
                for (int i = 0; i < TI; i++)
#pragma unroll
                    for (int j = 0; j < TJ; j++) {
                        const u32x4 x = MM::SWAP ? rb[q & 1][i] : ra[q & 1][i], y = MM::SWAP ? ra[q & 1][j] : rb[q & 1][j];
                        if constexpr (MM::BLOCKED) part[i][j] = MM::mma(x, y, part[i][j], ss);
                        else acc[i][j] = MM::mma(x, y, acc[i][j], ss);
                    }
        }
        if constexpr (MM::BLOCKED) {
#pragma unroll
            for (int i = 0; i < TI; i++)
#pragma unroll
                for (int j = 0; j < TJ; j++) acc[i][j] += part[i][j];
        }
    };

    // block tiles per k group (a group's tiles past K load as zeros)
    const int nk = ((K + BK - 1) / BK + KG - 1) / KG;
    const int kofs = kh * BK;
    auto buf = [&](int b) { return lds[b * KG + kh]; };
    // Interior tiles with whole k-steps load without bounds tests: the steady-state loop is then one basic block,
    // whose instruction order is pinned below so the LDS reads, global loads and LDS writes of a k-step run between
    // its MFMAs.
    const bool fast = VEC && m0 + BM <= p.M && n0 + BN <= p.N && K % (BK * KG) == 0;
    if (fast) {
        sa.template load<false>(A, p.lda, p.M, K, m0, kofs, tid);
        sb.template load<false>(B, p.ldb, p.N, K, n0, kofs, tid);
        sa.store(buf(0), tid);
        sb.store(buf(0) + BM * ROWB, tid);
        __syncthreads();
        for (int kt = 0; kt + 1 < nk; kt++) {
            const int cur = kt & 1;
            sa.template load<false>(A, p.lda, p.M, K, m0, (kt + 1) * KG * BK + kofs, tid);
            sb.template load<false>(B, p.ldb, p.N, K, n0, (kt + 1) * KG * BK + kofs, tid);
            compute(cur);
            sa.store(buf(cur ^ 1), tid);
            sb.store(buf(cur ^ 1) + BM * ROWB, tid);
            if constexpr (SCHED) {
                constexpr int NRD = TM + TN;                         // LDS fragment reads per group
                constexpr int NMF = SPG * TI * TJ;                   // MFMAs per group
                constexpr int NVM = Stage<T, BM, NT, AK, VEC>::N16 + Stage<T, BN, NT, BKC, VEC>::N16;
                constexpr int NWR = (AK ? Stage<T, BM, NT, AK, VEC>::N16 : Stage<T, BM, NT, AK, VEC>::NB * 8) +
                                    (BKC ? Stage<T, BN, NT, BKC, VEC>::N16 : Stage<T, BN, NT, BKC, VEC>::NB * 8);
                // global loads first, then group 0's fragments; each later group: its MFMAs interleaved with the next
                // group's reads, and over the last two groups the LDS writes of the next tile
                __builtin_amdgcn_sched_group_barrier(SG_VMEM_READ, NVM, 0);
                __builtin_amdgcn_sched_group_barrier(SG_DS_READ, NRD, 0);
#pragma unroll
                for (int q = 0; q < QG; q++) {
                    const int nrd = q + 1 < QG ? NRD : 0;
                    const int nwr = q >= QG - 2 ? (q == QG - 1 ? NWR - NWR / 2 : NWR / 2) : 0;
#pragma unroll
                    for (int t = 0; t < NMF; t++) {
                        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
                        if (t < nrd) __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
                        else if (t - nrd < nwr) __builtin_amdgcn_sched_group_barrier(SG_DS_WRITE, 1, 0);
                    }
                }
            }
            __syncthreads();
        }
        compute((nk - 1) & 1);
    } else {
        auto load_tile = [&](int k0) {
            sa.template load<true>(A, p.lda, p.M, K, m0, k0, tid);
            sb.template load<true>(B, p.ldb, p.N, K, n0, k0, tid);
        };
        load_tile(kofs);
        sa.store(buf(0), tid);
        sb.store(buf(0) + BM * ROWB, tid);
        __syncthreads();
        for (int kt = 0; kt < nk; kt++) {
            const int cur = kt & 1;
            if (kt + 1 < nk) load_tile((kt + 1) * KG * BK + kofs);
            compute(cur);
            if (kt + 1 < nk) {
                sa.store(buf(cur ^ 1), tid);
                sb.store(buf(cur ^ 1) + BM * ROWB, tid);
            }
            __syncthreads();
        }
    }

    if constexpr (KG > 1) {
        // groups 1 .. KG-1 leave their sums in LDS (value-major, so a wave's 64 lanes write 256 consecutive bytes);
        // group 0 adds them in group order and stores C
        constexpr int NV = TI * TJ * MM::NACC;
        static_assert((KG - 1) * NV * NT * sizeof(S) <= sizeof(lds), "k-group sums must fit in LDS");
        S *red = reinterpret_cast<S *>(&lds[0][0]);
        __syncthreads();   // the last block tile of every group has been read
        if (kh > 0) {
#pragma unroll
            for (int i = 0; i < TI; i++)
#pragma unroll
                for (int j = 0; j < TJ; j++)
#pragma unroll
                    for (int r = 0; r < MM::NACC; r++)
                        red[((kh - 1) * NV + (i * TJ + j) * MM::NACC + r) * NT + tid] = acc[i][j][r];
        }
        __syncthreads();
        if (kh > 0) return;
#pragma unroll
        for (int h = 1; h < KG; h++)
#pragma unroll
            for (int i = 0; i < TI; i++)
#pragma unroll
                for (int j = 0; j < TJ; j++)
#pragma unroll
                    for (int r = 0; r < MM::NACC; r++)
                        acc[i][j][r] += red[((h - 1) * NV + (i * TJ + j) * MM::NACC + r) * NT + tid];
    }

    if constexpr (MM::SWAP) {
        // lane holds D[n][m] with m = column, runs of 4 consecutive n: vector stores along a row of C
#pragma unroll
        for (int i = 0; i < TI; i++)
#pragma unroll
            for (int j = 0; j < TJ; j++) {
                const int m = m0 + wm * WTM + j * MI + lr;
                if (m >= p.M) continue;
#pragma unroll
                for (int q = 0; q < MM::NACC / 4; q++) {
                    const int n = n0 + wn * WTN + i * MI + MM::row(4 * q, lane);
                    if (n >= p.N) continue;
                    const S v[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                    if (diag) {
                        T *c = C + (long long)m * p.ldc + n;
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            if (n + e < p.N && in_tri(m, n + e)) {
                                S r = p.alpha * v[e];
                                if (p.beta != S(0)) r = fma_s(p.beta, (S)c[e], r);
                                c[e] = (T)r;
                            }
                        continue;
                    }
                    if constexpr (SPLIT)
                        store4<S, S>(p.P + z * p.M * (long long)p.N + (long long)m * p.N + n, v, S(1), S(0), p.vec_p, p.N - n);
                    else
                        store4<T, S>(C + (long long)m * p.ldc + n, v, p.alpha, p.beta, p.vec_c, p.N - n);
                }
            }
    } else {
        // lane holds D[m][n] with n = column: the lanes of a group store consecutive n of one row
#pragma unroll
        for (int i = 0; i < TI; i++)
#pragma unroll
            for (int j = 0; j < TJ; j++) {
                const int n = n0 + wn * WTN + j * MI + lr;
                if (n >= p.N) continue;
#pragma unroll
                for (int r = 0; r < MM::NACC; r++) {
                    const int m = m0 + wm * WTM + i * MI + MM::row(r, lane);
                    if (m >= p.M || (diag && !in_tri(m, n))) continue;
                    if constexpr (SPLIT) {
                        p.P[z * p.M * (long long)p.N + (long long)m * p.N + n] = acc[i][j][r];
                        continue;
                    }
                    T *c = C + (long long)m * p.ldc + n;
                    S v = p.alpha * acc[i][j][r];
                    if (p.beta != S(0)) v = fma_s(p.beta, (S)*c, v);
                    *c = (T)v;
                }
            }
    }
}

// C[0..3] = alpha·v + beta·C (C not read when beta = 0), rounded once to T; `valid` elements are inside C.
template <class T, class S>
__device__ __forceinline__ void store4(T *c, const S *v, S alpha, S beta, bool vec, int valid) {
    if (vec && valid >= 4) {
        if constexpr (sizeof(T) == 2) {
            u32x2 old = beta != S(0) ? *reinterpret_cast<const u32x2 *>(c) : u32x2{0, 0};
            union { u32x2 w; T e[4]; } o, n;
            o.w = old;
#pragma unroll
            for (int e = 0; e < 4; e++) n.e[e] = (T)(beta != S(0) ? __builtin_fmaf(beta, (S)o.e[e], alpha * v[e]) : alpha * v[e]);
            *reinterpret_cast<u32x2 *>(c) = n.w;
        } else if constexpr (sizeof(T) == 4) {
            f32x4 o = beta != S(0) ? *reinterpret_cast<const f32x4 *>(c) : f32x4{0, 0, 0, 0};
            f32x4 n;
#pragma unroll
            for (int e = 0; e < 4; e++) n[e] = beta != S(0) ? __builtin_fmaf(beta, o[e], alpha * v[e]) : alpha * v[e];
            *reinterpret_cast<f32x4 *>(c) = n;
        } else {
            f64x4 o = beta != S(0) ? *reinterpret_cast<const f64x4 *>(c) : f64x4{0, 0, 0, 0};
            f64x4 n;
#pragma unroll
            for (int e = 0; e < 4; e++) n[e] = beta != S(0) ? __builtin_fma(beta, o[e], alpha * v[e]) : alpha * v[e];
            *reinterpret_cast<f64x4 *>(c) = n;
        }
        return;
    }
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (e < valid) {
            S r = alpha * v[e];
            if (beta != S(0)) r = fma_s(beta, (S)c[e], r);
            c[e] = (T)r;
        }
}

// Split-K finish: C = alpha·(P[0] + ... + P[splits-1]) + beta·C (C not read when beta = 0), summed in slice order
// and rounded once to T. One thread per 4 consecutive elements of a row (N % 4 == 0 and aligned C), else per element.
template <class T, class S, bool VEC4>
__global__ void __launch_bounds__(256) splitk_reduce(const S *__restrict__ P, T *C, long long ldc, int M, int N, int splits,
                                                     S alpha, S beta) {
    const long long mn = (long long)M * N;
    const long long stride = (long long)gridDim.x * blockDim.x;
    if constexpr (VEC4) {
        for (long long g = blockIdx.x * (long long)blockDim.x + threadIdx.x; g < mn / 4; g += stride) {
            const long long e = 4 * g;
            const int m = (int)(e / N), n = (int)(e % N);
            S v[4] = {0, 0, 0, 0};
            for (int sp = 0; sp < splits; sp++)
#pragma unroll
                for (int t = 0; t < 4; t++) v[t] += P[sp * mn + e + t];
            store4<T, S>(C + (long long)m * ldc + n, v, alpha, beta, true, 4);
        }
    } else {
        for (long long e = blockIdx.x * (long long)blockDim.x + threadIdx.x; e < mn; e += stride) {
            const int m = (int)(e / N), n = (int)(e % N);
            S v = 0;
            for (int sp = 0; sp < splits; sp++) v += P[sp * mn + e];
            S r = alpha * v;
            T *c = C + (long long)m * ldc + n;
            if (beta != S(0)) r = fma_s(beta, (S)*c, r);
            *c = (T)r;
        }
    }
}

}  // namespace g9
