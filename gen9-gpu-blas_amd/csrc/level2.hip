// Level-2 routines on symmetric, triangular, banded and packed matrices: SYMV, TRMV, TRSV, SYR, SYR2 (full storage)
// and GBMV, SBMV, TBMV, TBSV, SPMV, TPMV, TPSV, SPR, SPR2 (reference: lib/src/level12.c:267-519, arithmetic of
// lib/kernels/level12.cl:424-640).
//
// One storage model covers every layout: element (i, j) sits at a[rs(i) + j] for j in the stored range
// [lo(i), hi(i)] of row i.
//   full storage, row stride ld:   rs(i) = i·ld                  range [0, ncols), cut to j ≤ i (lower) or j ≥ i (upper)
//   band, KL below / KU above:     rs(i) = i·(ld − 1) + KL       range [i − KL, i + KU] ∩ [0, ncols)
//   packed upper, order n:         rs(i) = i·n − i(i − 1)/2 − i  range [i, n)
//   packed lower:                  rs(i) = i(i + 1)/2            range [0, i]
// A unit diagonal takes j = i out of the range (the stored diagonal is not read).
//
// Products y = alpha·op(A)·x + beta·y make one pass over the stored elements. A wave owns a group of 64·V columns
// (V elements of 16 bytes per lane for aligned full storage, one element per lane otherwise) and a band of rows.
// Each element read adds a·x_j to its row sum (op(A) = A) and/or a·x_i to its column sum (op(A) = Aᵀ, and the
// mirrored half of a symmetric matrix), so a symmetric matrix is read once, from its stored triangle. Row sums are
// reduced across the wave (transposing butterfly) into one FP32 (FP64) partial per row and column group, column sums
// stay in registers into one partial per column and row band; a second kernel adds the partials of each output in a
// fixed order and applies alpha / beta once, so results do not depend on scheduling. FP16 is computed in FP32 as in
// the reference (level12.cl:1-3).
//
// Triangular solves run over diagonal blocks of 128 rows, one launch per block: one workgroup applies the previous
// block's update to this block's rows, loads the block of op(A) into LDS and one wave substitutes (lanes own rows,
// the solved value of each step is broadcast from its lane), while the other workgroups apply the previous block's
// update to the rows beyond (the reference alternates a solve and an update launch: level12.c:303-347). The work
// vector is FP32 (FP64 for FP64), also for FP16 (level12.c:301).
#include "internal.h"
#include "wave.h"
#include <algorithm>
#include <type_traits>

namespace g9 {
namespace l2 {

typedef long long ll;
typedef _Float16 f16;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
template <class T> struct Comp { using R = float; };
template <> struct Comp<double> { using R = double; };
template <class T> constexpr int VW = 16 / (int)sizeof(T);
template <class T> union Vec {
    u32x4 u;
    T e[VW<T>];
};
__device__ __forceinline__ float fma_r(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double fma_r(double a, double b, double c) { return __builtin_fma(a, b, c); }

enum { F_FULL = 0, F_BAND, F_PACKU, F_PACKL };
enum { TRI_NONE = 0, TRI_LOWER = 1, TRI_UPPER = 2 };
enum { DIR_ROW = 1, DIR_COL = 2 };

struct Shape {
    ll ld;              // row stride (full, band)
    int KL, KU;         // band widths below / above the diagonal
    int n;              // order of a packed matrix
    int nrows, ncols;
    int tri;            // TRI_*: the stored triangle
    int unit;           // unit diagonal: j = i not stored
};

template <int FMT> __device__ __forceinline__ ll row_start(const Shape &s, int i) {
    if constexpr (FMT == F_FULL) return (ll)i * s.ld;
    else if constexpr (FMT == F_BAND) return (ll)i * (s.ld - 1) + s.KL;
    else if constexpr (FMT == F_PACKU) return (ll)i * s.n - (ll)i * (i - 1) / 2 - i;
    else return (ll)i * (i + 1) / 2;
}
__device__ __forceinline__ void stored_range(const Shape &s, bool band, int i, int &lo, int &hi) {
    lo = 0;
    hi = s.ncols - 1;
    if (band) {
        lo = max(lo, i - s.KL);
        hi = min(hi, i + s.KU);
    }
    if (s.tri == TRI_LOWER) hi = min(hi, i - s.unit);
    else if (s.tri == TRI_UPPER) lo = max(lo, i + s.unit);
}

// ---------------- products ----------------
constexpr int NT = 256;
// Rows per batch: 8 with 16 bytes per lane (V > 1: a wave has 8 KiB of loads outstanding), 16 with one element per
// lane. From a sweep at n = 16384 FP32 (SYMV / TRMV / SPMV): 8 and 16 rows, 8 to 128 workgroups per CU.
template <int V> constexpr int UB = V > 1 ? 8 : 16;
// 16 bytes of a row from p: full storage keeps 16-byte aligned rows (nontemporal: the matrix is read once); band and
// packed rows are only element-aligned, a 16-byte load that the GPU serves at any 4-byte alignment (the compiler
// emits the same global_load_dwordx4 for a 4-byte-aligned 16-byte copy).
template <int FMT> __device__ __forceinline__ u32x4 row16(const void *p) {
    if constexpr (FMT == F_FULL) return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    u32x4 t;
    __builtin_memcpy(&t, p, 16);
    return t;
}
template <class T, int V, int FMT>
__global__ void __launch_bounds__(NT) mv_kernel(Shape s, const T *__restrict__ a, const T *__restrict__ x, ll ix, int rpp, int dirs,
                                                int skipdiag, typename Comp<T>::R *P, typename Comp<T>::R *Q) {
    using R = typename Comp<T>::R;
    constexpr bool band = FMT == F_BAND;
    constexpr int U = UB<V>;
    const int lane = threadIdx.x & 63;
    // A workgroup owns column group blockIdx.x and row band blockIdx.y; its waves take consecutive quarters of the
    // band (the wave index is uniform across a wave: loop bounds derived from it stay in scalar registers).
    const int g = blockIdx.x, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g0 = g * 64 * V, g1 = min(g0 + 64 * V, s.ncols) - 1, c0 = g0 + lane * V;
    const int rpw = rpp / (NT / 64);
    // rows whose stored range can reach the group's columns, within this wave's quarter of the band
    // an upper triangle's long row bands come first in the matrix: they are dispatched last, as a lower triangle's
    const int bandi = s.tri == TRI_UPPER ? (int)gridDim.y - 1 - (int)blockIdx.y : (int)blockIdx.y;
    int rb = bandi * rpp + w * rpw, re = min(s.nrows, rb + rpw);
    if (s.tri == TRI_LOWER) rb = max(rb, g0);
    if (s.tri == TRI_UPPER) re = min(re, g1 + 1);
    if (band) {
        rb = max(rb, g0 - s.KU);
        re = min(re, g1 + s.KL + 1);
    }
    R xc[V], sc[V];
#pragma unroll
    for (int e = 0; e < V; e++) {
        xc[e] = (dirs & DIR_ROW) && c0 + e < s.ncols ? (R)x[(ll)(c0 + e) * ix] : R(0);
        sc[e] = 0;
    }
    // Rows [fa, fb) store every column of the group and not its diagonal (the stored range is monotonic in the row
    // for every layout): they are read whole and used without masks. The other rows, near the diagonal or the band's
    // edges, take the checked path.
    int fa = rb, fb = re;
    if (g0 + 64 * V > s.ncols) {
        fb = fa;
    } else {
        if (band) {
            fa = max(fa, g1 - s.KU);
            fb = min(fb, g0 + s.KL + 1);
        }
        if (s.tri == TRI_LOWER) fa = max(fa, g1 + 1);
        if (s.tri == TRI_UPPER) fb = min(fb, g0);
    }
    fa = min(fa, re);                 // inside this band: rb <= fa <= fb <= re
    fb = max(fa, min(fb, re));
    fb = fa + (fb - fa) / U * U;      // whole batches
    auto reduce_rows = [&](int i, int rend, R (&rs)[U]) {
        int base = 0;
        butterfly<0, U>(rs, lane, base);
        if ((lane & (64 / U - 1)) == 0 && i + base < rend) Q[(ll)g * s.nrows + i + base] = rs[0];
    };
    // checked rows [r0, r1): an element is read only where stored, a 16-byte chunk whole when it meets the stored
    // range inside the matrix's columns (its elements outside the range are masked when used). Full storage holds
    // every column of every row, so there, when the whole column group lies inside the matrix (a wave-uniform test),
    // every row's chunk is read whole, from rows clamped into [r0, r1), and all of a batch's loads are in flight
    // together: a per-lane choice between a chunk and single elements written into the same registers had the
    // compiler wait for each row's loads before the next row's (SYMV n = 16384: the diagonal blocks' rows then
    // formed the kernel's tail). Packed storage takes the same whole chunks: element (r, c) of either triangle's
    // packing sits at rs(r) + c, and for 0 <= c <= n - 1 that address lies inside the packed array whether or not
    // (r, c) is stored (an unstored c falls into a neighbouring row; rs(r) >= 0 and rs(r) + n - 1 is at most the
    // last element), and the group inside the matrix keeps every chunk's columns in [0, n - 1] (SPMV n = 16384 FP32
    // 126.1 -> 124.0 us). Band rows keep the per-lane choice: their stored range ends at the band's edges.
    const bool whole = FMT != F_BAND && V > 1 && g0 + 64 * V <= s.ncols;
    auto checked = [&](int r0, int r1) {
        for (int i = r0; i < r1; i += U) {
            T el[U][V];
            R xr[U];
            if (whole) {
                if constexpr (FMT != F_BAND && V > 1) {
#pragma unroll
                    for (int u = 0; u < U; u++) {
                        const u32x4 t = row16<FMT>(a + row_start<FMT>(s, min(i + u, r1 - 1)) + c0);
                        __builtin_memcpy(el[u], &t, 16);
                        xr[u] = (dirs & DIR_COL) && i + u < r1 ? (R)x[(ll)(i + u) * ix] : R(0);
                    }
                }
            } else {
#pragma unroll
                for (int u = 0; u < U; u++) {
                    const int r = i + u;
                    int lo, hi;
                    stored_range(s, band, r, lo, hi);
                    if (r >= r1) hi = lo - 1;
                    const T *ar = a + row_start<FMT>(s, r);
                    if constexpr (V > 1) {
                        if (c0 <= hi && c0 + V - 1 >= lo && c0 + V <= s.ncols) {
                            const u32x4 t = row16<FMT>(ar + c0);
                            __builtin_memcpy(el[u], &t, 16);
                        } else {
#pragma unroll
                            for (int e = 0; e < V; e++) el[u][e] = c0 + e >= lo && c0 + e <= hi ? ar[c0 + e] : T(0);
                        }
                    } else {
                        el[u][0] = c0 >= lo && c0 <= hi ? ar[c0] : T(0);
                    }
                    xr[u] = (dirs & DIR_COL) && r < r1 ? (R)x[(ll)r * ix] : R(0);
                }
            }
            R rs[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int r = i + u;
                int lo, hi;
                stored_range(s, band, r, lo, hi);
                if (r >= r1) hi = lo - 1;
                R t = 0;
#pragma unroll
                for (int e = 0; e < V; e++) {
                    const int j = c0 + e;
                    const R av = j >= lo && j <= hi ? (R)el[u][e] : R(0);
                    if ((dirs & DIR_COL) && (!skipdiag || j != r)) sc[e] = fma_r(av, xr[u], sc[e]);
                    t = fma_r(av, xc[e], t);
                }
                rs[u] = t;
            }
            if (dirs & DIR_ROW) reduce_rows(i, r1, rs);
        }
    };
    // unchecked rows: every load of a batch is issued before the first product
    auto load = [&](int i, T (&el)[U][V], R (&xr)[U]) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const T *ar = a + row_start<FMT>(s, i + u) + c0;
            if constexpr (V > 1) {
                const u32x4 t = row16<FMT>(ar);
                __builtin_memcpy(el[u], &t, 16);
            } else {
                el[u][0] = *ar;
            }
            xr[u] = (dirs & DIR_COL) ? (R)x[(ll)(i + u) * ix] : R(0);
        }
    };
    auto use = [&](int i, const T (&el)[U][V], const R (&xr)[U]) {
        R rs[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            R t = 0;
#pragma unroll
            for (int e = 0; e < V; e++) {
                const R av = (R)el[u][e];
                if (dirs & DIR_COL) sc[e] = fma_r(av, xr[u], sc[e]);
                t = fma_r(av, xc[e], t);
            }
            rs[u] = t;
        }
        if (dirs & DIR_ROW) reduce_rows(i, fb, rs);
    };
    checked(rb, fa);
    for (int i = fa; i < fb; i += U) {
        T el[U][V];
        R xr[U];
        load(i, el, xr);
        use(i, el, xr);
    }
    checked(fb, re);
    if (dirs & DIR_COL) {   // the band's column sums: the 4 waves' sums added in wave order
        __shared__ R red[NT / 64][64 * V];
#pragma unroll
        for (int e = 0; e < V; e++) red[w][lane * V + e] = sc[e];
        __syncthreads();
        if (w == 0) {
#pragma unroll
            for (int e = 0; e < V; e++) {
                R t = red[0][lane * V + e];
#pragma unroll
                for (int q = 1; q < NT / 64; q++) t += red[q][lane * V + e];
                if (c0 + e < s.ncols) P[(ll)bandi * s.ncols + c0 + e] = t;
            }
        }
    }
}

// y_k = alpha·(Σ_band P[band][k] + Σ_group Q[group][k] (+ x_k for a unit diagonal)) + beta·y_k; y is not read when
// beta = 0 (reference: level12.cl:280). A workgroup of FT threads takes 64 outputs; wave q adds every G-th partial
// from the q-th (loads issued 8 at a time), then wave 0 adds the G sums in wave order: a fixed order for every output.
// G = 16 waves: with 4, the 16384 outputs of an n = 16384 product kept about 8 KiB of loads in flight per CU.
constexpr int FT = 1024;
template <class T>
__global__ void __launch_bounds__(FT) mv_finish(Shape s, int band, int ny, int dirs, int parts, int gw,
                                                const typename Comp<T>::R *P, const typename Comp<T>::R *Q,
                                                typename Comp<T>::R alpha, typename Comp<T>::R beta, const T *x, ll ix,
                                                int add_x, T *y, ll iy) {
    using R = typename Comp<T>::R;
    constexpr int G = FT / 64;
    const int lane = threadIdx.x & 63, q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int k = blockIdx.x * 64 + lane;
    auto sum = [&](const R *base, int first, int last, R t) {   // Σ base[j·ny], j = first + q, first + q + G, ... ≤ last
        int j = first + q;
        for (; j + 7 * G <= last; j += 8 * G) {
            R v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = base[(ll)(j + u * G) * ny];
#pragma unroll
            for (int u = 0; u < 8; u++) t += v[u];
        }
        for (; j <= last; j += G) t += base[(ll)j * ny];
        return t;
    };
    R t = 0;
    if (k < ny) {
        if (dirs & DIR_COL) t = sum(P + k, 0, parts - 1, t);
        if (dirs & DIR_ROW) {
            int lo, hi;
            stored_range(s, band, k, lo, hi);
            if (lo <= hi) t = sum(Q + k, lo / gw, hi / gw, t);
        }
    }
    __shared__ R red[G][64];
    red[q][lane] = t;
    __syncthreads();
    if (q != 0 || k >= ny) return;
    R u = red[0][lane];
#pragma unroll
    for (int w = 1; w < G; w++) u += red[w][lane];
    if (add_x) u += (R)x[(ll)k * ix];
    T *yp = y + (ll)k * iy;
    *yp = (T)(beta == R(0) ? alpha * u : fma_r(alpha, u, beta * (R)*yp));
}

// ---------------- rank-1 / rank-2 updates of the stored elements ----------------
// Rank updates A += alpha·x·yᵀ (+ alpha·y·xᵀ) on the stored elements: fma(alpha·x_i, y_j, a), then
// fma(alpha·y_i, x_j, ·) (reference: level12.cl:466-476), each element read and written once. The grid and the row
// classification are those of mv_kernel: a workgroup owns a group of 64·V columns and a band of rows, its waves a
// quarter of the band each; a lane loads its columns' y_j (and x_j) once. Rows that store the whole group take
// batches of U rows with every load issued before the first store; rows near the diagonal or the band's edges are
// checked per element.
template <class T, int V, int FMT>
__global__ void __launch_bounds__(NT) rank_kernel(Shape s, typename Comp<T>::R alpha, const T *x, ll ix, const T *y,
                                                  ll iy, int two, int rpp, T *a) {
    using R = typename Comp<T>::R;
    constexpr bool band = FMT == F_BAND;
    constexpr int U = UB<V>;
    const int lane = threadIdx.x & 63;
    const int g = blockIdx.x, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g0 = g * 64 * V, g1 = min(g0 + 64 * V, s.ncols) - 1, c0 = g0 + lane * V;
    const int rpw = rpp / (NT / 64);
    const int bandi = s.tri == TRI_UPPER ? (int)gridDim.y - 1 - (int)blockIdx.y : (int)blockIdx.y;   // as mv_kernel
    int rb = bandi * rpp + w * rpw, re = min(s.nrows, rb + rpw);
    if (s.tri == TRI_LOWER) rb = max(rb, g0);
    if (s.tri == TRI_UPPER) re = min(re, g1 + 1);
    if (band) {
        rb = max(rb, g0 - s.KU);
        re = min(re, g1 + s.KL + 1);
    }
    R yc[V], xc[V];
#pragma unroll
    for (int e = 0; e < V; e++) {
        yc[e] = c0 + e < s.ncols ? (R)y[(ll)(c0 + e) * iy] : R(0);
        xc[e] = two && c0 + e < s.ncols ? (R)x[(ll)(c0 + e) * ix] : R(0);
    }
    int fa = rb, fb = re;   // rows [fa, fb) store every column of the group (as in mv_kernel)
    if (g0 + 64 * V > s.ncols) {
        fb = fa;
    } else {
        if (band) {
            fa = max(fa, g1 - s.KU);
            fb = min(fb, g0 + s.KL + 1);
        }
        if (s.tri == TRI_LOWER) fa = max(fa, g1 + 1);
        if (s.tri == TRI_UPPER) fb = min(fb, g0);
    }
    fa = min(fa, re);
    fb = max(fa, min(fb, re));
    fb = fa + (fb - fa) / U * U;
    auto update = [&](R (&v)[V], R xi, R yi) {
#pragma unroll
        for (int e = 0; e < V; e++) {
            v[e] = fma_r(xi, yc[e], v[e]);
            if (two) v[e] = fma_r(yi, xc[e], v[e]);
        }
    };
    auto checked = [&](int r0, int r1) {
        for (int i = r0; i < r1; i++) {
            int lo, hi;
            stored_range(s, band, i, lo, hi);
            const R xi = alpha * (R)x[(ll)i * ix], yi = two ? alpha * (R)y[(ll)i * iy] : R(0);
            T *ar = a + row_start<FMT>(s, i);
            R v[V];
#pragma unroll
            for (int e = 0; e < V; e++) v[e] = c0 + e >= lo && c0 + e <= hi ? (R)ar[c0 + e] : R(0);
            update(v, xi, yi);
#pragma unroll
            for (int e = 0; e < V; e++)
                if (c0 + e >= lo && c0 + e <= hi) ar[c0 + e] = (T)v[e];
        }
    };
    checked(rb, fa);
    for (int i = fa; i < fb; i += U) {
        Vec<T> el[U];
        R xi[U], yi[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const T *ar = a + row_start<FMT>(s, i + u) + c0;
            if constexpr (V > 1) el[u].u = *reinterpret_cast<const u32x4 *>(ar);
            else el[u].e[0] = *ar;
            xi[u] = alpha * (R)x[(ll)(i + u) * ix];
            yi[u] = two ? alpha * (R)y[(ll)(i + u) * iy] : R(0);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            R v[V];
#pragma unroll
            for (int e = 0; e < V; e++) v[e] = (R)el[u].e[e];
            update(v, xi[u], yi[u]);
#pragma unroll
            for (int e = 0; e < V; e++) el[u].e[e] = (T)v[e];
            T *ar = a + row_start<FMT>(s, i + u) + c0;
            if constexpr (V > 1) *reinterpret_cast<u32x4 *>(ar) = el[u].u;
            else *ar = el[u].e[0];
        }
    }
    checked(fb, re);
}

// ---------------- triangular solves ----------------
constexpr int SB = 128;   // rows per diagonal block
template <class T, class R>
__global__ void __launch_bounds__(NT) to_work(int n, const T *x, ll ix, R *xf) {
    const int i = blockIdx.x * NT + threadIdx.x;
    if (i < n) xf[i] = (R)x[(ll)i * ix];
}
template <class T, class R>
__global__ void __launch_bounds__(NT) from_work(int n, const R *xf, T *x, ll ix) {
    const int i = blockIdx.x * NT + threadIdx.x;
    if (i < n) x[(ll)i * ix] = (T)xf[i];
}

__device__ __forceinline__ float lane_value(float v, int k) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), k));
}
__device__ __forceinline__ double lane_value(double v, int k) {
    const long long b = __builtin_bit_cast(long long, v);
    const int lo = __builtin_amdgcn_readlane((int)b, k), hi = __builtin_amdgcn_readlane((int)(b >> 32), k);
    return __builtin_bit_cast(double, (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}

// Diagonal block [p, p + b) of op(A), b ≤ SB: loaded by the whole workgroup (a thread's 64 loads all in flight at
// once), stored in LDS as it lies in A, and substituted by one wave (see solve).
template <class T, int FMT>
struct Diag {
    using R = typename Comp<T>::R;
    static constexpr int RPT = SB * SB / NT;   // elements per thread
    static constexpr int KS = 8;               // steps per LDS read
    T e[RPT];
    T d0, d1;   // wave 0: the diagonal entries of lane l's rows (see substitute)

    // Column w of A in the block; first row q0 (uniform across a wave: row offsets are scalar). Element (q, w),
    // A(p + q, p + w), is needed where it lies in A's stored triangle (the solve uses no other entry) and, for a
    // band, inside the band; elsewhere the value is zero. Every lane loads, without a branch, from an address
    // clamped into storage: rows past the block re-read its last row, and outside full storage the column is
    // clamped into the row's stored entries (the diagonal is always among them: a unit diagonal that is not
    // referenced is still in storage). The values that are not needed are replaced by zero when placed.
    __device__ __forceinline__ void load(const Shape &s, const T *__restrict__ a, int p, int b, int fwd) {
        if (threadIdx.x < 64) {   // the diagonal of the rows lane l substitutes (clamped into the block)
            const int l = threadIdx.x;
            const int i0 = min(fwd ? l : b - 1 - l, b - 1), i1 = min(fwd ? l + 64 : b - 1 - (l + 64), b - 1);
            const int j0 = max(i0, 0), j1 = max(i1, 0);
            d0 = a[row_start<FMT>(s, p + j0) + p + j0];
            d1 = a[row_start<FMT>(s, p + j1) + p + j1];
        }
        const int w = threadIdx.x % SB, q0 = __builtin_amdgcn_readfirstlane(threadIdx.x / SB);
        const bool lowA = s.tri == TRI_LOWER;
        const int bw = lowA ? s.KL : s.KU;   // band width on the stored side
#pragma unroll
        for (int u = 0; u < RPT; u++) {
            const int q = min(u * (NT / SB) + q0, b - 1);
            int c = min(w, b - 1);
            if constexpr (FMT != F_FULL) {
                c = lowA ? min(c, q) : max(c, q);
                if constexpr (FMT == F_BAND) c = lowA ? max(c, q - bw) : min(c, q + bw);
            }
            e[u] = a[row_start<FMT>(s, p + q) + p + c];
        }
    }

    // The loaded block goes to LDS as it lies in A: raw[q][w] = A(p + q, p + w), rows padded to SB + 1 elements, so a
    // thread's stores are constant offsets from one address. Only the strict stored triangle is kept (and, for a
    // band, the band): the diagonal and the other triangle are stored as zeros, so a row stops changing once its own
    // step is past. The substitution order (transpose, direction) is applied when the block is read.
    __device__ __forceinline__ void place(const Shape &s, R (*raw)[SB + 1]) const {
        const int w = threadIdx.x % SB, q0 = __builtin_amdgcn_readfirstlane(threadIdx.x / SB);
        const bool lowA = s.tri == TRI_LOWER;
        const int bw = lowA ? s.KL : s.KU;
#pragma unroll
        for (int u = 0; u < RPT; u++) {
            const int q = u * (NT / SB) + q0;
            const int d = lowA ? q - w : w - q;   // distance from the diagonal into the stored triangle
            raw[q][w] = d > 0 && (FMT != F_BAND || d <= bw) ? (R)e[u] : R(0);
        }
    }

    // Places the loaded block in LDS, then wave 0 substitutes, starting from the block's right-hand side rhs[0 .. b)
    // (in A's row order, in LDS), and writes x of the block to xf. Called by the whole workgroup; the barrier orders
    // the writes of rhs before wave 0 reads it.
    // In solve order (r' = r, c' = c forward; both reversed backward, so the solve is always forward) step k takes
    // x_k = v_k·(1/d_k) from lane k and subtracts op(A)(r', k)·x_k from every row r'. Lane l owns rows l and l + 64
    // and the reciprocals of their diagonal entries; a row's entries on and above the diagonal are zero in LDS, so
    // its value stops changing once its own step is past. Columns are read from LDS 8 steps at a time, so the
    // sequential chain per step is a multiply, a lane read and a fused multiply-add (reference: level12.cl:493-548;
    // the reference divides by the diagonal, here its reciprocal is taken once: the solution differs by rounding
    // only).
    __device__ __forceinline__ void solve(const Shape &s, int trans, int fwd, int p, int b, const R *rhs, R *xf,
                                          R (*raw)[SB + 1]) const {
        place(s, raw);
        __syncthreads();
        if (threadIdx.x >= 64) return;
        if (trans) {
            if (fwd) substitute<true, true>(s, p, b, rhs, xf, raw);
            else substitute<true, false>(s, p, b, rhs, xf, raw);
        } else {
            if (fwd) substitute<false, true>(s, p, b, rhs, xf, raw);
            else substitute<false, false>(s, p, b, rhs, xf, raw);
        }
    }
    template <bool TR, bool FW>
    __device__ __forceinline__ void substitute(const Shape &s, int p, int b, const R *rhs, R *xf, R (*raw)[SB + 1]) const {
        const int l = threadIdx.x, n0 = b < 64 ? b : 64;
        // row of the block in A's order for solve-order index x; lanes past b wrap into the block (values dropped)
        const auto idx = [&](int x) { return (FW ? x : b - 1 - x) & (SB - 1); };
        const bool has1 = l + 64 < b;
        const int i0 = idx(l), i1 = idx(l + 64);
        R v0 = l < b ? rhs[i0] : R(0), v1 = has1 ? rhs[i1] : R(0);
        const R r0 = s.unit || l >= b ? R(1) : R(1) / (R)d0, r1 = s.unit || !has1 ? R(1) : R(1) / (R)d1;
        // op(A) in solve order at (row of A i, step k); k < b, so the column index needs no wrap
        const auto col = [&](int k, int i) { const int j = FW ? k : b - 1 - k; return TR ? raw[j][i] : raw[i][j]; };
        int k = 0;
        for (; k + KS <= n0; k += KS) {
            R c0[KS], c1[KS];
#pragma unroll
            for (int u = 0; u < KS; u++) {
                c0[u] = col(k + u, i0);
                c1[u] = col(k + u, i1);
            }
#pragma unroll
            for (int u = 0; u < KS; u++) {
                const R xk = lane_value(v0 * r0, k + u);
                v0 = fma_r(-c0[u], xk, v0);
                v1 = fma_r(-c1[u], xk, v1);
            }
        }
        for (; k < n0; k++) {
            const R xk = lane_value(v0 * r0, k);
            v0 = fma_r(-col(k, i0), xk, v0);
            v1 = fma_r(-col(k, i1), xk, v1);
        }
        for (; k + KS <= b; k += KS) {
            R c1[KS];
#pragma unroll
            for (int u = 0; u < KS; u++) c1[u] = col(k + u, i1);
#pragma unroll
            for (int u = 0; u < KS; u++) v1 = fma_r(-c1[u], lane_value(v1 * r1, k + u - 64), v1);
        }
        for (; k < b; k++) v1 = fma_r(-col(k, i1), lane_value(v1 * r1, k - 64), v1);
        if (l < b) xf[p + i0] = v0 * r0;
        if (has1) xf[p + i1] = v1 * r1;
    }
};

// The region of A at rows [R0, R0 + br), columns [C0, C0 + bc) (br, bc ≤ SB) into e[], laid out as the diagonal block
// (thread: column w = t % SB, rows q0 + 2u). Every lane loads, without a branch, from an address inside its row's
// storage (rows past br re-read the last row; outside full storage the column is clamped into the row's stored
// entries); `needed` tells which values are elements of A in the region.
template <class T, int FMT>
__device__ __forceinline__ void load_region(const Shape &s, const T *__restrict__ a, int R0, int br, int C0, int bc,
                                            T (&e)[SB * SB / NT]) {
    const int w = threadIdx.x % SB, q0 = __builtin_amdgcn_readfirstlane(threadIdx.x / SB);
#pragma unroll
    for (int u = 0; u < SB * SB / NT; u++) {
        const int i = R0 + min(u * (NT / SB) + q0, br - 1);
        int j = C0 + min(w, bc - 1);
        if constexpr (FMT == F_PACKL) j = min(j, i);
        else if constexpr (FMT == F_PACKU) j = max(j, i);
        else if constexpr (FMT == F_BAND) j = max(min(j, i + s.KU), i - s.KL);
        e[u] = a[row_start<FMT>(s, i) + j];
    }
}
// Whether value u of load_region is an element of A, for a region that couples two different diagonal blocks: such a
// region lies strictly inside A's stored triangle (the solve runs over the triangle's blocks in order), so only the
// region's bounds and, for a band, the band decide.
template <int FMT>
__device__ __forceinline__ bool needed(const Shape &s, int R0, int br, int C0, int bc, int u) {
    const int w = threadIdx.x % SB, q = u * (NT / SB) + __builtin_amdgcn_readfirstlane(threadIdx.x / SB);
    const int dj = (C0 + w) - (R0 + q);   // column minus row
    return q < br && w < bc && (FMT != F_BAND || (dj >= -s.KL && dj <= s.KU));
}

// x_r -= Σ_{c in [p, p+b)} A(r, c)·x_c for rows r of [r0, r1) (op(A) = A), 32 rows per part: in part vb a wave takes
// 8 rows, its lanes the block's columns (b ≤ BW: BW / 64 per lane), then the butterfly sums the 8 rows. The block's
// solution x_c is read from xv (xf itself, or the separate solution vector of the inverse-based solve).
constexpr int UPD_ROWS = 8 * (NT / 64), UPD_COLS = 64;   // rows per part of the two updates
template <class T, int FMT, int BW = SB>
__device__ __forceinline__ void update_rows(const Shape &s, const T *__restrict__ a, int p, int b, int r0, int r1,
                                            typename Comp<T>::R *xf, const typename Comp<T>::R *xv, int vb) {
    using R = typename Comp<T>::R;
    constexpr int RW = 8, NC = BW / 64;
    const int lane = threadIdx.x & 63;
    const int rbase = r0 + (vb * (NT / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * RW;
    if (rbase >= r1) return;
    R xc[NC];
#pragma unroll
    for (int j = 0; j < NC; j++) xc[j] = lane + 64 * j < b ? xv[p + 64 * j + lane] : R(0);
    // the butterfly below leaves row rbase + lane / (64 / RW) in the lanes lane % (64 / RW) = 0: its old value is
    // loaded now, so the subtraction at the end waits for no load (no other workgroup of the launch writes these rows)
    const int rown = rbase + lane / (64 / RW);
    const R xold = rown < r1 ? xf[rown] : R(0);
    R t[RW];
#pragma unroll
    for (int u = 0; u < RW; u++) {
        const int r = rbase + u;
        int lo, hi;
        stored_range(s, FMT == F_BAND, r, lo, hi);
        if (r >= r1) hi = lo - 1;
        const T *ar = a + row_start<FMT>(s, r);
        R e[NC];
#pragma unroll
        for (int j = 0; j < NC; j++) {
            const int c = p + 64 * j + lane;
            e[j] = lane + 64 * j < b && c >= lo && c <= hi ? (R)ar[c] : R(0);
        }
        t[u] = e[0] * xc[0];
#pragma unroll
        for (int j = 1; j < NC; j++) t[u] = fma_r(e[j], xc[j], t[u]);
    }
    asm volatile("" ::"v"(xold));   // xold's load stays with the others (see upd_rows_full)
    int base = 0;
    butterfly<0, RW>(t, lane, base);
    if ((lane & (64 / RW - 1)) == 0 && rbase + base < r1) xf[rbase + base] = xold - t[0];
}

// x_r -= Σ_{c in [p, p+b)} A(c, r)·x_c for rows r of [r0, r1) (op(A) = Aᵀ), 64 consecutive r per part: each wave
// takes BW / 4 of the block's rows c (all of its loads in flight; neighbouring lanes read neighbouring elements of a
// row of A), then wave 0 adds the 4 sums in wave order. Called by the whole workgroup (two barriers; `red` is free
// again on return).
template <class T, int FMT, int BW = SB>
__device__ __forceinline__ void update_cols(const Shape &s, const T *__restrict__ a, int p, int b, int r0, int r1,
                                            typename Comp<T>::R *xf, const typename Comp<T>::R *xv, int vb,
                                            typename Comp<T>::R (*red)[64]) {
    using R = typename Comp<T>::R;
    constexpr int G = NT / 64, CW = BW / G;
    const int lane = threadIdx.x & 63, q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = r0 + vb * UPD_COLS + lane;
    const R xold = q == 0 && r < r1 ? xf[r] : R(0);   // loaded ahead of the sums (only this workgroup writes row r)
    R t = 0;
    if (r < r1) {
        R v[CW];
#pragma unroll
        for (int u = 0; u < CW; u++) {
            const int c = p + q * CW + u;
            int lo, hi;
            stored_range(s, FMT == F_BAND, c, lo, hi);
            v[u] = q * CW + u < b && r >= lo && r <= hi ? (R)a[row_start<FMT>(s, c) + r] : R(0);
        }
#pragma unroll
        for (int u = 0; u < CW; u++)
            if (q * CW + u < b) t = fma_r(v[u], xv[p + q * CW + u], t);
    }
    red[q][lane] = t;
    __syncthreads();
    if (q == 0 && r < r1) {
        R sum = red[0][lane];
#pragma unroll
        for (int w = 1; w < G; w++) sum += red[w][lane];
        xf[r] = xold - sum;
    }
    __syncthreads();
}

// One step of the blocked solve: block [p, p + b) in solve order, after block [pp, pp + pb) (pb = 0: the first step).
// The previous block's solution is final (the previous launch wrote it), and its update reaches rows [t0, t1) of
// this block and rows [o0, o1) beyond it. Workgroups 1.. apply the update to [o0, o1), one part each. Workgroup 0
// issues the loads of this block's diagonal part and of the 128×128 region of A that couples the two blocks
// (op(A) = A: this block's rows × the previous block's columns; op(A) = Aᵀ: the previous block's rows × this block's
// columns) at once, forms this block's right-hand side x_r − Σ_c op(A)(r, c)·x_c in LDS (row sums: transposing
// butterfly over each wave's 64 columns, then the two waves of a row set; column sums: per thread, then the two row
// sets), and substitutes. The two sides read only the previous block's solution and write disjoint rows, so one
// launch per block suffices (the update of block q and the solve of block q + 1 in one launch: a one-block
// look-ahead).
template <class T, int FMT>
__global__ void __launch_bounds__(NT) solve_step(Shape s, const T *__restrict__ a, int trans, int fwd, int pp, int pb, int p,
                                                 int b, int t0, int t1, int o0, int o1, typename Comp<T>::R *xf) {
    using R = typename Comp<T>::R;
    constexpr int RPT = SB * SB / NT;
    __shared__ R raw[SB][SB + 1];
    __shared__ R red[NT / 64][64];
    __shared__ R xp[SB], rhs[SB];
    if (blockIdx.x > 0) {
        if (trans) update_cols<T, FMT>(s, a, pp, pb, o0, o1, xf, xf, blockIdx.x - 1, red);
        else update_rows<T, FMT>(s, a, pp, pb, o0, o1, xf, xf, blockIdx.x - 1);
        return;
    }
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int w = tid % SB, q0 = __builtin_amdgcn_readfirstlane(tid / SB);
    const bool upd = t1 > t0;
    // coupling region: rows [R0, R0 + br), columns [C0, C0 + bc) of A
    const int R0 = trans ? pp : p, br = trans ? pb : b, C0 = trans ? p : pp, bc = trans ? b : pb;
    Diag<T, FMT> d;
    d.load(s, a, p, b, fwd);
    T eo[RPT];
    if (upd) load_region<T, FMT>(s, a, R0, br, C0, bc, eo);
    const R own = tid < b ? xf[p + tid] : R(0);
    if (tid < SB) xp[tid] = upd && tid < pb ? xf[pp + tid] : R(0);
    __syncthreads();
    R sum = 0;   // thread tid < b: Σ_c op(A)(p + tid, c)·x_c over the previous block
    if (upd) {
        if (!trans) {
            const R xw = xp[w];
            R t[RPT];
#pragma unroll
            for (int u = 0; u < RPT; u++) t[u] = needed<FMT>(s, R0, br, C0, bc, u) ? (R)eo[u] * xw : R(0);
            int base = 0;
            butterfly<0, RPT>(t, lane, base);   // lane l: the wave's sum for u = l, row q0 + 2l
            red[wave][lane] = t[0];
            __syncthreads();
            if (tid < b) sum = red[2 * (tid & 1)][tid >> 1] + red[2 * (tid & 1) + 1][tid >> 1];
        } else {
            R t = 0;
#pragma unroll
            for (int u = 0; u < RPT; u++)
                if (needed<FMT>(s, R0, br, C0, bc, u)) t = fma_r((R)eo[u], xp[u * (NT / SB) + q0], t);
            R *half = &red[0][0];   // [2][SB]: the column sums of row sets q0 = 0 and 1
            half[q0 * SB + w] = t;
            __syncthreads();
            if (tid < b) sum = half[tid] + half[SB + tid];
        }
    }
    if (tid < b) rhs[tid] = own - sum;
    d.solve(s, trans, fwd, p, b, rhs, xf, raw);
}

// ---------------- inverse-based solve (full storage) ----------------
// In solve order (index g is row g of A forward, n − 1 − g backward, so op(A) becomes lower triangular) the order
// is cut into blocks of IB rows (256 below order INV_BIG, 512 from there), q = 0 .. nbI − 1, the last one partial.
// The diagonal blocks D_q are inverted up front, all at once: their 128-row diagonal blocks in FP64 (one launch),
// then level by level the lower-left quadrants −inv(D₂)·C·inv(D₁) of the sub-blocks of 256 (and 512) rows by two
// batched GEMMs per level; one more batched GEMM forms E_q = inv(D_q)·C_q, C_q being the block of op(A) that couples
// block q to block q − 1. Step q is x_q = inv(D_q)·r_q − E_q·x_{q−1}, r_q being block q's right-hand side after the
// updates of blocks ≤ q − 2: two IB × IB matrix-vector products, split over IB / INV_ROWS workgroups (16 rows of 16
// lanes, or for IB = 512 4 rows of 64 lanes, so that each workgroup loads 32 KiB of FP32) with no synchronisation
// between them, while the launch's other workgroups apply x_{q−1} to the rows beyond block q (the one-block
// look-ahead of solve_step). The chain per block is a launch, the loads of the rows of inv(D_q) and E_q and a sum
// across each row's lanes, where solve_step has the diagonal block's loads, its right-hand side and a 128-step
// substitution. The solution goes to a second vector xs, since the solving workgroups read r_q
// from xf while others write x_q. The reference substitutes (level12.c:303-347, level12.cl:493-548); the results
// differ from substitution by rounding only.
// Sum over each row of 16 lanes, left in every lane of the row, by DPP moves (quad_perm [1,0,3,2] and [2,3,0,1],
// row_half_mirror, row_mirror); the order of the additions is fixed, and each lane's sum is the same value.
__device__ __forceinline__ int dpp_move(int v, int ctrl) {
    switch (ctrl) {   // the control must be a constant of the instruction
    case 0: return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
    case 1: return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
    case 2: return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
    default: return __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);
    }
}
__device__ __forceinline__ float row16_sum(float v) {
#pragma unroll
    for (int c = 0; c < 4; c++) v += __builtin_bit_cast(float, dpp_move(__builtin_bit_cast(int, v), c));
    return v;
}
__device__ __forceinline__ double row16_sum(double v) {
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const long long b = __builtin_bit_cast(long long, v);
        const int lo = dpp_move((int)b, c), hi = dpp_move((int)(b >> 32), c);
        v += __builtin_bit_cast(double, (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
    }
    return v;
}
// Smallest order solved this way: the set-up costs about 85 µs whatever the order (the inversion launch alone 46),
// substitution 10.5 µs per 128 rows. MI355X, FP32, µs per call, substitution against inverted blocks: n = 1024 80 /
// 96 (op(A) = A / Aᵀ) against 99; n = 1280 101 / 120 against 103; n = 1536 120 / 144 against 108; n = 2048 160 / 193
// against 118.
constexpr int INV_MIN = 1280;
// From this order on, blocks of 512 rows: half the dependent launches for a larger set-up (E_q of 512², one more
// composition level). MI355X, µs per call, op(A) = A / Aᵀ, 512 against 256 rows: FP32 n = 2048 115 / 117 against
// 103 / 103, n = 4096 131 / 136 against 137 / 136, n = 8192 179 / 187 against 209 / 206, n = 16384 400 / 398 against
// 427 / 396; FP64 n = 4096 131 / 133 against 138 / 138, n = 8192 176 / 174 against 207 / 203.
constexpr int INV_BIG = 4096;
// Rows of x_q per solving workgroup: each loads 32 KiB of FP32 (the IB = 512 step with 8 or 16 rows per workgroup
// loads 64-128 KiB in each: FP32 n = 16384 op(A) = A 413 and 466 µs against 400 with 4)
template <int IB> constexpr int INV_ROWS = IB == 256 ? 16 : 4;

// 128 × 128 tiles of D_q and C_q, in solve order, into Dg + q·IB·(IB + 1) and Cg + q·IB² (row stride IB; D_q's
// stride puts element (i, j) of the blocks' rows and columns, counted from block 0, at Dg[i·IB + j]), zero padded: past the
// order, D_q holds the identity and C_q zeros, so inv(D_q) and E_q keep the block's rows apart from the padding.
// Block q = blockIdx.x; blockIdx.y < Q² (Q = IB / 128) is quadrant (y / Q, y % Q) of D_q (diagonal quadrants: the
// triangle with the diagonal, or ones for a unit diagonal, which is not read; below: dense; above: zeros), the
// others quadrant y − Q² of C_q (dense; zeros for q = 0). The region of A goes through LDS, read and written
// coalesced.
template <class T, int IB>
__global__ void __launch_bounds__(NT) inv_gather(Shape s, const T *__restrict__ a, int trans, int fwd,
                                                 typename Comp<T>::R *Dg, typename Comp<T>::R *Cg) {
    using R = typename Comp<T>::R;
    constexpr int Q = IB / SB, RPT = SB * SB / NT;
    __shared__ R tile[SB][SB + 1];
    const int n = s.nrows, q = blockIdx.x, tid = threadIdx.x, w = tid % SB;
    const bool coup = blockIdx.y >= Q * Q;
    const int y = coup ? blockIdx.y - Q * Q : blockIdx.y, qr = y / Q, qc = y % Q;
    R *out = (coup ? Cg + (ll)q * IB * IB : Dg + (ll)q * IB * (IB + 1)) + (ll)qr * SB * IB + qc * SB;
    // mode 0: zeros, 1: dense, 2: lower triangle with the diagonal
    const int mode = coup ? (q > 0 ? 1 : 0) : (qr == qc ? 2 : qr > qc ? 1 : 0);
    const int G0 = q * IB + qr * SB, H0 = (coup ? q - 1 : q) * IB + qc * SB;   // solve-order row and column
    const int kmax = min(max(n - G0, 0), SB), cmax = min(max(n - H0, 0), SB);
    if (mode == 1 && kmax > 0 && cmax > 0) {
        // tile[i][j] = A(ar0 + i, ac0 + j): op(A) = A: rows from the tile's rows; op(A) = Aᵀ: from its columns
        const int gs = fwd ? G0 : n - G0 - kmax, hs = fwd ? H0 : n - H0 - cmax;
        const int ar0 = trans ? hs : gs, nr = trans ? cmax : kmax, ac0 = trans ? gs : hs, nc = trans ? kmax : cmax;
        T e[RPT];   // every load in flight before the first store to LDS (addresses clamped into the region)
#pragma unroll
        for (int u = 0; u < RPT; u++) {
            const int i = u * (NT / SB) + tid / SB;
            e[u] = a[(ll)(ar0 + min(i, nr - 1)) * s.ld + ac0 + min(w, nc - 1)];
        }
#pragma unroll
        for (int u = 0; u < RPT; u++) tile[u * (NT / SB) + tid / SB][w] = (R)e[u];
    }
    if (mode == 2 && kmax > 0) {   // the diagonal tile: A rows and columns are the same range
        const int gs = fwd ? G0 : n - G0 - kmax;
        T e[RPT];
#pragma unroll
        for (int u = 0; u < RPT; u++) {
            const int i = u * (NT / SB) + tid / SB;
            e[u] = a[(ll)(gs + min(i, kmax - 1)) * s.ld + gs + min(w, kmax - 1)];
        }
#pragma unroll
        for (int u = 0; u < RPT; u++) tile[u * (NT / SB) + tid / SB][w] = (R)e[u];
    }
    __syncthreads();
    const int c = w, ic = fwd ? c : cmax - 1 - c;   // the column's offset in its A range
    for (int k = tid / SB; k < SB; k += NT / SB) {
        const int ik = fwd ? k : kmax - 1 - k;
        R v = R(0);
        if (k < kmax && c < cmax) {
            const R e = trans ? tile[ic][ik] : tile[ik][ic];
            if (mode == 1 || (mode == 2 && c < k)) v = e;
            else if (mode == 2 && c == k) v = s.unit ? R(1) : e;
        } else if (mode == 2 && k == c) {
            v = R(1);
        }
        out[(ll)k * IB + c] = v;
    }
}

// The updates of the inverse-based solve: x_r −= Σ_c op(A)(r, c)·x_c over a whole previous block c ∈ [p, p + BW)
// of full storage, for rows r of [r0, r1). Every element they read lies inside the stored triangle (the rows are
// after the block in solve order), so each lane loads without a condition, from a row clamped into [r0, r1), and
// all of a wave's loads are in flight at once; results of clamped rows are not stored. op(A) = A: 32 rows per part,
// a wave per 8 rows, BW / 64 columns per lane, a transposing butterfly over the 8 rows (row rbase + lane / 8 ends in
// lanes lane % 8 = 0). op(A) = Aᵀ: 64 consecutive rows r per part, each wave BW / 4 of the block's rows c, the 4
// waves' sums added in wave order by wave 0. No other workgroup of the launch writes rows [r0, r1), so the old
// values are loaded with the rest.
template <class T, int BW>
__device__ __forceinline__ void upd_rows_full(const Shape &s, const T *__restrict__ a, int p, int r0, int r1,
                                              typename Comp<T>::R *xf, const typename Comp<T>::R *xv, int vb) {
    using R = typename Comp<T>::R;
    constexpr int RW = 8, NC = BW / 64;
    const int lane = threadIdx.x & 63;
    const int rbase = r0 + (vb * (NT / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * RW;
    if (rbase >= r1) return;
    const int rown = rbase + lane / (64 / RW);
    const R xold = xf[min(rown, r1 - 1)];
    R xc[NC], e[RW][NC];
#pragma unroll
    for (int j = 0; j < NC; j++) xc[j] = xv[p + 64 * j + lane];
#pragma unroll
    for (int u = 0; u < RW; u++) {
        const T *ar = a + (ll)min(rbase + u, r1 - 1) * s.ld + p + lane;
#pragma unroll
        for (int j = 0; j < NC; j++) e[u][j] = (R)ar[64 * j];
    }
    // keeps the load of xold issued with the others: left alone, the compiler sinks it to the store, one more round
    // trip at the end of the launch's critical path
    asm volatile("" ::"v"(xold));
    R t[RW];
#pragma unroll
    for (int u = 0; u < RW; u++) {
        t[u] = e[u][0] * xc[0];
#pragma unroll
        for (int j = 1; j < NC; j++) t[u] = fma_r(e[u][j], xc[j], t[u]);
    }
    int base = 0;
    butterfly<0, RW>(t, lane, base);
    if ((lane & (64 / RW - 1)) == 0 && rown < r1) xf[rown] = xold - t[0];
}
template <class T, int BW>
__device__ __forceinline__ void upd_cols_full(const Shape &s, const T *__restrict__ a, int p, int r0, int r1,
                                              typename Comp<T>::R *xf, const typename Comp<T>::R *xv, int vb,
                                              typename Comp<T>::R (*red)[64]) {
    using R = typename Comp<T>::R;
    constexpr int G = NT / 64, CW = BW / G;
    const int lane = threadIdx.x & 63, q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = r0 + vb * UPD_COLS + lane, rc = min(r, r1 - 1);
    const R xold = xf[rc];
    const T *ac = a + (ll)(p + q * CW) * s.ld + rc;
    R v[CW];
#pragma unroll
    for (int u = 0; u < CW; u++) v[u] = (R)ac[(ll)u * s.ld];
    R t = 0;
#pragma unroll
    for (int u = 0; u < CW; u++) t = fma_r(v[u], xv[p + q * CW + u], t);
    red[q][lane] = t;
    __syncthreads();
    if (q == 0 && r < r1) {
        R sum = red[0][lane];
#pragma unroll
        for (int w = 1; w < G; w++) sum += red[w][lane];
        xf[r] = xold - sum;
    }
}

// Step q of the inverse-based solve: block q covers rows [p, p + b) of A, block q − 1 rows [pp, pp + pb) (pb = 0:
// the first step). Workgroups 0 .. IB / ROWS − 1 form ROWS rows each of x_q = Di·r_q − Eq·x_{q−1} (L = 256 / ROWS
// lanes per row, IB / L columns per lane, then a fixed-order sum over the row's lanes) into xs; the others apply
// x_{q−1} (in xs) to rows [o0, o1) of xf.
template <class T, int IB>
__global__ void __launch_bounds__(NT) inv_step(Shape s, const T *__restrict__ a, int trans, int fwd, int pp, int pb, int p,
                                               int b, int o0, int o1, const typename Comp<T>::R *__restrict__ Di,
                                               const typename Comp<T>::R *__restrict__ Eq, typename Comp<T>::R *xf,
                                               typename Comp<T>::R *xs) {
    using R = typename Comp<T>::R;
    constexpr int ROWS = INV_ROWS<IB>;
    constexpr int WGS = IB / ROWS, L = NT / ROWS, CPL = IB / L;   // solving workgroups, lanes per row, columns per lane
    static_assert(L >= 16 && L <= 64 && CPL % 4 == 0, "16 to 64 lanes per row, whole 4-column chunks");
    __shared__ R red[NT / 64][64];
    if (blockIdx.x >= WGS) {
        if (trans) upd_cols_full<T, IB>(s, a, pp, o0, o1, xf, xs, blockIdx.x - WGS, red);
        else upd_rows_full<T, IB>(s, a, pp, o0, o1, xf, xs, blockIdx.x - WGS);
        return;
    }
    // lane l of a row takes columns 4Lj + 4l .. 4Lj + 4l + 3: the L lanes of a row read 16·L contiguous bytes of
    // inv(D_q) and E_q per load
    typedef R R4 __attribute__((ext_vector_type(4)));
    constexpr int NJ = CPL / 4;
    const int k = blockIdx.x * ROWS + threadIdx.x / L, l = threadIdx.x % L;
    R4 dv[NJ], ev[NJ];
    R rv[NJ][4], xv[NJ][4];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int c0 = 4 * L * j + 4 * l;
        dv[j] = *reinterpret_cast<const R4 *>(Di + (ll)k * IB + c0);
        if (pb > 0) ev[j] = *reinterpret_cast<const R4 *>(Eq + (ll)k * IB + c0);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // indices clamped into the blocks (the first step has no previous block: pp = pb = 0, index pp)
            const int c = c0 + i, cr = min(c, b - 1), cx = min(c, max(pb - 1, 0));
            rv[j][i] = xf[fwd ? p + cr : p + b - 1 - cr];
            xv[j][i] = pb > 0 ? xs[fwd ? pp + cx : pp + max(pb - 1 - cx, 0)] : R(0);
            if (c >= b) rv[j][i] = R(0);
            if (c >= pb) xv[j][i] = R(0);
        }
    }
    R t = 0;
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) t = fma_r(dv[j][i], rv[j][i], t);
    if (pb > 0) {
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) t = fma_r(-ev[j][i], xv[j][i], t);
    }
    t = row16_sum(t);
#pragma unroll
    for (int d = 16; d < L; d *= 2) t += __shfl_xor(t, d);   // rows of 32 or 64 lanes: the 16-lane sums, in lane order
    if (threadIdx.x % L == 0 && k < b) xs[fwd ? p + k : p + b - 1 - k] = t;
}

// ---------------- launchers ----------------
template <class F> static int by_type(int es, F f) {
    if (es == 2) return f((f16 *)nullptr);
    if (es == 4) return f((float *)nullptr);
    return f((double *)nullptr);
}
template <class F> static int by_fmt(int fmt, F f) {
    if (fmt == F_FULL) return f(std::integral_constant<int, F_FULL>());
    if (fmt == F_BAND) return f(std::integral_constant<int, F_BAND>());
    if (fmt == F_PACKU) return f(std::integral_constant<int, F_PACKU>());
    return f(std::integral_constant<int, F_PACKL>());
}
static unsigned blocks(ll n, int per) { return (unsigned)((n + per - 1) / per); }

// y = alpha·(sums over the stored elements in the directions `dirs`) + beta·y (+ x for add_x); ny outputs.
// Grid of mv_kernel and rank_kernel: a workgroup per (column group of 64·V columns, band of rpp rows), its 4 waves on
// quarters of the band; about 64 workgroups per CU, so the dispatcher balances the uneven work of a triangle (about
// half the workgroups find no rows). At n = 16384 FP32 this is 113 µs for SYMV against 136 with 16 workgroups per CU
// and 16-row batches. Returns the number of column groups.
static ll grid_2d(const Shape &s, int V, ll &parts, ll &rpp) {
    const ll gw = 64LL * V, groups = (s.ncols + gw - 1) / gw;
    const int RU = (V > 1 ? UB<2> : UB<1>) * (NT / 64);   // a band is whole batches for each wave
    const int cus = num_cus > 0 ? num_cus : 256;
    parts = (64LL * cus + groups - 1) / groups;
    const ll maxparts = (s.nrows + RU - 1) / RU;
    if (parts > maxparts) parts = maxparts;
    if (parts < 1) parts = 1;
    if (parts > 65535) parts = 65535;
    rpp = (s.nrows + parts - 1) / parts;
    rpp = (rpp + RU - 1) / RU * RU;
    parts = (s.nrows + rpp - 1) / rpp;
    return groups;
}

static int launch_mv(int es, int fmt, const Shape &s, const void *a, const void *x, ll ix, int dirs, int skipdiag,
                     double alpha, double beta, int add_x, void *y, ll iy, int ny) {
    return by_type(es, [&](auto *tag) -> int {
        using T = std::remove_pointer_t<decltype(tag)>;
        using R = typename Comp<T>::R;
        // 16 bytes per lane: full storage with 16-byte aligned rows; packed storage of 4- and 8-byte elements, whose rows
        // are element-aligned only (row16)
        const bool packed = fmt == F_PACKL || fmt == F_PACKU;
        const bool vec = fmt == F_FULL ? (uintptr_t)a % 16 == 0 && (s.ld * (ll)sizeof(T)) % 16 == 0
                                       : packed && sizeof(T) >= 4 && (uintptr_t)a % sizeof(T) == 0;
        const int V = vec ? VW<T> : 1, gw = 64 * V;
        ll parts, rpp;
        const ll groups = grid_2d(s, V, parts, rpp);
        if (groups > 0x7fffffffLL) G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "level 2: %lld column groups", groups);
        void *pp = nullptr, *qq = nullptr;
        if (dirs & DIR_COL) G9_TRY(scratch(SLOT_P, (size_t)parts * s.ncols * sizeof(R), &pp));
        if (dirs & DIR_ROW) G9_TRY(scratch(SLOT_Q, (size_t)groups * s.nrows * sizeof(R), &qq));
        R *P = (R *)pp, *Q = (R *)qq;
        const T *ap = (const T *)a, *xp = (const T *)x;
        const dim3 grid((unsigned)groups, (unsigned)parts);
        G9_TRY(by_fmt(fmt, [&](auto fc) -> int {
            constexpr int FMT = decltype(fc)::value;
            if constexpr (FMT == F_FULL || ((FMT == F_PACKL || FMT == F_PACKU) && sizeof(T) >= 4)) {
                if (vec) {
                    hipLaunchKernelGGL((mv_kernel<T, VW<T>, FMT>), grid, dim3(NT), 0, stream, s, ap, xp, ix, (int)rpp, dirs,
                                       skipdiag, P, Q);
                    return 0;
                }
            }
            hipLaunchKernelGGL((mv_kernel<T, 1, FMT>), grid, dim3(NT), 0, stream, s, ap, xp, ix, (int)rpp, dirs, skipdiag,
                               P, Q);
            return 0;
        }));
        G9_HIP(hipGetLastError());
        hipLaunchKernelGGL((mv_finish<T>), dim3(blocks(ny, 64)), dim3(FT), 0, stream, s, (int)(fmt == F_BAND), ny, dirs,
                           (int)parts, gw, (const R *)P, (const R *)Q, (R)alpha, (R)beta, xp, ix, add_x, (T *)y, iy);
        G9_HIP(hipGetLastError());
        return 0;
    });
}

static int launch_rank(int es, int fmt, const Shape &s, double alpha, const void *x, ll ix, const void *y, ll iy, int two,
                       void *a) {
    return by_type(es, [&](auto *tag) -> int {
        using T = std::remove_pointer_t<decltype(tag)>;
        using R = typename Comp<T>::R;
        const bool vec = fmt == F_FULL && (uintptr_t)a % 16 == 0 && (s.ld * (ll)sizeof(T)) % 16 == 0;
        const int V = vec ? VW<T> : 1;
        ll parts, rpp;
        const ll groups = grid_2d(s, V, parts, rpp);
        const dim3 grid((unsigned)groups, (unsigned)parts);
        G9_TRY(by_fmt(fmt, [&](auto fc) -> int {
            constexpr int FMT = decltype(fc)::value;
            if constexpr (FMT == F_FULL) {
                if (vec) {
                    hipLaunchKernelGGL((rank_kernel<T, VW<T>, FMT>), grid, dim3(NT), 0, stream, s, (R)alpha, (const T *)x, ix,
                                       (const T *)y, iy, two, (int)rpp, (T *)a);
                    return 0;
                }
            }
            hipLaunchKernelGGL((rank_kernel<T, 1, FMT>), grid, dim3(NT), 0, stream, s, (R)alpha, (const T *)x, ix,
                               (const T *)y, iy, two, (int)rpp, (T *)a);
            return 0;
        }));
        G9_HIP(hipGetLastError());
        return 0;
    });
}

// Work space of the inverse-based solve for order n: the solution vector, then D (later E) and the inverses, nbI·IB·
// (IB + 1) each, C, nbI·IB², and the products of the compositions, at most nbI·IB²/4.
template <class R>
static size_t inv_bytes(int n, int ib) {
    const size_t nbI = (size_t)(n + ib - 1) / ib, m2 = (size_t)ib * ib, sd = m2 + ib;
    return (((size_t)n * sizeof(R) + 255) & ~(size_t)255) + (2 * nbI * sd + nbI * m2 + nbI * m2 / 4) * sizeof(R);
}
// The inverse-based solve of full storage (inv_gather, inv_step) in the work space w (inv_bytes).
template <class T, int IB>
static int solve_inv(const Shape &s, const T *a, int trans, int fwd, typename Comp<T>::R *xf, void *w) {
    using R = typename Comp<T>::R;
    constexpr int QB = IB / SB;
    const int n = s.nrows, nbI = (n + IB - 1) / IB, type = sizeof(R) == 8 ? GEN9BLAS_D : GEN9BLAS_S;
    // D_q and inv(D_q) at stride sd = IB·(IB + 1), so that the sub-blocks of 2h rows of every level of the composition
    // below start at the uniform stride 2h·(IB + 1); C_q and E_q (which reuses D's space) at stride IB²
    const ll m2 = (ll)IB * IB, sd = m2 + IB;
    R *xs = (R *)w;
    R *D = (R *)((char *)w + (((size_t)n * sizeof(R) + 255) & ~(size_t)255));
    R *Di = D + nbI * sd, *C = Di + nbI * sd, *Tm = C + nbI * m2, *E = D;
    // A forward solve on A itself (lower, not transposed) in the work precision, with whole blocks, reads D_q, the
    // quadrants below its diagonal and C_q where they lie in A, at the uniform strides of its diagonal (no gather);
    // every other case gathers them in solve order first (transposing, reversing, converting, padding)
    const bool direct = std::is_same<T, R>::value && !trans && fwd && n % IB == 0;
    const R *Ad = reinterpret_cast<const R *>(a);
    const ll lda = s.ld;
    if (direct) {
        G9_TRY(launch_tri_inverse((int)sizeof(R), Ad, lda, IB * (lda + 1), nbI * QB, Di, IB, sd, s.unit));
    } else {
        hipLaunchKernelGGL((inv_gather<T, IB>), dim3(nbI, 2 * QB * QB), dim3(NT), 0, stream, s, a, trans, fwd, D, C);
        G9_HIP(hipGetLastError());
        // the 128-row diagonal blocks of every D_q, in FP64, into their places in inv(D_q) (zeros right of them)
        G9_TRY(launch_tri_inverse((int)sizeof(R), D, IB, sd, nbI * QB, Di, IB, sd, 0));
    }
    // count products C_z = alpha·A_z·B_z of M × K by K × N, (row stride, batch stride) of each operand given; klim: A
    // is lower triangular and each tile takes only the k range where it is non-zero
    const auto gemm = [&](int M, int N, int K, double alpha, const R *A, ll lda, ll sA, const R *B, ll ldb, ll sB, R *Cp,
                          ll ldc, ll sC, int count, bool klim = false) {
        GemmCall g;
        g.type = type;
        g.tA = g.tB = 0;
        g.M = M; g.N = N; g.K = K;
        g.count = count;
        g.alpha = alpha;
        g.beta = 0.0;
        g.A = A; g.lda = lda; g.sA = sA;
        g.B = B; g.ldb = ldb; g.sB = sB;
        g.C = Cp; g.ldc = ldc; g.sC = sC;
        return klim ? launch_gemm_klim(g, 1) : launch_gemm(g);
    };
    // inv(D_q) by levels, h = 128 .. IB / 2: a sub-block [I1 0; K I2] of 2h rows (every one whole: D_q is padded) has the
    // inverse [inv(I1) 0; −inv(I2)·K·inv(I1) inv(I2)]; two GEMMs batched over all of them form the lower-left quadrants
    for (ll h = SB; h < IB; h *= 2) {
        const int cnt = (int)(nbI * (IB / (2 * h)));
        const ll st = 2 * h * (IB + 1), t2 = h * h;
        if (direct)   // the sub-blocks' lower-left quadrants at A + 2hk·(lda + 1) + h·lda
            G9_TRY(gemm((int)h, (int)h, (int)h, 1.0, Di + h * (IB + 1), IB, st, Ad + h * lda, lda, 2 * h * (lda + 1), Tm,
                        h, t2, cnt));
        else
            G9_TRY(gemm((int)h, (int)h, (int)h, 1.0, Di + h * (IB + 1), IB, st, D + h * IB, IB, st, Tm, h, t2, cnt));
        G9_TRY(gemm((int)h, (int)h, (int)h, -1.0, Tm, h, t2, Di, IB, st, Di + h * IB, IB, st, cnt));
    }
    // E_q = inv(D_q)·C_q, q ≥ 1, each tile over the k range where inv(D_q) is non-zero (256³ × 63 FP32: 27.9 → 24.8 µs)
    if (nbI > 1) {
        if (direct)   // C_q = A[q·IB .., (q − 1)·IB ..]: from A + IB·lda at the stride IB·(lda + 1)
            G9_TRY(gemm(IB, IB, IB, 1.0, Di + sd, IB, sd, Ad + IB * lda, lda, IB * (lda + 1), E + m2, IB, m2, nbI - 1,
                        true));
        else
            G9_TRY(gemm(IB, IB, IB, 1.0, Di + sd, IB, sd, C + m2, IB, m2, E + m2, IB, m2, nbI - 1, true));
    }
    const int per = trans ? UPD_COLS : UPD_ROWS;
    for (int q = 0; q < nbI; q++) {
        const int g0 = q * IB, b = n - g0 < IB ? n - g0 : IB, p = fwd ? g0 : n - g0 - b;
        int pp = 0, pb = 0, o0 = 0, o1 = 0;
        if (q > 0) {   // the previous block (always whole) reaches every row after it in solve order
            pb = IB;
            pp = fwd ? g0 - IB : n - g0;
            o0 = fwd ? p + b : 0;
            o1 = fwd ? n : p;
        }
        const unsigned grid = IB / INV_ROWS<IB> + (o1 > o0 ? blocks(o1 - o0, per) : 0u);
        hipLaunchKernelGGL((inv_step<T, IB>), dim3(grid), dim3(NT), 0, stream, s, a, trans, fwd, pp, pb, p, b, o0, o1,
                           Di + q * sd, E + q * m2, xf, xs);
        G9_HIP(hipGetLastError());
    }
    return 0;
}

// Solves op(A)·z = x in place. `lower`: op(A) is lower triangular (forward substitution); kb: rows below (forward)
// or above (backward) a block that op(A) can reach, n for full and packed storage, the band width for a band.
static int launch_solve(int es, int fmt, const Shape &s, const void *a, int trans, int lower, int kb, void *x, ll ix) {
    return by_type(es, [&](auto *tag) -> int {
        using T = std::remove_pointer_t<decltype(tag)>;
        using R = typename Comp<T>::R;
        const int n = s.nrows, nb = (n + SB - 1) / SB;
        const bool inv = fmt == F_FULL && n >= INV_MIN, big = n >= INV_BIG;
        void *wp, *w2 = nullptr;
        G9_TRY(scratch(SLOT_T, (size_t)n * sizeof(R), &wp));
        if (inv) G9_TRY(scratch(SLOT_X, inv_bytes<R>(n, big ? 512 : 256), &w2));
        R *xf = (R *)wp;
        hipLaunchKernelGGL((to_work<T, R>), dim3(blocks(n, NT)), dim3(NT), 0, stream, n, (const T *)x, ix, xf);
        G9_HIP(hipGetLastError());
        if (inv) {
            G9_TRY((big ? solve_inv<T, 512>(s, (const T *)a, trans, lower, xf, w2)
                        : solve_inv<T, 256>(s, (const T *)a, trans, lower, xf, w2)));
            hipLaunchKernelGGL((from_work<T, R>), dim3(blocks(n, NT)), dim3(NT), 0, stream, n, (const R *)w2, (T *)x, ix);
            G9_HIP(hipGetLastError());
            return 0;
        }
        G9_TRY(by_fmt(fmt, [&](auto fc) -> int {
            constexpr int FMT = decltype(fc)::value;
            const int per = trans ? UPD_COLS : UPD_ROWS;
            for (int q = 0; q < nb; q++) {
                const int p = (lower ? q : nb - 1 - q) * SB, b = n - p < SB ? n - p : SB;
                int pp = 0, pb = 0, t0 = 0, t1 = 0, o0 = 0, o1 = 0;
                if (q > 0) {
                    // rows [r0, r1) reached by the previous block (after it in solve order), split at this block
                    pp = (lower ? q - 1 : nb - q) * SB;
                    pb = n - pp < SB ? n - pp : SB;
                    int r0, r1;
                    if (lower) {
                        r0 = pp + pb;
                        r1 = (ll)pp + pb + kb < n ? pp + pb + kb : n;
                    } else {
                        r0 = pp - kb > 0 ? pp - kb : 0;
                        r1 = pp;
                    }
                    t0 = std::max(r0, p);
                    t1 = std::min(r1, p + b);
                    o0 = lower ? std::max(r0, p + b) : r0;
                    o1 = lower ? r1 : std::min(r1, p);
                }
                const unsigned grid = 1 + (o1 > o0 ? (unsigned)blocks(o1 - o0, per) : 0u);
                hipLaunchKernelGGL((solve_step<T, FMT>), dim3(grid), dim3(NT), 0, stream, s, (const T *)a, trans, lower, pp, pb,
                                   p, b, t0, t1, o0, o1, xf);
                G9_HIP(hipGetLastError());
            }
            return 0;
        }));
        hipLaunchKernelGGL((from_work<T, R>), dim3(blocks(n, NT)), dim3(NT), 0, stream, n, (const R *)xf, (T *)x, ix);
        G9_HIP(hipGetLastError());
        return 0;
    });
}

// ---------------- entry-point helpers ----------------
static int l2_es(int type, int *es) {
    G9_TRY(begin());
    if (type == GEN9BLAS_H || type == GEN9BLAS_HS) *es = 2;
    else if (type == GEN9BLAS_S) *es = 4;
    else if (type == GEN9BLAS_D) *es = 8;
    else G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "type %d unavailable", type);
    return 0;
}
static void vec(Operand &o, const void *p, int n, int inc, int es) {
    o.host = p;
    o.es = es;
    o.rows = 1;
    o.cols = (ll)(n - 1) * (inc < 0 ? -(ll)inc : inc) + 1;
    o.caller_ld = o.cols;
}
static void mat(Operand &o, const void *p, int rows, int cols, int ld, int es) {
    o.host = p;
    o.es = es;
    o.rows = rows;
    o.cols = cols;
    o.caller_ld = ld;
}
static ll voff(int n, int inc) { return inc < 0 ? (ll)(n - 1) * -(ll)inc : 0; }
static ll packed_len(int n) { return (ll)n * (n + 1) / 2; }
static int tri_of(int uplo) { return uplo == GEN9BLAS_UPPER ? TRI_UPPER : TRI_LOWER; }

#define L2_BEGIN(n, bad_inc)                                                          \
    const double t0_ = now_s();                                                       \
    int es;                                                                           \
    G9_TRY(l2_es(type, &es));                                                         \
    if ((n) <= 0) return 0;                                                           \
    if (bad_inc) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "vector increment 0");

// y = alpha·op(A)·x + beta·y with the matrix operand already described in `oa` (resolved here).
static int product_y(double t0, int es, int fmt, Shape s, Operand &oa, bool repitch, int dirs, int skipdiag, double alpha,
                     const void *x, int incx, int nx, double beta, void *y, int incy, int ny) {
    Operand o[3];
    o[0] = oa;
    vec(o[1], x, nx, incx, es);
    vec(o[2], y, ny, incy, es);
    G9_TRY(resolve(o[0], SLOT_A, true, false, repitch));
    G9_TRY(resolve(o[1], SLOT_B, true, false, false));
    G9_TRY(resolve(o[2], SLOT_C, beta != 0.0 || (incy != 1 && incy != -1), true, false));
    s.ld = o[0].ld;
    prof_begin();
    G9_TRY(launch_mv(es, fmt, s, o[0].dev, (const char *)o[1].dev + voff(nx, incx) * es, incx, dirs, skipdiag, alpha, beta,
                     0, (char *)o[2].dev + voff(ny, incy) * es, incy, ny));
    prof_end();
    G9_TRY(finish(o, 3));
    prof_collect(t0);
    return 0;
}

// x = op(A)·x (triangular): the product goes through the partial buffers, so x may be overwritten by the finish.
static int product_x(double t0, int es, int fmt, Shape s, Operand &oa, bool repitch, int trans, void *x, int incx, int n) {
    Operand o[2];
    o[0] = oa;
    vec(o[1], x, n, incx, es);
    G9_TRY(resolve(o[0], SLOT_A, true, false, repitch));
    G9_TRY(resolve(o[1], SLOT_B, true, true, false));
    s.ld = o[0].ld;
    char *xd = (char *)o[1].dev + voff(n, incx) * es;
    prof_begin();
    G9_TRY(launch_mv(es, fmt, s, o[0].dev, xd, incx, trans ? DIR_COL : DIR_ROW, 0, 1.0, 0.0, s.unit, xd, incx, n));
    prof_end();
    G9_TRY(finish(o, 2));
    prof_collect(t0);
    return 0;
}

static int solve_x(double t0, int es, int fmt, Shape s, Operand &oa, bool repitch, int trans, int kb, void *x, int incx,
                   int n) {
    Operand o[2];
    o[0] = oa;
    vec(o[1], x, n, incx, es);
    G9_TRY(resolve(o[0], SLOT_A, true, false, repitch));
    G9_TRY(resolve(o[1], SLOT_B, true, true, false));
    s.ld = o[0].ld;
    const int lower = (s.tri == TRI_LOWER) != (trans != 0);
    prof_begin();
    G9_TRY(launch_solve(es, fmt, s, o[0].dev, trans != 0, lower, kb, (char *)o[1].dev + voff(n, incx) * es, incx));
    prof_end();
    G9_TRY(finish(o, 2));
    prof_collect(t0);
    return 0;
}

static int rank_update(double t0, int es, int fmt, Shape s, Operand &oa, double alpha, const void *x, int incx,
                       const void *y, int incy, int n) {
    const int two = y != nullptr;
    Operand o[3];
    o[0] = oa;
    vec(o[1], x, n, incx, es);
    if (two) vec(o[2], y, n, incy, es);
    G9_TRY(resolve(o[0], SLOT_A, true, true, fmt == F_FULL));
    G9_TRY(resolve(o[1], SLOT_B, true, false, false));
    if (two) G9_TRY(resolve(o[2], SLOT_C, true, false, false));
    s.ld = o[0].ld;
    const char *xd = (const char *)o[1].dev + voff(n, incx) * es;
    const char *yd = two ? (const char *)o[2].dev + voff(n, incy) * es : xd;
    prof_begin();
    G9_TRY(launch_rank(es, fmt, s, alpha, xd, incx, yd, two ? incy : incx, two, o[0].dev));
    prof_end();
    G9_TRY(finish(o, two ? 3 : 2));
    prof_collect(t0);
    return 0;
}

static Shape full_shape(int n, int tri, int unit) {
    Shape s{};
    s.nrows = s.ncols = s.n = n;
    s.tri = tri;
    s.unit = unit;
    return s;
}
static Shape band_shape(int rows, int cols, int KL, int KU, int tri, int unit) {
    Shape s{};
    s.nrows = rows;
    s.ncols = s.n = cols;
    s.KL = KL;
    s.KU = KU;
    s.tri = tri;
    s.unit = unit;
    return s;
}

}  // namespace l2
}  // namespace g9

using namespace g9;
using namespace g9::l2;

extern "C" {

// ---- full storage (reference: lib/src/level12.c:267-370) ----
int gen9blas_symv(int type, int uplo, int n, double alpha, const void *A, int lda, const void *x, int incx, double beta,
                  void *y, int incy) {
    L2_BEGIN(n, !incx || !incy);
    if (lda < n) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "lda < n");
    Operand oa;
    mat(oa, A, n, n, lda, es);
    return product_y(t0_, es, F_FULL, full_shape(n, tri_of(uplo), 0), oa, true, DIR_ROW | DIR_COL, 1, alpha, x, incx, n,
                     beta, y, incy, n);
}

int gen9blas_trmv(int type, int uplo, int trans, int diag, int n, const void *A, int lda, void *x, int incx) {
    L2_BEGIN(n, !incx);
    if (lda < n) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "lda < n");
    Operand oa;
    mat(oa, A, n, n, lda, es);
    return product_x(t0_, es, F_FULL, full_shape(n, tri_of(uplo), diag != 0), oa, true, trans != 0, x, incx, n);
}

int gen9blas_trsv(int type, int uplo, int trans, int diag, int n, const void *A, int lda, void *x, int incx) {
    L2_BEGIN(n, !incx);
    if (lda < n) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "lda < n");
    Operand oa;
    mat(oa, A, n, n, lda, es);
    return solve_x(t0_, es, F_FULL, full_shape(n, tri_of(uplo), diag != 0), oa, true, trans, n, x, incx, n);
}

int gen9blas_syr(int type, int uplo, int n, double alpha, const void *x, int incx, void *A, int lda) {
    L2_BEGIN(n, !incx);
    if (lda < n) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "lda < n");
    Operand oa;
    mat(oa, A, n, n, lda, es);
    return rank_update(t0_, es, F_FULL, full_shape(n, tri_of(uplo), 0), oa, alpha, x, incx, nullptr, 0, n);
}

int gen9blas_syr2(int type, int uplo, int n, double alpha, const void *x, int incx, const void *y, int incy, void *A,
                  int lda) {
    L2_BEGIN(n, !incx || !incy);
    if (lda < n) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "lda < n");
    Operand oa;
    mat(oa, A, n, n, lda, es);
    return rank_update(t0_, es, F_FULL, full_shape(n, tri_of(uplo), 0), oa, alpha, x, incx, y, incy, n);
}

// ---- band and packed storage (reference: lib/src/level12.c:372-519) ----
int gen9blas_gbmv(int type, int trans, int M, int N, int KL, int KU, double alpha, const void *A, int lda, const void *x,
                  int incx, double beta, void *y, int incy) {
    if (KL < 0 || KU < 0 || lda < KL + KU + 1) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "gbmv: KL, KU, lda");
    const int nx = trans ? M : N, ny = trans ? N : M;
    L2_BEGIN(nx < ny ? nx : ny, !incx || !incy);
    Operand oa;
    mat(oa, A, M, KL + KU + 1, lda, es);
    return product_y(t0_, es, F_BAND, band_shape(M, N, KL, KU, TRI_NONE, 0), oa, false, trans ? DIR_COL : DIR_ROW, 0,
                     alpha, x, incx, nx, beta, y, incy, ny);
}

int gen9blas_sbmv(int type, int uplo, int N, int K, double alpha, const void *A, int lda, const void *x, int incx,
                  double beta, void *y, int incy) {
    if (K < 0 || lda < K + 1) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "sbmv: K, lda");
    L2_BEGIN(N, !incx || !incy);
    const int up = uplo == GEN9BLAS_UPPER;
    Operand oa;
    mat(oa, A, N, K + 1, lda, es);
    return product_y(t0_, es, F_BAND, band_shape(N, N, up ? 0 : K, up ? K : 0, tri_of(uplo), 0), oa, false,
                     DIR_ROW | DIR_COL, 1, alpha, x, incx, N, beta, y, incy, N);
}

int gen9blas_tbmv(int type, int uplo, int trans, int diag, int N, int K, const void *A, int lda, void *x, int incx) {
    if (K < 0 || lda < K + 1) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "tbmv: K, lda");
    L2_BEGIN(N, !incx);
    const int up = uplo == GEN9BLAS_UPPER;
    Operand oa;
    mat(oa, A, N, K + 1, lda, es);
    return product_x(t0_, es, F_BAND, band_shape(N, N, up ? 0 : K, up ? K : 0, tri_of(uplo), diag != 0), oa, false,
                     trans != 0, x, incx, N);
}

int gen9blas_tbsv(int type, int uplo, int trans, int diag, int N, int K, const void *A, int lda, void *x, int incx) {
    if (K < 0 || lda < K + 1) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "tbsv: K, lda");
    L2_BEGIN(N, !incx);
    const int up = uplo == GEN9BLAS_UPPER;
    Operand oa;
    mat(oa, A, N, K + 1, lda, es);
    return solve_x(t0_, es, F_BAND, band_shape(N, N, up ? 0 : K, up ? K : 0, tri_of(uplo), diag != 0), oa, false, trans, K,
                   x, incx, N);
}

int gen9blas_spmv(int type, int uplo, int N, double alpha, const void *Ap, const void *x, int incx, double beta, void *y,
                  int incy) {
    L2_BEGIN(N, !incx || !incy);
    Operand oa;
    vec(oa, Ap, (int)0, 1, es);
    oa.cols = packed_len(N);
    oa.caller_ld = oa.cols;
    const int up = uplo == GEN9BLAS_UPPER;
    return product_y(t0_, es, up ? F_PACKU : F_PACKL, full_shape(N, tri_of(uplo), 0), oa, false, DIR_ROW | DIR_COL, 1,
                     alpha, x, incx, N, beta, y, incy, N);
}

int gen9blas_tpmv(int type, int uplo, int trans, int diag, int N, const void *Ap, void *x, int incx) {
    L2_BEGIN(N, !incx);
    Operand oa;
    vec(oa, Ap, (int)0, 1, es);
    oa.cols = packed_len(N);
    oa.caller_ld = oa.cols;
    const int up = uplo == GEN9BLAS_UPPER;
    return product_x(t0_, es, up ? F_PACKU : F_PACKL, full_shape(N, tri_of(uplo), diag != 0), oa, false, trans != 0, x,
                     incx, N);
}

int gen9blas_tpsv(int type, int uplo, int trans, int diag, int N, const void *Ap, void *x, int incx) {
    L2_BEGIN(N, !incx);
    Operand oa;
    vec(oa, Ap, (int)0, 1, es);
    oa.cols = packed_len(N);
    oa.caller_ld = oa.cols;
    const int up = uplo == GEN9BLAS_UPPER;
    return solve_x(t0_, es, up ? F_PACKU : F_PACKL, full_shape(N, tri_of(uplo), diag != 0), oa, false, trans, N, x, incx, N);
}

int gen9blas_spr(int type, int uplo, int N, double alpha, const void *x, int incx, void *Ap) {
    L2_BEGIN(N, !incx);
    Operand oa;
    vec(oa, Ap, (int)0, 1, es);
    oa.cols = packed_len(N);
    oa.caller_ld = oa.cols;
    const int up = uplo == GEN9BLAS_UPPER;
    return rank_update(t0_, es, up ? F_PACKU : F_PACKL, full_shape(N, tri_of(uplo), 0), oa, alpha, x, incx, nullptr, 0, N);
}

int gen9blas_spr2(int type, int uplo, int N, double alpha, const void *x, int incx, const void *y, int incy, void *Ap) {
    L2_BEGIN(N, !incx || !incy);
    Operand oa;
    vec(oa, Ap, (int)0, 1, es);
    oa.cols = packed_len(N);
    oa.caller_ld = oa.cols;
    const int up = uplo == GEN9BLAS_UPPER;
    return rank_update(t0_, es, up ? F_PACKU : F_PACKL, full_shape(N, tri_of(uplo), 0), oa, alpha, x, incx, y, incy, N);
}

}  // extern "C"
