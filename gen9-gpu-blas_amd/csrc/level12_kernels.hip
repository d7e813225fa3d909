// Level 1-2 kernels: HBM-streaming, one pass over the operands, FP16 / FP32 / FP64 storage.
//
// Arithmetic follows the reference's level-1/2 kernels (reference: lib/kernels/level12.cl:1-423): FP16 is computed
// in FP32 (R = float for FP16 and FP32, double for FP64); axpy is fma(a, x, y) (level12.cl:133-139); dot / asum / nrm2
// accumulate in FP64 with one partial per workgroup (level12.cl:189-214; the partials are summed here on the device
// in a fixed order instead of on the host); gemv accumulates in R and writes alpha·sum (+ beta·y, y not read when
// beta = 0) (level12.cl:243-423). Vector element i lives at p[o + i·inc] with o = (n-1)·(-inc) for inc < 0, as in
// BLAS. Contiguous, 16-byte-aligned operands move as 16-byte vectors; strided ones element by element.
#include "internal.h"
#include "wave.h"
#include <type_traits>
#include <stdlib.h>

namespace g9 {
namespace l12 {

typedef _Float16 f16;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef long long ll;

template <class T> struct Comp { using R = float; };
template <> struct Comp<double> { using R = double; };

template <class T> constexpr int VW = 16 / (int)sizeof(T);
template <class T> union Vec {
    u32x4 u;
    T e[VW<T>];
};
template <class T> __device__ __forceinline__ Vec<T> vload(const T *p) {
    Vec<T> v;
    v.u = *reinterpret_cast<const u32x4 *>(p);
    return v;
}
// Streamed operands are read once: nontemporal loads keep them from displacing reusable lines in L2 and MALL (about
// +10 % HBM rate on gfx950 for a single pass). Stores stay ordinary, nontemporal stores measured slower.
template <class T> __device__ __forceinline__ Vec<T> vload_nt(const T *p) {
    Vec<T> v;
    v.u = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return v;
}
template <class T> __device__ __forceinline__ void vstore(T *p, const Vec<T> &v) { *reinterpret_cast<u32x4 *>(p) = v.u; }
__device__ __forceinline__ float fma_r(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double fma_r(double a, double b, double c) { return __builtin_fma(a, b, c); }

constexpr int NT = 256;
// Grid of a streaming kernel: one 16-byte chunk per thread and grid-stride step, at most `per_cu` blocks per CU
// (4 for kernels with two input streams, 8 for a single read stream: the best HBM rate in a sweep on gfx950).
static unsigned stream_grid(ll chunks, int per_cu = 4) {
    ll g = (chunks + NT - 1) / NT;
    const ll cap = (ll)(num_cus > 0 ? num_cus : 256) * per_cu;
    return (unsigned)(g < 1 ? 1 : g > cap ? cap : g);
}

// ---------------- elementwise: axpy / scal / copy / rot ----------------
// op 0 axpy: y = fma(a, x, y); 1 scal: x = a·x; 2 copy: y = x; 3 rot: x' = h11·x + h12·y, y' = h21·x + h22·y;
// 4 swap.
template <class T, int OP>
__global__ void __launch_bounds__(NT) elem_kernel(int n, typename Comp<T>::R h11, typename Comp<T>::R h12,
                                                  typename Comp<T>::R h21, typename Comp<T>::R h22, T *x, ll ix, T *y,
                                                  ll iy, int vec) {
    using R = typename Comp<T>::R;
    constexpr int V = VW<T>;
    const ll stride = (ll)gridDim.x * NT;
    auto one = [&](T &xe, T &ye) {
        if constexpr (OP == 0) ye = (T)fma_r(h11, (R)xe, (R)ye);
        else if constexpr (OP == 1) xe = (T)(h11 * (R)xe);
        else if constexpr (OP == 2) ye = xe;
        else if constexpr (OP == 3) {
            const R a = (R)xe, b = (R)ye;
            xe = (T)fma_r(h11, a, h12 * b);
            ye = (T)fma_r(h21, a, h22 * b);
        } else {
            const T t = xe;
            xe = ye;
            ye = t;
        }
    };
    if (vec) {
        const ll nv = n / V;
        for (ll c = (ll)blockIdx.x * NT + threadIdx.x; c < nv; c += stride) {
            Vec<T> xv, yv;
            xv = vload_nt(x + c * V);
            if constexpr (OP == 0 || OP >= 3) yv = vload_nt(y + c * V);
#pragma unroll
            for (int e = 0; e < V; e++) one(xv.e[e], yv.e[e]);
            if constexpr (OP == 1 || OP >= 3) vstore(x + c * V, xv);
            if constexpr (OP == 0 || OP == 2 || OP >= 3) vstore(y + c * V, yv);
        }
        for (ll i = nv * V + (ll)blockIdx.x * NT + threadIdx.x; i < n; i += stride) {
            T dummy = T(0);
            one(x[i], OP == 1 ? dummy : y[i]);
        }
        return;
    }
    for (ll i = (ll)blockIdx.x * NT + threadIdx.x; i < n; i += stride) {
        T dummy = T(0);
        one(x[i * ix], OP == 1 ? dummy : y[i * iy]);
    }
}

// ---------------- reductions (FP64) ----------------
__device__ __forceinline__ double wave_sum(double s) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) s += __shfl_xor(s, d);
    return s;
}
__device__ __forceinline__ double block_sum(double s) {
    __shared__ double ws[NT / 64];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = s;
    __syncthreads();
    double t = 0;
    if (threadIdx.x == 0)
#pragma unroll
        for (int w = 0; w < NT / 64; w++) t += ws[w];
    return t;   // valid in thread 0
}

// Two kernels: every block writes its FP64 partial, then reduce_final adds the partials in index order, so the
// result does not depend on block scheduling. (Finishing in the last block instead needs a device-scope fence per
// block, which writes back and invalidates the L2 of the XCD: about 35 % of the HBM rate at 1 GiB on gfx950.)
template <class T, int MODE>
__global__ void __launch_bounds__(NT) reduce_kernel(int n, const T *x, ll ix, const T *y, ll iy, int vec, double *part) {
    constexpr int V = VW<T>;
    const ll stride = (ll)gridDim.x * NT;
    double s0 = 0, s1 = 0;   // two chains: FP64 fma latency does not serialize the stream
    auto acc = [&](double &s, double a, double b) {
        if constexpr (MODE == 0) s = __builtin_fma(a, b, s);
        else if constexpr (MODE == 1) s += __builtin_fabs(a);
        else s = __builtin_fma(a, a, s);
    };
    ll tail = 0;
    if (vec) {
        // Each step a block reads U·NT consecutive chunks (16 KiB for FP32 asum) with every load issued before the
        // first add: 4 loads of 16 bytes in flight per lane (dot: 2 of x and 2 of y), and the blocks in flight cover
        // one contiguous span of memory.
        constexpr int U = MODE == 0 ? 2 : 4;
        const ll nv = n / V, big = (ll)U * NT, nsc = nv / big;
        for (ll sc = blockIdx.x; sc < nsc; sc += gridDim.x) {
            const ll c0 = sc * big + threadIdx.x;
            Vec<T> xv[U], yv[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                xv[u] = vload_nt(x + (c0 + u * NT) * V);
                if constexpr (MODE == 0) yv[u] = vload_nt(y + (c0 + u * NT) * V);
            }
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int e = 0; e < V; e++)
                    acc(e & 1 ? s1 : s0, (double)xv[u].e[e], MODE == 0 ? (double)yv[u].e[e] : 0.0);
        }
        ll c = nsc * big + (ll)blockIdx.x * NT + threadIdx.x;   // the chunks past the last whole super-chunk
        for (; c < nv; c += stride) {
            const Vec<T> xv = vload_nt(x + c * V);
            Vec<T> yv;
            if constexpr (MODE == 0) yv = vload_nt(y + c * V);
#pragma unroll
            for (int e = 0; e < V; e++) acc(e & 1 ? s1 : s0, (double)xv.e[e], MODE == 0 ? (double)yv.e[e] : 0.0);
        }
        tail = nv * V;
        ix = 1;
        iy = 1;
    }
    for (ll i = tail + (ll)blockIdx.x * NT + threadIdx.x; i < n; i += stride)
        acc(s0, (double)x[i * ix], MODE == 0 ? (double)y[i * iy] : 0.0);
    const double t = block_sum(s0 + s1);
    if (threadIdx.x == 0) part[blockIdx.x] = t;
}

// Sum of np ≤ FIN·NT partials (more are handled by the plain loop): all loads are issued before the first add, so
// the kernel costs about one memory latency.
constexpr int FIN = 8;
__global__ void __launch_bounds__(NT) reduce_final(int np, const double *part, int mode, double *out) {
    double v[FIN];
#pragma unroll
    for (int j = 0; j < FIN; j++) {
        const int i = threadIdx.x + j * NT;
        v[j] = i < np ? part[i] : 0.0;
    }
    double s = 0;
#pragma unroll
    for (int j = 0; j < FIN; j++) s += v[j];
    for (int i = threadIdx.x + FIN * NT; i < np; i += NT) s += part[i];
    const double t = block_sum(s);
    if (threadIdx.x == 0) *out = mode == 2 ? __builtin_sqrt(t) : t;
}

// ---------------- iamax: first index of the largest |x|; NaN skipped, all NaN (or n = 0 in a part) → index 0 ----------------
struct ValIdx {
    double v;
    long long i;
};
__device__ __forceinline__ ValIdx better(ValIdx a, ValIdx b) {
    return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a;
}
__device__ __forceinline__ ValIdx block_best(ValIdx b) {
    __shared__ double sv[NT];
    __shared__ long long si[NT];
    sv[threadIdx.x] = b.v;
    si[threadIdx.x] = b.i;
    __syncthreads();
    for (int d = NT / 2; d >= 1; d >>= 1) {
        if ((int)threadIdx.x < d) {
            const ValIdx o = better(ValIdx{sv[threadIdx.x], si[threadIdx.x]}, ValIdx{sv[threadIdx.x + d], si[threadIdx.x + d]});
            sv[threadIdx.x] = o.v;
            si[threadIdx.x] = o.i;
        }
        __syncthreads();
    }
    return ValIdx{sv[0], si[0]};
}
template <class T>
__global__ void __launch_bounds__(NT) iamax_kernel(int n, const T *x, ll ix, double *pv, long long *pi) {
    ValIdx b{-1.0, 0x7fffffffffffffffLL};
    for (ll i = (ll)blockIdx.x * NT + threadIdx.x; i < n; i += (ll)gridDim.x * NT) {
        const double a = __builtin_fabs((double)x[i * ix]);
        if (a == a) b = better(b, ValIdx{a, i});   // a != a: NaN, skipped
    }
    b = block_best(b);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = b.v;
        pi[blockIdx.x] = b.i;
    }
}
__global__ void __launch_bounds__(NT) iamax_final(int np, const double *pv, const long long *pi, long long *out) {
    ValIdx b{-1.0, 0x7fffffffffffffffLL};
    for (int i = threadIdx.x; i < np; i += NT) b = better(b, ValIdx{pv[i], pi[i]});
    b = block_best(b);
    if (threadIdx.x == 0) *out = b.i == 0x7fffffffffffffffLL ? 0 : b.i;
}

// ---------------- GEMV no-trans: y = alpha·A·x + beta·y ----------------
// A wave owns RWN consecutive rows; its lanes stream 16 bytes of each row per step (1 KiB per row per wave-step) and
// reuse each x chunk for the RWN rows. The RWN sums are reduced across the wave by the transposing butterfly.
constexpr int RWN = 4;
template <class T, bool VEC>
__global__ void __launch_bounds__(NT) gemv_n_kernel(int M, int N, typename Comp<T>::R alpha, const T *A, ll lda, const T *x,
                                                    ll ix, typename Comp<T>::R beta, T *y, ll iy) {
    using R = typename Comp<T>::R;
    constexpr int V = VW<T>;
    const int lane = threadIdx.x & 63;
    const int r0 = (blockIdx.x * (NT / 64) + (threadIdx.x >> 6)) * RWN;
    if (r0 >= M) return;
    const T *ar[RWN];
#pragma unroll
    for (int r = 0; r < RWN; r++) ar[r] = A + (ll)min(r0 + r, M - 1) * lda;
    R s[RWN];
#pragma unroll
    for (int r = 0; r < RWN; r++) s[r] = 0;
    int j = lane * V;
    if (VEC) {
        const int nvec = N - N % V;
        // U steps per batch: all U·RWN loads of A (nontemporal: A is read once) are issued before the first product
        constexpr int U = 4;
        for (; j + (U - 1) * 64 * V < nvec; j += U * 64 * V) {
            Vec<T> xv[U], av[U][RWN];
#pragma unroll
            for (int u = 0; u < U; u++) {
                xv[u] = vload(x + j + u * 64 * V);
#pragma unroll
                for (int r = 0; r < RWN; r++) av[u][r] = vload_nt(ar[r] + j + u * 64 * V);
            }
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int r = 0; r < RWN; r++)
#pragma unroll
                    for (int e = 0; e < V; e++) s[r] = fma_r((R)av[u][r].e[e], (R)xv[u].e[e], s[r]);
        }
        for (; j < nvec; j += 64 * V) {
            const Vec<T> xv = vload(x + j);
#pragma unroll
            for (int r = 0; r < RWN; r++) {
                const Vec<T> av = vload_nt(ar[r] + j);
#pragma unroll
                for (int e = 0; e < V; e++) s[r] = fma_r((R)av.e[e], (R)xv.e[e], s[r]);
            }
        }
        for (int jt = nvec + lane; jt < N; jt += 64)
#pragma unroll
            for (int r = 0; r < RWN; r++) s[r] = fma_r((R)ar[r][jt], (R)x[jt], s[r]);
    } else {
        for (int jt = lane; jt < N; jt += 64) {
            const R xj = (R)x[(ll)jt * ix];
#pragma unroll
            for (int r = 0; r < RWN; r++) s[r] = fma_r((R)ar[r][jt], xj, s[r]);
        }
    }
    // butterfly over the RWN row sums: two halving exchanges, then plain sums
    int base = 0;
    butterfly<0, RWN>(s, lane, base);
    if ((lane & (64 / RWN - 1)) == 0) {
        const int row = r0 + base;
        if (row < M) {
            T *yp = y + (ll)row * iy;
            *yp = (T)(beta == R(0) ? alpha * s[0] : fma_r(alpha, s[0], beta * (R)*yp));
        }
    }
}

// ---------------- GEMV trans: y = alpha·Aᵀ·x + beta·y ----------------
// Stage 1: a thread owns V consecutive columns (16 bytes) and a band of rpp rows, partial sums to P[part][col].
// Stage 2: y[col] = alpha·Σ_part P[part][col] + beta·y[col] in a fixed order. With one part stage 1 writes y.
template <class T, bool VEC>
__global__ void __launch_bounds__(NT) gemv_t1_kernel(int M, int N, int rpp, const T *A, ll lda, const T *x, ll ix,
                                                     typename Comp<T>::R *P, int direct, typename Comp<T>::R alpha,
                                                     typename Comp<T>::R beta, T *y, ll iy) {
    using R = typename Comp<T>::R;
    constexpr int V = VW<T>;
    const int c0 = (blockIdx.x * NT + threadIdx.x) * V;
    if (c0 >= N) return;
    const int part = blockIdx.y, i0 = part * rpp, i1 = min(M, i0 + rpp);
    R s[V];
#pragma unroll
    for (int e = 0; e < V; e++) s[e] = 0;
    const bool full = VEC && c0 + V <= N;
    if (full) {
        // U rows per step: their loads (nontemporal: A is read once) are all issued before the first product
        constexpr int U = 8;
        int i = i0;
        for (; i + U <= i1; i += U) {
            Vec<T> av[U];
            R xv[U];
#pragma unroll
            for (int u = 0; u < U; u++) av[u] = vload_nt(A + (ll)(i + u) * lda + c0);
#pragma unroll
            for (int u = 0; u < U; u++) xv[u] = (R)x[(ll)(i + u) * ix];
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int e = 0; e < V; e++) s[e] = fma_r((R)av[u].e[e], xv[u], s[e]);
        }
        for (; i < i1; i++) {
            const R xv = (R)x[(ll)i * ix];
            const Vec<T> av = vload_nt(A + (ll)i * lda + c0);
#pragma unroll
            for (int e = 0; e < V; e++) s[e] = fma_r((R)av.e[e], xv, s[e]);
        }
    } else {
        for (int i = i0; i < i1; i++) {
            const R xv = (R)x[(ll)i * ix];
#pragma unroll
            for (int e = 0; e < V; e++)
                if (c0 + e < N) s[e] = fma_r((R)A[(ll)i * lda + c0 + e], xv, s[e]);
        }
    }
#pragma unroll
    for (int e = 0; e < V; e++) {
        if (c0 + e >= N) break;
        if (direct) {
            T *yp = y + (ll)(c0 + e) * iy;
            *yp = (T)(beta == R(0) ? alpha * s[e] : fma_r(alpha, s[e], beta * (R)*yp));
        } else {
            P[(ll)part * N + c0 + e] = s[e];
        }
    }
}
template <class T>
__global__ void __launch_bounds__(NT) gemv_t2_kernel(int N, int parts, const typename Comp<T>::R *P,
                                                     typename Comp<T>::R alpha, typename Comp<T>::R beta, T *y, ll iy) {
    // 64 columns per block; the block's 4 waves each sum every 4th part (loads issued 8 at a time, added in part
    // order), then wave 0 adds the 4 sums in wave order: a fixed summation order for every column.
    using R = typename Comp<T>::R;
    constexpr int G = NT / 64;
    const int j = blockIdx.x * 64 + (threadIdx.x & 63), gq = threadIdx.x >> 6;
    R t = 0;
    if (j < N) {
        int r = gq;
        for (; r + 7 * G < parts; r += 8 * G) {
            R v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = P[(ll)(r + u * G) * N + j];
#pragma unroll
            for (int u = 0; u < 8; u++) t += v[u];
        }
        for (; r < parts; r += G) t += P[(ll)r * N + j];
    }
    __shared__ R red[G][64];
    red[gq][threadIdx.x & 63] = t;
    __syncthreads();
    if (gq == 0 && j < N) {
        R sum = red[0][threadIdx.x];
#pragma unroll
        for (int q = 1; q < G; q++) sum += red[q][threadIdx.x];
        T *yp = y + (ll)j * iy;
        *yp = (T)(beta == R(0) ? alpha * sum : fma_r(alpha, sum, beta * (R)*yp));
    }
}

// ---------------- GER: A = alpha·x·yᵀ + A ----------------
template <class T>
__global__ void __launch_bounds__(NT) ger_kernel(int M, int N, typename Comp<T>::R alpha, const T *x, ll ix, const T *y,
                                                 ll iy, T *A, ll lda) {
    using R = typename Comp<T>::R;
    const int i = blockIdx.y;
    const R ax = alpha * (R)x[(ll)i * ix];
    for (int j = blockIdx.x * NT + threadIdx.x; j < N; j += gridDim.x * NT) {
        T *a = A + (ll)i * lda + j;
        *a = (T)fma_r(ax, (R)y[(ll)j * iy], (R)*a);
    }
}

}  // namespace l12

using namespace l12;

// ---------------- launchers ----------------
template <class F> static int by_type(int es, F f) {
    if (es == 2) return f((f16 *)nullptr);
    if (es == 4) return f((float *)nullptr);
    return f((double *)nullptr);
}
static bool al16(const void *p) { return (uintptr_t)p % 16 == 0; }

template <int OP>
static int elem(int es, int n, double h11, double h12, double h21, double h22, void *x, ll ox, ll ix, void *y, ll oy, ll iy) {
    return by_type(es, [&](auto *tag) -> int {
        using T = std::remove_pointer_t<decltype(tag)>;
        using R = typename Comp<T>::R;
        T *xp = (T *)x + ox, *yp = y ? (T *)y + oy : nullptr;
        const bool vec = ix == 1 && (OP == 1 || iy == 1) && al16(xp) && (OP == 1 || al16(yp));
        const unsigned g = stream_grid(vec ? (n + VW<T> - 1) / VW<T> : n);
        hipLaunchKernelGGL((elem_kernel<T, OP>), dim3(g), dim3(NT), 0, stream, n, (R)h11, (R)h12, (R)h21, (R)h22, xp, ix,
                           yp, iy, (int)vec);
        G9_HIP(hipGetLastError());
        return 0;
    });
}

int launch_axpy(int es, int n, double a, const void *x, ll ox, ll ix, void *y, ll oy, ll iy) {
    return elem<0>(es, n, a, 0, 0, 0, const_cast<void *>(x), ox, ix, y, oy, iy);
}
int launch_scal(int es, int n, double a, void *x, ll ox, ll ix) { return elem<1>(es, n, a, 0, 0, 0, x, ox, ix, nullptr, 0, 1); }
int launch_copy(int es, int n, const void *x, ll ox, ll ix, void *y, ll oy, ll iy) {
    return elem<2>(es, n, 0, 0, 0, 0, const_cast<void *>(x), ox, ix, y, oy, iy);
}
int launch_rot(int es, int n, void *x, ll ox, ll ix, void *y, ll oy, ll iy, double h11, double h12, double h21, double h22,
               int swap) {
    if (swap) return elem<4>(es, n, 0, 0, 0, 0, x, ox, ix, y, oy, iy);
    return elem<3>(es, n, h11, h12, h21, h22, x, ox, ix, y, oy, iy);
}

int launch_reduce(int es, int mode, int n, const void *x, ll ox, ll ix, const void *y, ll oy, ll iy, double *result) {
    return by_type(es, [&](auto *tag) -> int {
        using T = std::remove_pointer_t<decltype(tag)>;
        const T *xp = (const T *)x + ox, *yp = y ? (const T *)y + oy : xp;
        const bool vec = ix == 1 && (mode != 0 || iy == 1) && al16(xp) && (mode != 0 || al16(yp));
        const unsigned g = stream_grid(vec ? (n + VW<T> - 1) / VW<T> : n, mode == 0 ? 4 : 8);
        void *pp;
        G9_TRY(scratch(SLOT_P, g * sizeof(double), &pp));
        double *part = (double *)pp;
        if (mode == 0) hipLaunchKernelGGL((reduce_kernel<T, 0>), dim3(g), dim3(NT), 0, stream, n, xp, ix, yp, iy, (int)vec, part);
        else if (mode == 1) hipLaunchKernelGGL((reduce_kernel<T, 1>), dim3(g), dim3(NT), 0, stream, n, xp, ix, yp, iy, (int)vec, part);
        else hipLaunchKernelGGL((reduce_kernel<T, 2>), dim3(g), dim3(NT), 0, stream, n, xp, ix, yp, iy, (int)vec, part);
        G9_HIP(hipGetLastError());
        hipLaunchKernelGGL(reduce_final, dim3(1), dim3(NT), 0, stream, (int)g, (const double *)part, mode, result);
        G9_HIP(hipGetLastError());
        return 0;
    });
}

int launch_iamax(int es, int n, const void *x, ll ox, ll ix, long long *result) {
    return by_type(es, [&](auto *tag) -> int {
        using T = std::remove_pointer_t<decltype(tag)>;
        const T *xp = (const T *)x + ox;
        const unsigned g = stream_grid(n);
        void *pp;
        G9_TRY(scratch(SLOT_P, g * (sizeof(double) + sizeof(long long)), &pp));
        double *pv = (double *)pp;
        long long *pi = (long long *)(pv + g);
        hipLaunchKernelGGL((iamax_kernel<T>), dim3(g), dim3(NT), 0, stream, n, xp, ix, pv, pi);
        G9_HIP(hipGetLastError());
        hipLaunchKernelGGL(iamax_final, dim3(1), dim3(NT), 0, stream, (int)g, (const double *)pv, (const long long *)pi,
                           result);
        G9_HIP(hipGetLastError());
        return 0;
    });
}

int launch_gemv(int es, int trans, int M, int N, double alpha, const void *A, ll lda, const void *x, ll ox, ll ix,
                double beta, void *y, ll oy, ll iy) {
    return by_type(es, [&](auto *tag) -> int {
        using T = std::remove_pointer_t<decltype(tag)>;
        using R = typename Comp<T>::R;
        const T *Ap = (const T *)A, *xp = (const T *)x + ox;
        T *yp = (T *)y + oy;
        const bool avec = al16(Ap) && (lda * (ll)sizeof(T)) % 16 == 0;
        if (!trans) {
            const bool vec = avec && ix == 1 && al16(xp);
            const unsigned g = (unsigned)((M + RWN * (NT / 64) - 1) / (RWN * (NT / 64)));
            if (vec) hipLaunchKernelGGL((gemv_n_kernel<T, true>), dim3(g), dim3(NT), 0, stream, M, N, (R)alpha, Ap, lda, xp, ix, (R)beta, yp, iy);
            else hipLaunchKernelGGL((gemv_n_kernel<T, false>), dim3(g), dim3(NT), 0, stream, M, N, (R)alpha, Ap, lda, xp, ix, (R)beta, yp, iy);
            G9_HIP(hipGetLastError());
            return 0;
        }
        constexpr int V = VW<T>;
        const int cblocks = (N + NT * V - 1) / (NT * V);
        // about 3 blocks per CU, each summing a band of rows into FP32 (FP64) partials: the best HBM rate in a sweep of
        // 256-8192 blocks at 16384² (fewer, longer bands keep more loads in flight per thread)
        const int tgt = 3 * (num_cus > 0 ? num_cus : 256);
        int parts = (tgt + cblocks - 1) / cblocks;
        const int maxparts = (M + 15) / 16;
        if (parts > maxparts) parts = maxparts;
        if (parts < 1) parts = 1;
        const int rpp = (M + parts - 1) / parts;
        parts = (M + rpp - 1) / rpp;
        R *P = nullptr;
        if (parts > 1) {
            void *pp;
            G9_TRY(scratch(SLOT_P, (size_t)parts * N * sizeof(R), &pp));
            P = (R *)pp;
        }
        const dim3 grid((unsigned)cblocks, (unsigned)parts);
        if (avec) hipLaunchKernelGGL((gemv_t1_kernel<T, true>), grid, dim3(NT), 0, stream, M, N, rpp, Ap, lda, xp, ix, P, (int)(parts == 1), (R)alpha, (R)beta, yp, iy);
        else hipLaunchKernelGGL((gemv_t1_kernel<T, false>), grid, dim3(NT), 0, stream, M, N, rpp, Ap, lda, xp, ix, P, (int)(parts == 1), (R)alpha, (R)beta, yp, iy);
        G9_HIP(hipGetLastError());
        if (parts > 1) {
            hipLaunchKernelGGL((gemv_t2_kernel<T>), dim3((unsigned)((N + 63) / 64)), dim3(NT), 0, stream, N, parts,
                               (const R *)P, (R)alpha, (R)beta, yp, iy);
            G9_HIP(hipGetLastError());
        }
        return 0;
    });
}

int launch_ger(int es, int M, int N, double alpha, const void *x, ll ox, ll ix, const void *y, ll oy, ll iy, void *A, ll lda) {
    return by_type(es, [&](auto *tag) -> int {
        using T = std::remove_pointer_t<decltype(tag)>;
        using R = typename Comp<T>::R;
        if (M > 65535) G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "ger: M = %d > 65535", M);
        const unsigned gx = (unsigned)((N + NT - 1) / NT < 64 ? (N + NT - 1) / NT : 64);
        hipLaunchKernelGGL((ger_kernel<T>), dim3(gx, (unsigned)M), dim3(NT), 0, stream, M, N, (R)alpha, (const T *)x + ox, ix,
                           (const T *)y + oy, iy, (T *)A, lda);
        G9_HIP(hipGetLastError());
        return 0;
    });
}

}  // namespace g9
