// Skinny GEMM kernel template: C (M×N) = alpha·a·wᵀ + beta·C for M ≤ 16, a (M×K) and w (N×K) both K-contiguous.
//
// Semantics follow the reference's skinny kernels (reference: lib/kernels/level12.cl:640-801, skinny_k* / skinny_r*):
// FP32 accumulation of the products of the FP16 (or FP32) inputs, then alpha·sum (+ beta·C, C not read when
// beta = 0), rounded once to the element type. The MI355X design streams the weights once from HBM:
// - a workgroup of KS waves owns RW consecutive weight rows and one tile of MT rows of a; its waves split K, each
//   lane loading 16 bytes of every weight row per step (a wave reads 1 KiB contiguous per row per step), with the
//   small operand a re-read from L1/L2;
// - FP16 products are accumulated with v_dot2_f32_f16 (two products and an FP32 add per instruction, exact
//   products), FP32 with fma; no matrix cores;
// - the RW·MT partial sums of a lane are reduced across the 64 lanes by a transposing butterfly: at each exchange
//   distance the lane keeps half of its values and adds its partner's copy of them, so 64 sums cost about one
//   exchange per value instead of six; then the KS waves combine through LDS.
#pragma once
#include "internal.h"
#include "wave.h"

namespace g9 {
namespace sk {

typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct Params {
    const void *a, *w;
    void *C;
    long long sam, swn, scm, scn;
    int M, N, K;
    float alpha, beta;
};

// Vector elements are copied to scalars before __builtin_bit_cast: hipcc (ROCm 7.2) evaluates
// __builtin_bit_cast(T, v[i]) of an ext_vector element as element 0 for every i.
template <class T> __device__ __forceinline__ float dot16(u32x4 w, u32x4 a, float acc);
template <> __device__ __forceinline__ float dot16<f16>(u32x4 w, u32x4 a, float acc) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const unsigned wi = w[i], ai = a[i];
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, wi), __builtin_bit_cast(f16x2, ai), acc, false);
    }
    return acc;
}
template <> __device__ __forceinline__ float dot16<float>(u32x4 w, u32x4 a, float acc) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const unsigned wi = w[i], ai = a[i];
        acc = __builtin_fmaf(__builtin_bit_cast(float, wi), __builtin_bit_cast(float, ai), acc);
    }
    return acc;
}

// NTL: nontemporal load, for the weights (read once per call, they should not evict the small operand from L2).
template <class T, bool VEC, bool NTL = false> __device__ __forceinline__ u32x4 ld16(const T *p) {
    if constexpr (VEC && NTL) return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    if constexpr (VEC) return *reinterpret_cast<const u32x4 *>(p);
    constexpr int V = 16 / sizeof(T);
    union { u32x4 v; T e[V]; } u;
#pragma unroll
    for (int e = 0; e < V; e++) u.e[e] = p[e];
    return u.v;
}

template <class T, int MT, int RW, int KS, int NC, bool VEC>
__global__ void __launch_bounds__(KS * 64) skinny_kernel(Params p) {
    constexpr int V = 16 / (int)sizeof(T);
    constexpr int NV = RW * MT;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int n0 = blockIdx.x * RW, m0 = blockIdx.y * MT;
    const T *a = reinterpret_cast<const T *>(p.a), *w = reinterpret_cast<const T *>(p.w);
    // rows past the end are computed from a copy of the last valid row and never stored
    const T *wr[RW], *ar[MT];
#pragma unroll
    for (int r = 0; r < RW; r++) wr[r] = w + (long long)min(n0 + r, p.N - 1) * p.swn;
#pragma unroll
    for (int m = 0; m < MT; m++) ar[m] = a + (long long)min(m0 + m, p.M - 1) * p.sam;

    float v[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) v[i] = 0.f;

    // Super-steps of NC chunks per lane: every weight load of a super-step is issued before its first product, so
    // a wave keeps NC·RW 16-byte loads per lane in flight. Chunk j of lane l in wave wv covers
    // k = k0 + ((j·KS + wv)·64 + l)·V .. +V-1 (a wave reads 1 KiB contiguous per row and chunk).
    const int K = p.K, kvec = K - K % V;
    constexpr int SUPER = NC * KS * 64 * V;
    const u32x4 zero = {0, 0, 0, 0};
    for (int k0 = 0; k0 < kvec; k0 += SUPER) {
        u32x4 wq[NC][RW];
#pragma unroll
        for (int j = 0; j < NC; j++) {
            const int k = k0 + ((j * KS + wv) * 64 + lane) * V;
#pragma unroll
            for (int r = 0; r < RW; r++) wq[j][r] = k < kvec ? ld16<T, VEC, true>(wr[r] + k) : zero;
        }
#pragma unroll
        for (int j = 0; j < NC; j++) {
            const int k = k0 + ((j * KS + wv) * 64 + lane) * V;
            u32x4 aq[MT];
#pragma unroll
            for (int m = 0; m < MT; m++) aq[m] = k < kvec ? ld16<T, VEC>(ar[m] + k) : zero;
#pragma unroll
            for (int r = 0; r < RW; r++)
#pragma unroll
                for (int m = 0; m < MT; m++) v[r * MT + m] = dot16<T>(wq[j][r], aq[m], v[r * MT + m]);
        }
    }
    // K tail (K % V elements): one element per lane
    for (int kt = kvec + wv * 64 + lane; kt < K; kt += KS * 64) {
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const float x = (float)wr[r][kt];
#pragma unroll
            for (int m = 0; m < MT; m++) v[r * MT + m] = __builtin_fmaf(x, (float)ar[m][kt], v[r * MT + m]);
        }
    }

    // transposing butterfly across the wave
    int base = 0;
    butterfly<0, NV>(v, lane, base);
    constexpr int NF = Butterfly<NV>::per_lane;
    const bool writer = (lane & (Butterfly<NV>::dup - 1)) == 0;

    T *C = reinterpret_cast<T *>(p.C);
    auto emit = [&](int idx, float s) {
        const int n = n0 + idx / MT, m = m0 + idx % MT;
        if (n < p.N && m < p.M) {
            T *c = C + (long long)m * p.scm + (long long)n * p.scn;
            const float r = p.beta == 0.f ? p.alpha * s : __builtin_fmaf(p.alpha, s, p.beta * (float)*c);
            *c = (T)r;
        }
    };
    if constexpr (KS == 1) {
        if (writer)
#pragma unroll
            for (int i = 0; i < NF; i++) emit(base + i, v[i]);
    } else {
        __shared__ float part[KS][NV];
        if (writer)
#pragma unroll
            for (int i = 0; i < NF; i++) part[wv][base + i] = v[i];
        __syncthreads();
        for (int t = threadIdx.x; t < NV; t += KS * 64) {
            float s = 0.f;
#pragma unroll
            for (int q = 0; q < KS; q++) s += part[q][t];
            emit(t, s);
        }
    }
}

}  // namespace sk
}  // namespace g9
