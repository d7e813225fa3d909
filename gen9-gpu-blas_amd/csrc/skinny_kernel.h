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
#include "lds_dma.h"
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

// FP16 skinny kernel on the matrix cores, for 4 < M ≤ 16 (and M tiles beyond). The dot-product kernel above is
// issue-bound there: it needs 4·M v_dot2 instructions per 16 bytes of w. Here one v_mfma_f32_16x16x32_f16 multiplies
// 16 rows of w by 16 rows of a (rows of a beyond M are zero) over 32 k, so the instruction count no longer grows
// with M and the kernel stays bound by the weight stream:
// - a workgroup owns 16 rows of w (n0 .. n0+15) and one tile of MT rows of a; its KS waves split K in groups of
//   GK = 256 k, round robin (wave wv takes groups wv, wv + KS, ...);
// - each wave streams its groups through a private NS-stage LDS ring with global_load_lds_dwordx4: per group, 8
//   copies of 1 KiB bring 16 rows × 512 bytes of w (one copy = 2 rows, contiguous in memory), and ⌈MT/2⌉ copies
//   bring the MT rows of a. No barrier is needed until the end: a wave only reads what it loaded itself;
// - chunk c (16 bytes, k = 8c .. 8c+7) of row r of a group sits at position c ^ r of the row, so the 16 lanes that
//   read one chunk of 16 different rows hit distinct banks;
// - the 16×16 FP32 partial tiles of the KS waves are summed through LDS, then alpha (and beta·C, C not read when
//   beta = 0) is applied and rounded once to FP16, as in the dot-product kernel.
// Requires K % 256 == 0 and 16-byte aligned rows of a and w (the launcher checks; other shapes take the kernel above).
template <int MT, int KS, int NS>
__global__ void __launch_bounds__(KS * 64) skinny_mfma_kernel(Params p) {
    typedef f16 f16x8 __attribute__((ext_vector_type(8)));
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    constexpr int GK = 256, ROWB = GK * 2;                 // 512 bytes of a row per group
    constexpr int NA = (MT + 1) / 2;                       // copies of a per group (2 rows each)
    constexpr int WB = 16 * ROWB, AB = NA * 1024, SB = WB + AB;
    constexpr int LPG = 8 + NA;                            // copies per group
    static_assert((NS - 1) * LPG < 64, "copies in flight must fit vmcnt");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[KS * NS * SB];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const int n0 = blockIdx.x * 16, m0 = blockIdx.y * MT;
    const unsigned lbase = (unsigned)(uintptr_t)smem + wv * NS * SB;
    const G9_LDS unsigned char *lds = (const G9_LDS unsigned char *)smem + wv * NS * SB;
    const int G = p.K / GK;
    const int ng = G > wv ? (G - wv + KS - 1) / KS : 0;

    // copy i of w covers rows 2i, 2i+1 of the group; lane L: row 2i + L/32, position L % 32 = chunk (L % 32) ^ row.
    // Rows past N (and of a past M) load the last valid row; their results are never stored (a: zeroed below).
    const int rsub = lane >> 5, pos = lane & 31;
    unsigned woff[8], aoff[NA];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = 2 * i + rsub, rr = min(n0 + r, p.N - 1) - n0;
        woff[i] = (unsigned)((long long)rr * p.swn * 2 + ((pos ^ r) << 4));
    }
#pragma unroll
    for (int i = 0; i < NA; i++) {
        const int r = 2 * i + rsub, rr = min(m0 + r, p.M - 1) - m0;
        aoff[i] = (unsigned)((long long)rr * p.sam * 2 + ((pos ^ r) << 4));
    }
    const char *wb = reinterpret_cast<const char *>(reinterpret_cast<const f16 *>(p.w) + (long long)n0 * p.swn);
    const char *ab = reinterpret_cast<const char *>(reinterpret_cast<const f16 *>(p.a) + (long long)m0 * p.sam);
    // Every workgroup reads the same rows of a. Walking the k groups in the same order everywhere would have all of an
    // XCD's workgroups on the same 512-byte columns of a at once, a few L2 channels serving them all; each wave
    // therefore starts its walk at an offset given by the workgroup's place on its XCD (dispatch slot / 8).
    const int rot = ng > 1 ? (int)((blockIdx.x >> 3) % (unsigned)ng) : 0;
    auto issue = [&](int j, int st) {   // group wv + KS·((j + rot) mod ng) into stage st
        const int jj = j + rot < ng ? j + rot : j + rot - ng;
        const long long kofs = (long long)(wv + KS * jj) * ROWB;
        const unsigned dst = lbase + st * SB;
#pragma unroll
        for (int i = 0; i < 8; i++) lds_dma16(wb + kofs, woff[i], dst + i * 1024);
#pragma unroll
        for (int i = 0; i < NA; i++) lds_dma16(ab + kofs, aoff[i], dst + WB + i * 1024);
    };

    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const bool mval = r16 < MT && m0 + r16 < p.M;
    const int arow = r16 < MT ? r16 : 0;
#pragma unroll
    for (int s = 0; s < NS; s++)
        if (s < ng) issue(s, s);
    int st = 0;
    for (int j = 0; j < ng; j++) {
        wait_vm_stages<NS - 1, LPG>(min(NS - 1, ng - 1 - j));   // group j has landed
        const G9_LDS unsigned char *sg = lds + st * SB;
        u32x4 wf[8], af[8];
#pragma unroll
        for (int t = 0; t < 8; t++) {
            wf[t] = *reinterpret_cast<const G9_LDS u32x4 *>(sg + r16 * ROWB + (((4 * t + g) ^ r16) << 4));
            af[t] = *reinterpret_cast<const G9_LDS u32x4 *>(sg + WB + arow * ROWB + (((4 * t + g) ^ arow) << 4));
        }
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const u32x4 av = mval ? af[t] : u32x4{0, 0, 0, 0};
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, wf[t]), __builtin_bit_cast(f16x8, av),
                                                         acc, 0, 0, 0);
        }
        wait_lgkm0();   // the stage is refilled next: its reads must be done
        if (j + NS < ng) issue(j + NS, st);
        st = st + 1 == NS ? 0 : st + 1;
    }

    // lane holds D[n = 4g + i][m = r16]; sum the KS waves' tiles
    __syncthreads();
    float *part = reinterpret_cast<float *>(smem);   // [KS][16 n][16 m]
#pragma unroll
    for (int i = 0; i < 4; i++) part[(wv * 16 + 4 * g + i) * 16 + r16] = acc[i];
    __syncthreads();
    f16 *C = reinterpret_cast<f16 *>(p.C);
    for (int idx = threadIdx.x; idx < 16 * MT; idx += KS * 64) {
        const int n = idx / MT, m = idx % MT;
        float sum = 0.f;
#pragma unroll
        for (int q = 0; q < KS; q++) sum += part[(q * 16 + n) * 16 + m];
        const int gm = m0 + m, gn = n0 + n;
        if (gm < p.M && gn < p.N) {
            f16 *c = C + (long long)gm * p.scm + (long long)gn * p.scn;
            const float r = p.beta == 0.f ? p.alpha * sum : __builtin_fmaf(p.alpha, sum, p.beta * (float)*c);
            *c = (f16)r;
        }
    }
}

}  // namespace sk
}  // namespace g9
