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

// ---------------- weights contiguous along N ----------------
// C (M×N) = alpha·a·W + beta·C with a M×K (K-contiguous) and W K×N, element (k, n) at w[k·swk + n]: row-major x·W with
// W stored (in, out).
// Matrix-core form: a workgroup owns a strip of SW = 64 or 128 columns (SWB = 128 or 256 bytes of each W row: whole
// cache lines) and one of P parts of K; the FP32 partial tiles go to P·M·N sums that skinny_n_sum adds in part order
// (the reference's skinny_n4 / skinny_n2 split, reference: lib/kernels/level12.cl:803-862). With P = 1 the workgroup
// applies alpha / beta and stores C itself. Narrower strips without the split (16 columns over all of K, N = 4096:
// 256 workgroups, no second kernel) were measured and not kept: a strip then reads 32-byte pieces of 4 lines per W
// row and the kernel is bound by the count of requests, not by bytes (17.3 µs per call at M = 1..16 against
// 11.8-13.0 here, MI355X, W 4096² rotated over 32 copies); so was finishing the sum in the kernel by the last part
// to arrive (agent-scope atomic stores, an arrival counter, atomic loads: exact, but 11.5 µs at M = 1 and up to 20 µs
// at M = 16).
// Per wave an NS-stage LDS ring of groups of GK = 8192 / SWB k (8 KiB of W), filled by global_load_lds_dwordx4:
// - W: 8 copies of 1 KiB, copy i = k-rows RPI·i .. (RPI = 1024 / SWB rows of CPR = SWB / 16 chunks), lane L = chunk
//   L % CPR of row RPI·i + L / CPR; logical chunk c of row r sits at physical chunk c ^ wswz(r), which puts the four
//   k-rows each 16-lane group of a transposing read touches, and the two groups one LDS cycle serves (k-rows 8g + 0..3
//   for g = 0 and 1), on 64 distinct banks;
// - a: the MT rows of GK k, chunk c of row r at c ^ ((r / rows per 256 bytes) mod chunks per row).
// Per group SW/16 n tiles × GK/32 substeps: 8 MFMAs per 8 KiB of W.
// The MFMA's first operand needs 8 consecutive k of one column per lane: ds_read_b64_tr_b16 gives it. In 16-lane
// group g, lane j reads 4 consecutive columns 4·(j & 3) of k-row 8g + (j >> 2) (then + 4), and lane i receives column
// i of those 4 k-rows.
// Requires K % (GK·P) == 0, N ≥ SW, N % 8 == 0 and 16-byte aligned rows of a and W (the launcher checks). The last
// strip is shifted back to end at N; its columns below its own start are computed again but not stored.
struct ParamsNP {
    const void *a, *w;
    float *P;              // partial sums [part][m][n] (P > 1)
    void *C;               // P = 1: the result
    long long sam, swk, scm, scn;
    int M, N, K, parts;
    float alpha, beta;
};

template <int SWB> __device__ __forceinline__ int wswz(int r) {
    if constexpr (SWB == 64) return ((r >> 3) & 1) << 1;
    if constexpr (SWB == 128) return (((r >> 1) & 1) << 2) ^ (((r >> 3) & 1) << 1);
    else return 2 * (r & 3) + 8 * ((r >> 3) & 1);
}

template <int SWB, int MT, int KS, int NS>
__global__ void __launch_bounds__(KS * 64) skinny_np_mfma_kernel(ParamsNP p) {
    typedef f16 f16x8 __attribute__((ext_vector_type(8)));
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef short i16x4 __attribute__((ext_vector_type(4)));
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    static_assert(SWB == 64 || SWB == 128 || SWB == 256, "strips of 32, 64 or 128 columns");
    constexpr int SW = SWB / 2, NT = SW / 16, GK = 8192 / SWB, NSUB = GK / 32;
    constexpr int RPI = 1024 / SWB, CPR = SWB / 16;
    constexpr int AROWB = GK * 2, CPRA = AROWB / 16, RPIA = 1024 / AROWB, RPBA = 256 / AROWB;
    constexpr int NA = (MT + RPIA - 1) / RPIA;
    constexpr int WB = 8 * 1024, AB = NA * 1024, SB = WB + AB;
    constexpr int LPG = 8 + NA;
    static_assert((NS - 1) * LPG < 64, "copies in flight must fit vmcnt");
    static_assert(KS * NS * SB >= KS * SW * 16 * 4, "the stage ring holds the wave tiles' sums");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[KS * NS * SB];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, r16 = lane & 15;
    const int part = blockIdx.x % p.parts, strip = blockIdx.x / p.parts;
    const int nown = strip * SW, n0 = min(nown, p.N - SW), m0 = blockIdx.y * MT;
    const unsigned lbase = (unsigned)(uintptr_t)smem + wv * NS * SB;
    const G9_LDS unsigned char *lds = (const G9_LDS unsigned char *)smem + wv * NS * SB;
    const int gpp = p.K / GK / p.parts;            // groups per part
    const int g0 = part * gpp;
    const int ng = gpp > wv ? (gpp - wv + KS - 1) / KS : 0;

    unsigned woff[8], aoff[NA];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = RPI * i + lane / CPR;
        woff[i] = (unsigned)(((long long)r * p.swk + 8 * ((lane % CPR) ^ wswz<SWB>(r))) * 2);
    }
#pragma unroll
    for (int i = 0; i < NA; i++) {
        const int r = RPIA * i + lane / CPRA, rr = min(m0 + r, p.M - 1) - m0;
        aoff[i] = (unsigned)(((long long)rr * p.sam + 8 * ((lane % CPRA) ^ ((r / RPBA) % CPRA))) * 2);
    }
    const char *wb = reinterpret_cast<const char *>(reinterpret_cast<const f16 *>(p.w) + n0);
    const char *ab = reinterpret_cast<const char *>(reinterpret_cast<const f16 *>(p.a) + (long long)m0 * p.sam);
    const long long wgroup = (long long)GK * p.swk * 2;
    auto issue = [&](int j, int st) {   // group g0 + wv + KS·j into stage st
        const int grp = g0 + wv + KS * j;
        const unsigned dst = lbase + st * SB;
        const char *wg = wb + grp * wgroup;
#pragma unroll
        for (int i = 0; i < 8; i++) lds_dma16(wg, woff[i], dst + i * 1024);
        const char *ag = ab + (long long)grp * AROWB;
#pragma unroll
        for (int i = 0; i < NA; i++) lds_dma16(ag, aoff[i], dst + WB + i * 1024);
    };

    f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const bool mval = r16 < MT && m0 + r16 < p.M;
    const int arow = r16 < MT ? r16 : 0;
    const int q = r16 >> 2, c4 = r16 & 3;
#pragma unroll
    for (int st0 = 0; st0 < NS; st0++)
        if (st0 < ng) issue(st0, st0);
    int st = 0;
    for (int j = 0; j < ng; j++) {
        wait_vm_stages<NS - 1, LPG>(min(NS - 1, ng - 1 - j));
        const G9_LDS unsigned char *sg = lds + st * SB;
#pragma unroll
        for (int t = 0; t < NSUB; t++) {
            u32x4 wf[NT];
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                u32x2 hv[2];
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    // transposing read: k-row 32t + 8g + 4h + (j >> 2), columns 16·nt + 4·(j & 3) .. + 3
                    const int r = 32 * t + 8 * g + 4 * h + q;
                    const int chunk = (2 * nt + (c4 >> 1)) ^ wswz<SWB>(r);
                    const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (G9_LDS i16x4 *)(sg + r * SWB + chunk * 16 + 8 * (c4 & 1)));
                    hv[h] = __builtin_bit_cast(u32x2, v);
                }
                wf[nt] = u32x4{hv[0][0], hv[0][1], hv[1][0], hv[1][1]};
            }
            const u32x4 afr = *reinterpret_cast<const G9_LDS u32x4 *>(
                sg + WB + arow * AROWB + (((4 * t + g) ^ ((arow / RPBA) % CPRA)) << 4));
            const u32x4 av = mval ? afr : u32x4{0, 0, 0, 0};
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, wf[nt]),
                                                                 __builtin_bit_cast(f16x8, av), acc[nt], 0, 0, 0);
        }
        wait_lgkm0();
        if (j + NS < ng) issue(j + NS, st);
        st = st + 1 == NS ? 0 : st + 1;
    }

    // lane holds D[n = n0 + 16·nt + 4g + i][m = r16]; sum the KS waves' tiles
    __syncthreads();
    float *red = reinterpret_cast<float *>(smem);   // [KS][SW n][16 m]
#pragma unroll
    for (int nt = 0; nt < NT; nt++)
#pragma unroll
        for (int i = 0; i < 4; i++) red[(wv * SW + 16 * nt + 4 * g + i) * 16 + r16] = acc[nt][i];
    __syncthreads();
    f16 *C = reinterpret_cast<f16 *>(p.C);
    const long long plane = (long long)p.M * p.N;
    for (int idx = threadIdx.x; idx < SW * MT; idx += KS * 64) {
        const int m = idx / SW, n = idx % SW;   // consecutive threads: consecutive n
        if (m0 + m >= p.M || n0 + n < nown) continue;
        float sum = 0.f;
#pragma unroll
        for (int qq = 0; qq < KS; qq++) sum += red[(qq * SW + n) * 16 + m];
        if (p.parts == 1) {
            f16 *c = C + (long long)(m0 + m) * p.scm + (long long)(n0 + n) * p.scn;
            *c = (f16)(p.beta == 0.f ? p.alpha * sum : __builtin_fmaf(p.alpha, sum, p.beta * (float)*c));
        } else {
            p.P[part * plane + (long long)(m0 + m) * p.N + n0 + n] = sum;
        }
    }
}

// C[m][n] = alpha·Σ_part P[part][m][n] + beta·C (C not read when beta = 0), parts added in index order.
template <class T>
__global__ void __launch_bounds__(256) skinny_n_sum_kernel(const float *P, int parts, int M, int N, float alpha,
                                                           float beta, T *C, long long scm, long long scn) {
    const long long total = (long long)M * N;
    for (long long i = blockIdx.x * 256LL + threadIdx.x; i < total; i += (long long)gridDim.x * 256) {
        float s = 0.f;
        for (int q = 0; q < parts; q++) s += P[(long long)q * total + i];
        const int m = (int)(i / N), n = (int)(i % N);
        T *c = C + (long long)m * scm + (long long)n * scn;
        *c = (T)(beta == 0.f ? alpha * s : __builtin_fmaf(alpha, s, beta * (float)*c));
    }
}

// Parameters of the vector form below: a workgroup per strip of 16 columns over all of K. The strips that share a
// 128-byte line of a W row run on one XCD (dispatch places workgroup b on XCD b mod 8; each XCD takes a contiguous
// range of strips), so their L2 fetches the line once.
struct ParamsN {
    const void *a, *w;
    void *C;
    long long sam, swk, scm, scn;
    int M, N, K;
    float alpha, beta;
    int strips, per_xcd;   // 16-column strips, strips per XCD (workgroups = 8·per_xcd per m tile)
};

// Strip of workgroup blockIdx.x (or -1 past the end).
__device__ __forceinline__ int strip_of(const ParamsN &p) {
    const int s = (int)(blockIdx.x & 7) * p.per_xcd + (int)(blockIdx.x >> 3);
    return s < p.strips ? s : -1;
}

// General form on the vector ALU (FP32, and FP16 shapes the matrix-core form does not take): FP32 sums of products
// of the inputs, as in skinny_kernel. A workgroup of KS waves owns a strip of 16 columns; a wave covers R = 64·V/16
// k-rows per step (V elements per lane: 16 bytes when VEC, else V = 4 single-element loads), its lanes holding V
// consecutive columns of one k-row and MT partial sums per column. The a values of a step are staged in LDS by the
// wave itself and read as broadcasts. Sums: across the lanes of one column group (shuffles), then across the waves
// (LDS).
template <class T, int MT, int KS, bool VEC>
__global__ void __launch_bounds__(KS * 64) skinny_n_valu_kernel(ParamsN p) {
    constexpr int V = VEC ? 16 / (int)sizeof(T) : 4;   // columns per lane
    constexpr int LPR = 16 / V;                         // lanes per k-row of the strip
    constexpr int R = 64 / LPR;                         // k-rows per wave step
    __shared__ float abuf[KS][MT][R];
    __shared__ float part[KS][MT][16];
    const int s = strip_of(p);
    if (s < 0) return;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int nown = s * 16, m0 = blockIdx.y * MT;
    const int n0 = VEC ? min(nown, p.N - 16) : nown;   // VEC: N ≥ 16, shifted back at the end
    const int col = n0 + (lane % LPR) * V, kr = lane / LPR;
    const T *w = reinterpret_cast<const T *>(p.w), *a = reinterpret_cast<const T *>(p.a);
    float acc[MT][V];
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
        for (int v = 0; v < V; v++) acc[m][v] = 0.f;
    for (int k0 = wv * R; k0 < p.K; k0 += KS * R) {
        // stage a[m0 .. m0+MT-1][k0 .. k0+R-1] (zero past K or M)
        for (int t = lane; t < MT * R; t += 64) {
            const int m = t / R, kk = k0 + t % R;
            abuf[wv][m][t % R] = (m0 + m < p.M && kk < p.K) ? (float)a[(long long)(m0 + m) * p.sam + kk] : 0.f;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        const int k = k0 + kr;
        float x[V];
        if (k < p.K) {
            const T *row = w + (long long)k * p.swk;
            if constexpr (VEC) {
                const u32x4 q = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(row + col));
                const T *e = reinterpret_cast<const T *>(&q);
#pragma unroll
                for (int v = 0; v < V; v++) x[v] = (float)e[v];
            } else {
#pragma unroll
                for (int v = 0; v < V; v++) x[v] = col + v < p.N ? (float)row[col + v] : 0.f;
            }
        } else {
#pragma unroll
            for (int v = 0; v < V; v++) x[v] = 0.f;
        }
#pragma unroll
        for (int m = 0; m < MT; m++) {
            const float am = abuf[wv][m][kr];
#pragma unroll
            for (int v = 0; v < V; v++) acc[m][v] = __builtin_fmaf(am, x[v], acc[m][v]);
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // sum over the lanes of one column group (lane bits above log2(LPR))
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
        for (int v = 0; v < V; v++)
            for (int d = LPR; d < 64; d *= 2) acc[m][v] += __shfl_xor(acc[m][v], d);
    if (lane < LPR)
#pragma unroll
        for (int m = 0; m < MT; m++)
#pragma unroll
            for (int v = 0; v < V; v++) part[wv][m][lane * V + v] = acc[m][v];
    __syncthreads();
    T *C = reinterpret_cast<T *>(p.C);
    for (int idx = threadIdx.x; idx < 16 * MT; idx += KS * 64) {
        const int n = idx / MT, m = idx % MT;
        float sum = 0.f;
#pragma unroll
        for (int qq = 0; qq < KS; qq++) sum += part[qq][m][n];
        const int gm = m0 + m, gn = n0 + n;
        if (gm < p.M && gn >= nown && gn < p.N) {
            T *c = C + (long long)gm * p.scm + (long long)gn * p.scn;
            const float r = p.beta == 0.f ? p.alpha * sum : __builtin_fmaf(p.alpha, sum, p.beta * (float)*c);
            *c = (T)r;
        }
    }
}

// a with a k stride (a[m][k] at a[m·sam + k·sak]) copied K-contiguous into `out` (row stride ldo), for the kernels
// above, which read a k-contiguously.
template <class T>
__global__ void __launch_bounds__(256) gather_a_kernel(const T *a, long long sam, long long sak, int M, int K, T *out,
                                                       long long ldo) {
    const long long total = (long long)M * K;
    for (long long i = blockIdx.x * 256LL + threadIdx.x; i < total; i += (long long)gridDim.x * 256) {
        const int m = (int)(i % M), k = (int)(i / M);   // consecutive threads: consecutive m (contiguous when sam = 1)
        out[(long long)m * ldo + k] = a[(long long)m * sam + (long long)k * sak];
    }
}

}  // namespace sk
}  // namespace g9
