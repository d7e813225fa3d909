// FP32 GEMM kernel for gfx950 with direct global→LDS loads: C = alpha·op(A)·op(B) + beta·C in true FP32 on
// v_mfma_f32_32x32x2_f32, rounded once.
//
// Semantics are those of the reference's FP32 GEMM (reference: lib/kernels/sgemm.cl:192-230 sgemm_v and its epilogue
// gen9blas_epilog_fb): every C element is the sum over k of the A·B products in FP32, then alpha·sum + beta·C (C not
// read when beta = 0).
//
// This kernel serves products whose tiles are all full (M % BM = N % BN = K % 32 = 0) with 16-byte aligned operands;
// the general kernel in gemm_kernel.h takes every other shape. Design (the FP16 whole-tile kernel's, for FP32):
// - operand tiles go from global memory straight into LDS with global_load_lds_dwordx4, through the FP16 kernel's
//   loaders (an FP32 tile seen as FP16 pairs: a k-contiguous row of 32 FP32 is one of 64 FP16); NS LDS stages of
//   32 k form a ring, and the loads for k-step t+NS are issued as soon as stage t is free;
// - k order inside a k-step: MFMA step (j, s), j = 0..3 and s = 0..3, takes k = 8j + s from lanes 0-31 and
//   k = 8j + 4 + s from lanes 32-63, for A and B alike, so every product is summed once. A k-contiguous operand is
//   read 16 bytes per lane (ds_read_b128: k = 8j + 4h .. +3, h = lane / 32, the four steps of group j), with the
//   FP16 kernel's row swizzle; an mn-contiguous operand one FP32 per lane and step (lanes 0-31 read 32 consecutive
//   mn of k-row 8j + s, lanes 32-63 of k-row 8j + 4 + s; the loader puts chunk c of k-row k at c ^ (8·((k >> 2) & 1)),
//   so the two halves fall on different banks);
// - blocked accumulation: the MFMAs of BLK consecutive k-steps (32·BLK k) of a tile sum into a fresh accumulator (its
//   first MFMA takes a zero C), which is then added to the running sum, so the FP32 rounding error grows with
//   K/(32·BLK) + 16·BLK terms instead of K/2;
// - operands are swapped in the MFMA (the B fragment is the first input), so lane l holds D[n][m = l % 32] for 16 n
//   in runs of 4: 16-byte stores of C;
// - one barrier per k-step, before its last group of MFMAs: after it the wave issues the next stage's loads and its
//   first fragment reads, then runs the last group;
// - the workgroup → tile mapping gives each XCD a contiguous range of tiles in groups of 4 tile rows.
// Two modes serve level-3 routines, as in the general kernel:
// - TRI (1: lower, 2: upper): C is square, the grid holds only the T(T+1)/2 square tiles that meet the triangle, and
//   diagonal tiles write only the elements inside it (SYRK, SYR2K);
// - KLIM: each tile's k range is cut to where a triangular operand is non-zero (NN, TRMM on the explicit triangular
//   matrix): 1 op(A) lower, k < m0 + BM; 2 op(A) upper, k >= m0; 3 op(B) lower, k >= n0; 4 op(B) upper,
//   k < n0 + BN. Tiles are dispatched longest range first, without the XCD remap (every XCD gets long and short
//   tiles alike); when every tile is resident at once, two per CU, the second half of the order is reversed.
// MSKIP: rows m < p.m_skip of C are computed but not stored (the edge strip of a product shifted up onto rows that
// the interior tiles already wrote: every load stays inside A, and no C element is written twice).
#pragma once
#include "hgemm_kernel.h"
#include <type_traits>
#include <utility>

namespace g9 {
namespace sg {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct Params {
    const float *A, *B;
    float *C;
    long long lda, ldb, ldc, sA, sB, sC;
    int M, N, K, tiles_m, tiles_n;
    float alpha, beta;
    int m_skip = 0;   // MSKIP: leading rows of C not stored
    int kpair = 0;    // KLIM: the second half of the dispatch order reversed (see the tile mapping)
};

// Fragment reads of one operand for a wave's TT tiles of 32 rows (m or n) from wave row w0 (a multiple of 32): per
// tile and group j, a u32x4 whose element s is this lane's value for MFMA step (j, s).
template <int RT, int TT, bool KC>
struct Frags {
    unsigned base;            // k-contiguous: row w0 + l % 32; mn-contiguous: k-row 4h, mn w0 + l % 32 (tile 0)
    unsigned off[KC ? 4 : TT];   // k-contiguous: chunk of group j; mn-contiguous: tile t
    __device__ __forceinline__ void init(int w0, int lane) {
        const int h = lane >> 5, i = lane & 31;
        if constexpr (KC) {
            const int sw = hg::kswz<64>(w0 + i);   // period 32 in the row
            base = (unsigned)(w0 + i) * 128;
#pragma unroll
            for (int j = 0; j < 4; j++) off[j] = (unsigned)(((2 * j + h) ^ sw) << 4);
        } else {
            constexpr int RB = RT * 4;   // bytes per k-row
            base = (unsigned)(4 * h * RB + (i & 3) * 4);
#pragma unroll
            for (int t = 0; t < TT; t++) off[t] = (unsigned)((((w0 + 32 * t + i) >> 2) ^ (8 * h)) << 4);
        }
    }
    __device__ __forceinline__ u32x4 read(const G9_LDS unsigned char *stg, int t, int j) const {
        if constexpr (KC) {
            return *reinterpret_cast<const G9_LDS u32x4 *>(stg + base + t * 32 * 128 + off[j]);
        } else {
            constexpr int RB = RT * 4;
            const G9_LDS unsigned char *b = stg + base + off[t] + 8 * j * RB;
            u32x4 v;
#pragma unroll
            for (int s = 0; s < 4; s++) v[s] = *reinterpret_cast<const G9_LDS unsigned *>(b + s * RB);
            return v;
        }
    }
};

__device__ __forceinline__ f32x16 mma(unsigned b, unsigned a, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(__builtin_bit_cast(float, b), __builtin_bit_cast(float, a), c, 0, 0, 0);
}

template <int BM, int BN, int WM, int WN, int NS, bool AK, bool BKC, int BLK = 1, int TRI = 0, int KLIM = 0,
          bool MSKIP = false>
__global__ void __launch_bounds__(WM *WN * 64) sgemm_kernel(Params p) {
    constexpr int NW = WM * WN, KB = 32;
    constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
    constexpr int ABYTES = BM * KB * 4, BBYTES = BN * KB * 4, SBYTES = ABYTES + BBYTES;
    // loaders on the FP16 view: k-contiguous RT rows of 64 FP16, or 32 k-rows of 2·RT FP16
    using LA = hg::Loader<AK ? BM : 2 * BM, AK ? 64 : KB, NW, AK, 1>;
    using LB = hg::Loader<BKC ? BN : 2 * BN, BKC ? 64 : KB, NW, BKC, 1>;
    constexpr int LPS = LA::NI + LB::NI;   // loads per stage per wave
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32");
    static_assert(NS >= 2 && (NS - 1) * LPS < 64, "loads in flight must fit vmcnt");
    static_assert(NS * SBYTES <= 160 * 1024, "stages must fit in LDS");
    static_assert(TRI == 0 || BM == BN, "triangle mode: square tiles");
    static_assert(KLIM == 0 || (TRI == 0 && AK && !BKC), "k-limited tiles: NN layout, no triangle");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[NS * SBYTES];
    G9_LDS unsigned char *lds = (G9_LDS unsigned char *)smem;
    const unsigned lds_addr = (unsigned)(uintptr_t)lds;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WM, wn = wave / WM;

    int bid = blockIdx.x, m0, n0;
    if constexpr (KLIM != 0) {
        // kpair (all tiles resident at once, two per CU): workgroups i and i + T/2 share a CU, and the second half
        // takes the ranks in reverse, so that each CU pairs a long range with a short one
        if (p.kpair) {
            const int nt = p.tiles_m * p.tiles_n, h = nt / 2;
            if (bid >= h) bid = nt - 1 - (bid - h);
        }
        if constexpr (KLIM <= 2) {   // the range depends on the tile row
            const int tr = bid / p.tiles_n;
            m0 = (KLIM == 1 ? p.tiles_m - 1 - tr : tr) * BM;
            n0 = (bid % p.tiles_n) * BN;
        } else {                     // on the tile column
            const int tc = bid / p.tiles_m;
            n0 = (KLIM == 4 ? p.tiles_n - 1 - tc : tc) * BN;
            m0 = (bid % p.tiles_m) * BM;
        }
    } else {
        const int nt = TRI ? p.tiles_m * (p.tiles_m + 1) / 2 : p.tiles_m * p.tiles_n, nt8 = nt & ~7;
        if (bid < nt8) bid = (bid & 7) * (nt8 >> 3) + (bid >> 3);
        if constexpr (TRI != 0) {
            // tile bid of the lower triangle of tiles, row by row: (tr, tc) with tc <= tr; upper: transposed
            int tr = (int)((__builtin_sqrtf(8.f * (float)bid + 1.f) - 1.f) * 0.5f);
            while ((tr + 1) * (tr + 2) / 2 <= bid) tr++;
            while (tr * (tr + 1) / 2 > bid) tr--;
            const int tc = bid - tr * (tr + 1) / 2;
            m0 = (TRI == 1 ? tr : tc) * BM;
            n0 = (TRI == 1 ? tc : tr) * BN;
        } else {
            constexpr int GM = 4;
            const int group = bid / (GM * p.tiles_n), first_m = group * GM;
            const int gsz = min(p.tiles_m - first_m, GM);
            const int in_group = bid % (GM * p.tiles_n);
            m0 = (first_m + in_group % gsz) * BM;
            n0 = (in_group / gsz) * BN;
        }
    }
    // k range of this tile (KLIM), a multiple of 32 at both ends
    int k0 = 0, k1 = p.K;
    if constexpr (KLIM == 1) k1 = min(p.K, m0 + BM);
    if constexpr (KLIM == 2) k0 = m0;
    if constexpr (KLIM == 3) k0 = n0;
    if constexpr (KLIM == 4) k1 = min(p.K, n0 + BN);

    const long long z = blockIdx.y;
    const hg::f16 *A = reinterpret_cast<const hg::f16 *>(p.A + z * p.sA + (AK ? (long long)k0 : (long long)k0 * p.lda));
    const hg::f16 *B = reinterpret_cast<const hg::f16 *>(p.B + z * p.sB + (BKC ? (long long)k0 : (long long)k0 * p.ldb));
    float *C = p.C + z * p.sC;

    LA la;
    LB lb;
    la.init(A, 2 * p.lda, AK ? m0 : 2 * m0, wave, lane);
    lb.init(B, 2 * p.ldb, BKC ? n0 : 2 * n0, wave, lane);
    Frags<BM, TM, AK> fa;
    Frags<BN, TN, BKC> fb;
    fa.init(wm * WTM, lane);
    fb.init(wn * WTN, lane);

    f32x16 acc[TN][TM], part[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; i++)
#pragma unroll
        for (int j = 0; j < TM; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    u32x4 ra[2][TM], rb[2][TN];
    auto read_group = [&](const G9_LDS unsigned char *stg, int g, int buf) {
#pragma unroll
        for (int i = 0; i < TN; i++) rb[buf][i] = fb.read(stg + ABYTES, i, g);
#pragma unroll
        for (int j = 0; j < TM; j++) ra[buf][j] = fa.read(stg, j, g);
    };
    // the four MFMA steps of group g on fragment set buf; the first step of a block starts from zero
    auto mfma_group = [&](int g, int buf, bool first) {
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int i = 0; i < TN; i++)
#pragma unroll
                for (int j = 0; j < TM; j++) {
                    const unsigned bv = rb[buf][i][s], av = ra[buf][j][s];
                    part[i][j] = mma(bv, av, first && g == 0 && s == 0 ? f32x16{} : part[i][j]);
                }
    };
    auto add_part = [&]() {
#pragma unroll
        for (int i = 0; i < TN; i++)
#pragma unroll
            for (int j = 0; j < TM; j++) acc[i][j] += part[i][j];
    };

    const int nk = (k1 - k0) / KB;
    // prologue: k-steps 0 .. NS-1 into stages 0 .. NS-1 (past the last k-step, the last one is loaded again into a
    // stage nobody reads, so every k-step issues the same number of loads), then wait for k-step 0
#pragma unroll
    for (int s = 0; s < NS; s++) {
        la.issue(lds_addr + s * SBYTES, wave);
        lb.issue(lds_addr + s * SBYTES + ABYTES, wave);
        if (s + 1 >= nk) { la.org -= la.step_k; lb.org -= lb.step_k; }
    }
    wait_vm<(NS - 1) * LPS>();
    __syncthreads();
    read_group(lds, 0, 0);

    int st = 0;   // stage holding k-step kt
    // k-step kt at position b (a constant) of its block of BLK k-steps
    auto kstep = [&](auto b_c, int kt) {
        constexpr int b = decltype(b_c)::value;
        const G9_LDS unsigned char *cur = lds + st * SBYTES;
        const int nst = st + 1 == NS ? 0 : st + 1;
        // groups 0..2: the next group's reads, then this group's MFMAs (group g uses fragment set g & 1)
#pragma unroll
        for (int g = 0; g < 3; g++) {
            read_group(cur, g + 1, (g + 1) & 1);
            mfma_group(g, g & 1, b == 0);
        }
        // k-step kt+1 in LDS (this wave's loads; after the barrier every other wave's), and every wave is done
        // reading stage st (lgkmcnt(0) before the barrier) before it is reloaded
        wait_vm<(NS - 2) * LPS>();
        wait_lgkm0();
        __syncthreads();
        la.issue(lds_addr + st * SBYTES, wave);
        lb.issue(lds_addr + st * SBYTES + ABYTES, wave);
        {
            const bool more = kt + NS + 1 < nk;   // the next issue loads k-step kt+NS+1, if it exists
            if (!more) { la.org -= la.step_k; lb.org -= lb.step_k; }
        }
        // the group after the barrier runs at raised wave priority (n = 1024 102.7 → 107.5 TFLOP/s, n = 4096 unchanged)
        __builtin_amdgcn_s_setprio(1);
        read_group(lds + nst * SBYTES, 0, 0);   // the last k-step reads a stage nobody uses (values unused)
        mfma_group(3, 1, false);
        __builtin_amdgcn_s_setprio(0);
        if constexpr (b == BLK - 1) add_part();
        st = nst;
    };
    int kt = 0;
    const auto block = [&]<int... bs>(std::integer_sequence<int, bs...>, int k0) {
        (kstep(std::integral_constant<int, bs>{}, k0 + bs), ...);
    };
    for (; kt + BLK <= nk; kt += BLK) block(std::make_integer_sequence<int, BLK>{}, kt);
    if (kt < nk) {   // a last, shorter block
        kstep(std::integral_constant<int, 0>{}, kt);
        for (kt++; kt < nk; kt++) kstep(std::integral_constant<int, 1>{}, kt);
        add_part();
    }
    wait_vm<0>();   // the loads into stages nobody reads have landed before the wave ends

    // Epilogue. Lane l holds D[n][m] of tile (i, j) for m = 32j + l % 32 and, in accumulator r, n = 32i + 8·(r / 4)
    // + 4·(l / 32) + r % 4: runs of 4 consecutive n, one 16-byte store each (alpha·acc + beta·C in FP32).
    // On a diagonal tile of the triangle mode each element inside the triangle is stored on its own.
    const float alpha = p.alpha, beta = p.beta;
    const int h = lane >> 5;
    const bool diag = TRI != 0 && m0 == n0;
#pragma unroll
    for (int i = 0; i < TN; i++)
#pragma unroll
        for (int j = 0; j < TM; j++) {
            const int m = m0 + wm * WTM + 32 * j + (lane & 31);
            if (MSKIP && m < p.m_skip) continue;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int n = n0 + wn * WTN + 32 * i + 8 * q + 4 * h;
                float *cp = C + (long long)m * p.ldc + n;
                if (diag) {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (TRI == 1 ? n + e <= m : n + e >= m) {
                            const float x = alpha * acc[i][j][4 * q + e];
                            cp[e] = beta != 0.f ? __builtin_fmaf(beta, cp[e], x) : x;
                        }
                    continue;
                }
                f32x4 o = beta != 0.f ? *reinterpret_cast<const f32x4 *>(cp) : f32x4{0.f, 0.f, 0.f, 0.f};
                f32x4 v;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float x = alpha * acc[i][j][4 * q + e];
                    v[e] = beta != 0.f ? __builtin_fmaf(beta, o[e], x) : x;
                }
                *reinterpret_cast<f32x4 *>(cp) = v;
            }
        }
}

}  // namespace sg
}  // namespace g9
