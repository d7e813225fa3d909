// FP16 GEMM kernel for gfx950 with direct global→LDS loads: C = alpha·op(A)·op(B) + beta·C, FP32 accumulation on
// v_mfma_f32_32x32x16_f16, result rounded once to FP16.
//
// Semantics are those of the reference's FP16 GEMM (reference: lib/kernels/hgemm.cl:838-898 hgemm_v / hgemm_kc_v,
// lib/kernels/hgemm.cl:558-564 gen9blas_epilog_b): every C element is the sum over k of the A·B products, then
// alpha·sum + beta·C in FP32 (C not read when beta = 0), rounded once to FP16. The MFMA accumulates in FP32, which
// gives both reference modes (FP16 chains, or FP32 partial sums every 32 products) at least their accuracy.
//
// This kernel serves products whose tiles are all full (M % BM = N % BN = K % KB = 0) with 16-byte aligned
// operands; the general FP16 kernel in gemm_kernel.h takes every other shape. Design:
// - operand tiles go from global memory straight into LDS with global_load_lds_dwordx4 (no register staging, no
//   LDS write instructions): lane L of one instruction writes the 16 bytes at LDS offset base + 16·L, so each lane
//   is given the global address whose data belongs at that LDS position;
// - NS LDS stages of KB k each form a ring: the loads for k-step t+NS are issued as soon as stage t is free, so a
//   load has about NS-1 k-steps to arrive;
// - one barrier per k-step, placed before the last k16 substep: after it the wave issues the next stage's loads and
//   its first fragment reads, then runs the last substep's MFMAs, so neither the barrier nor the first LDS reads of
//   a k-step leave the matrix cores idle for long;
// - a k-contiguous operand (A not transposed, B transposed) is held as rows of KB k and read with ds_read_b128,
//   one 16-byte fragment per lane. Chunk c (k = 8c .. 8c+7) of row r sits at physical chunk c ^ ((r / R) % CPR)
//   (CPR chunks per row, R rows per 256 bytes): the 16 lanes that one LDS cycle serves read 16 consecutive rows at
//   one logical chunk, and the swizzle spreads them over all 64 banks;
// - an mn-contiguous operand (A transposed, B not transposed) is held as KB rows of k, each BM (or BN) elements
//   long, and read with ds_read_b64_tr_b16, which transposes 16-lane groups: lane j of a group reads 4 consecutive
//   mn of row kb + j/4, and lane i receives mn i of rows kb .. kb+3. Chunk c of row k sits at c ^ (4·(k & 3)), so
//   the four rows of a group fall on distinct banks;
// - operands are swapped in the MFMA (the B fragment is the first input), so each lane ends with runs of 4
//   consecutive n of one row of C; v_permlane32_swap joins two runs, giving 16-byte stores;
// - the workgroup → tile mapping gives each XCD a contiguous range of tiles, ordered in groups of 4 tile rows, so
//   one XCD's L2 serves the A and B panels its tiles share.
#pragma once
#include "internal.h"
#include "lds_dma.h"

namespace g9 {
namespace hg {

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

struct Params {
    const f16 *A, *B;
    f16 *C;
    long long lda, ldb, ldc, sA, sB, sC;
    int M, N, K, tiles_m, tiles_n;
    float alpha, beta;
};

// Global → LDS loads of one operand tile: RT rows (m or n) × KB k, RT·KB·2 bytes, issued by NW waves.
// KC: stored k-contiguous (element (mn, k) at X[mn·ld + k]); otherwise mn-contiguous (element (mn, k) at X[k·ld + mn]).
// Each lane's byte offset from the tile origin is fixed for the whole kernel; the wave-uniform origin advances.
template <int RT, int KB, int NW, bool KC>
struct Loader {
    static constexpr int NINST = RT * KB * 2 / 1024;       // 1 KiB instructions per tile
    static constexpr int NI = NINST / NW;                  // per wave
    static constexpr int CPRK = KB / 8, RPIK = 512 / KB, RK = 128 / KB;   // k-contiguous: chunks per row, rows per
                                                                          // instruction, rows per 256 bytes
    static constexpr int CPR = RT / 8, RPI = 512 / RT;                    // mn-contiguous: chunks per row, rows per
                                                                          // instruction
    static_assert(NINST % NW == 0, "tile instructions must divide over the waves");
    static_assert(!KC || (4 * NW) % CPRK == 0, "k-contiguous swizzle must repeat over a wave's instructions");
    static_assert(KC || (RT >= 128 && (RPI * NW) % 4 == 0), "mn-contiguous swizzle must repeat over a wave's instructions");
    const char *org;      // wave-uniform: tile origin at the next k-step to load
    unsigned voff;        // this lane's byte offset for instruction 0
    long long step_i;     // bytes between consecutive instructions of this wave
    long long step_k;     // bytes per k-step

    __device__ __forceinline__ void init(const f16 *X, long long ld, int mn0, int wave, int lane) {
        if constexpr (KC) {
            // instruction j = wave + NW·i covers rows RPIK·j ..; lane L: row RPIK·j + L / CPRK, physical chunk L % CPRK
            const int r = RPIK * wave + lane / CPRK;
            const int c = (lane % CPRK) ^ ((r / RK) % CPRK);
            org = reinterpret_cast<const char *>(X + (long long)mn0 * ld);
            voff = (unsigned)(((long long)r * ld + 8 * c) * 2);
            step_i = (long long)RPIK * NW * ld * 2;
            step_k = KB * 2;
        } else {
            // instruction j covers k rows RPI·j ..; lane L: row RPI·j + L / CPR, physical chunk L % CPR
            const int k = RPI * wave + lane / CPR;
            const int c = (lane % CPR) ^ (4 * (k & 3));
            org = reinterpret_cast<const char *>(X + mn0);
            voff = (unsigned)(((long long)k * ld + 8 * c) * 2);
            step_i = (long long)RPI * NW * ld * 2;
            step_k = (long long)KB * ld * 2;
        }
    }
    // Issues this wave's loads of the next k-step into the tile at LDS address `dst`, then advances.
    __device__ __forceinline__ void issue(unsigned dst, int wave) {
#pragma unroll
        for (int i = 0; i < NI; i++) one(i, dst, wave);
        org += step_k;
    }
    // Instruction i of this wave's loads of the current k-step; advance() moves to the next k-step.
    __device__ __forceinline__ void one(int i, unsigned dst, int wave) const {
        lds_dma16(org + i * step_i, voff, dst + 1024 * (wave + NW * i));
    }
    __device__ __forceinline__ void advance(bool more) { if (more) org += step_k; }
};

// Fragment reads of one operand for a wave's TT MFMA tiles (32 rows of m or n each, starting at wave row w0).
template <int RT, int KB, int TT, bool KC>
struct Frags {
    static constexpr int NSUB = KB / 16, CPRK = KB / 8, RK = 128 / KB;
    unsigned off[KC ? NSUB : TT];   // per-lane byte offsets: per k16 substep (KC) or per tile (transposed reads)
    __device__ __forceinline__ void init(int w0, int lane) {
        if constexpr (KC) {
            const int r = lane & 31, hi = lane >> 5, sw = (r / RK) % CPRK;   // w0 + 32·t adds nothing to sw
#pragma unroll
            for (int s = 0; s < NSUB; s++) off[s] = (w0 + r) * (KB * 2) + (((2 * s + hi) ^ sw) << 4);
        } else {
            const int G = lane >> 4, j = lane & 15, q = j >> 2;
            const int krow = 8 * (G >> 1) + q;                      // + 16·s + 4·h (immediates)
            const int low = 2 * (G & 1) + ((j & 3) >> 1);           // chunk bits 0-1
#pragma unroll
            for (int t = 0; t < TT; t++) {
                const int tc = (w0 >> 5) + t;                       // 32-wide tile index = chunk bits 2 and up
                off[t] = krow * (RT * 2) + ((tc ^ q) << 6) + (low << 4) + 8 * (j & 1);   // q < 4 flips bits 2-3 only
            }
        }
    }
    // 16-byte fragment of tile t, substep s from the stage at `base`.
    __device__ __forceinline__ u32x4 read(const G9_LDS unsigned char *base, int t, int s) const {
        if constexpr (KC) {
            return *reinterpret_cast<const G9_LDS u32x4 *>(base + off[s] + t * 32 * (KB * 2));
        } else {
            const G9_LDS unsigned char *b = base + off[t] + 16 * s * (RT * 2);
            const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((G9_LDS i16x4 *)(b));
            const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((G9_LDS i16x4 *)(b + 4 * (RT * 2)));
            const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
            return u32x4{l2[0], l2[1], h2[0], h2[1]};
        }
    }
};

template <int BM, int BN, int WM, int WN, int KB, int NS, bool AK, bool BKC>
__global__ void __launch_bounds__(WM *WN * 64) hgemm_kernel(Params p) {
    constexpr int NW = WM * WN;
    constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
    constexpr int ABYTES = BM * KB * 2, BBYTES = BN * KB * 2, SBYTES = ABYTES + BBYTES;
    constexpr int NSUB = KB / 16;
    using LA = Loader<BM, KB, NW, AK>;
    using LB = Loader<BN, KB, NW, BKC>;
    constexpr int LPS = LA::NI + LB::NI;   // loads per stage per wave
    static_assert(TM * 32 == WTM && TN * 32 == WTN, "wave tile must be a multiple of 32");
    static_assert(NSUB % 2 == 0, "fragment double buffer alternates over an even number of substeps");
    static_assert(NS >= 2 && (NS - 1) * LPS < 64, "loads in flight must fit vmcnt");
    // stage s: [A tile | B tile] at s·SBYTES
    __shared__ __attribute__((aligned(1024))) unsigned char smem[NS * SBYTES];
    G9_LDS unsigned char *lds = (G9_LDS unsigned char *)smem;
    const unsigned lds_addr = (unsigned)(uintptr_t)lds;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WM, wn = wave / WM;

    int bid = blockIdx.x;
    const int nt = p.tiles_m * p.tiles_n, nt8 = nt & ~7;
    if (bid < nt8) bid = (bid & 7) * (nt8 >> 3) + (bid >> 3);
    constexpr int GM = 4;
    const int group = bid / (GM * p.tiles_n), first_m = group * GM;
    const int gsz = min(p.tiles_m - first_m, GM);
    const int in_group = bid % (GM * p.tiles_n);
    const int m0 = (first_m + in_group % gsz) * BM, n0 = (in_group / gsz) * BN;

    const long long z = blockIdx.y;
    const f16 *A = p.A + z * p.sA;
    const f16 *B = p.B + z * p.sB;
    f16 *C = p.C + z * p.sC;

    LA la;
    LB lb;
    la.init(A, p.lda, m0, wave, lane);
    lb.init(B, p.ldb, n0, wave, lane);
    Frags<BM, KB, TM, AK> fa;
    Frags<BN, KB, TN, BKC> fb;
    fa.init(wm * WTM, lane);
    fb.init(wn * WTN, lane);

    f32x16 acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; i++)
#pragma unroll
        for (int j = 0; j < TM; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    u32x4 ra[2][TM], rb[2][TN];
    auto read_frags = [&](const G9_LDS unsigned char *stg, int s, int buf) {
#pragma unroll
        for (int j = 0; j < TM; j++) ra[buf][j] = fa.read(stg, j, s);
#pragma unroll
        for (int i = 0; i < TN; i++) rb[buf][i] = fb.read(stg + ABYTES, i, s);
    };
    const int nk = p.K / KB;
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
    read_frags(lds, 0, 0);

    // One k-step: NSUB substeps of TM·TN MFMAs. The instruction order is pinned (sched_barrier between slots):
    // slot t of a substep holds MFMA t followed by its share of the next substep's fragment reads (in the order the
    // MFMAs use them); before the last
    // substep, the wait for k-step kt+1 and the barrier; in the last substep, the reads of k-step kt+1's first
    // substep and the loads of k-step kt+NS into the stage just released, spread over the MFMA slots.
    constexpr int NMF = TM * TN;
    constexpr int NRF = TM + TN;                 // fragments per substep
    constexpr int NLD = LPS;                     // global→LDS copies per k-step
    int st = 0;   // stage holding k-step kt
    for (int kt = 0; kt < nk; kt++) {
        const G9_LDS unsigned char *cur = lds + st * SBYTES;
        const int nst = st + 1 == NS ? 0 : st + 1;
#pragma unroll
        for (int s = 0; s < NSUB - 1; s++) {
            const int nb = (s + 1) & 1;
#pragma unroll
            for (int t = 0; t < NMF; t++) {
                const int i = t / TM, j = t % TM;
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, rb[s & 1][i]),
                                                                   __builtin_bit_cast(f16x8, ra[s & 1][j]), acc[i][j], 0, 0, 0);
                constexpr int PER = (NRF + NMF - 1) / NMF;
#pragma unroll
                for (int q = t * PER; q < (t + 1) * PER && q < NRF; q++) {   // in order of first use
                    if (q == 0) rb[nb][0] = fb.read(cur + ABYTES, 0, s + 1);
                    else if (q <= TM) ra[nb][q - 1] = fa.read(cur, q - 1, s + 1);
                    else rb[nb][q - TM] = fb.read(cur + ABYTES, q - TM, s + 1);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // k-step kt+1 in LDS: this wave's loads (NS-2 later k-steps may stay in flight) and, after the barrier, every
        // other wave's; all waves are done reading stage st (lgkmcnt(0) before the barrier) before it is reloaded.
        wait_vm<(NS - 2) * LPS>();
        wait_lgkm0();
        __syncthreads();
        {
            constexpr int s = NSUB - 1;
            const G9_LDS unsigned char *nxt = lds + nst * SBYTES;
            const unsigned dsta = lds_addr + st * SBYTES, dstb = dsta + ABYTES;
            constexpr int NIT = NRF + NLD, PER = (NIT + NMF - 1) / NMF;
#pragma unroll
            for (int t = 0; t < NMF; t++) {
                const int i = t / TM, j = t % TM;
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, rb[s & 1][i]),
                                                                   __builtin_bit_cast(f16x8, ra[s & 1][j]), acc[i][j], 0, 0, 0);
#pragma unroll
                for (int q = t * PER; q < (t + 1) * PER && q < NIT; q++) {
                    if (q == 0) rb[0][0] = fb.read(nxt + ABYTES, 0, 0);
                    else if (q <= TM) ra[0][q - 1] = fa.read(nxt, q - 1, 0);
                    else if (q < NRF) rb[0][q - TM] = fb.read(nxt + ABYTES, q - TM, 0);
                    else if (q - NRF < LA::NI) la.one(q - NRF, dsta, wave);
                    else lb.one(q - NRF - LA::NI, dstb, wave);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            const bool more = kt + NS + 1 < nk;   // the next issue loads k-step kt+NS+1, if it exists
            la.advance(more);
            lb.advance(more);
        }
        st = nst;
    }
    wait_vm<0>();   // the loads into stages nobody reads have landed before the wave ends

    // Epilogue. Lane l holds D[n][m] for m = lane % 32 of MFMA tile j and n in runs of 4: rows 8q + 4·(l / 32) .. +3
    // of tile i, q = 0..3. Each run becomes 4 FP16 values (alpha·acc + beta·C in FP32, rounded once); then lanes l and
    // l+32 trade runs with v_permlane32_swap, so that each lane holds 8 consecutive n (16 bytes): lane l < 32 those of
    // q = 2p, lane l + 32 those of q = 2p + 1, for p = 0, 1. Two 16-byte stores per MFMA tile and lane.
    const float alpha = p.alpha, beta = p.beta;
    const int hi = lane >> 5;
#pragma unroll
    for (int i = 0; i < TN; i++)
#pragma unroll
        for (int j = 0; j < TM; j++) {
            const int m = m0 + wm * WTM + j * 32 + (lane & 31);
            f16 *crow = C + (long long)m * p.ldc + n0 + wn * WTN + i * 32;
#pragma unroll
            for (int pr = 0; pr < 2; pr++) {
                unsigned w[2][2];   // [q - 2·pr][dword]: the lane's own run of q, 4 FP16 values
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int q = 2 * pr + h;
                    union { u32x2 w; f16 e[4]; } o, v;
                    if (beta != 0.f) o.w = *reinterpret_cast<const u32x2 *>(crow + 8 * q + 4 * hi);
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float x = alpha * acc[i][j][4 * q + e];
                        v.e[e] = (f16)(beta != 0.f ? __builtin_fmaf(beta, (float)o.e[e], x) : x);
                    }
                    w[h][0] = v.w[0];
                    w[h][1] = v.w[1];
                }
                // swap lanes 32..63 of the q = 2pr run with lanes 0..31 of the q = 2pr+1 run
                const auto s0 = __builtin_amdgcn_permlane32_swap(w[0][0], w[1][0], false, false);
                const auto s1 = __builtin_amdgcn_permlane32_swap(w[0][1], w[1][1], false, false);
                const u32x4 out = {s0[0], s1[0], s0[1], s1[1]};
                *reinterpret_cast<u32x4 *>(crow + 8 * (2 * pr + hi)) = out;
            }
        }
}

}  // namespace hg
}  // namespace g9
