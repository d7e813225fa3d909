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
// - operands are swapped in the MFMA (the B fragment is the first input), so each lane ends with 4 consecutive n
//   of one row of C: 8-byte stores;
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
        for (int i = 0; i < NI; i++) lds_dma16(org + i * step_i, voff, dst + 1024 * (wave + NW * i));
        org += step_k;
    }
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
    auto mfmas = [&](int buf) {
#pragma unroll
        for (int i = 0; i < TN; i++)
#pragma unroll
            for (int j = 0; j < TM; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, rb[buf][i]),
                                                                   __builtin_bit_cast(f16x8, ra[buf][j]), acc[i][j], 0, 0, 0);
    };
    auto issue = [&](int stg) {
        la.issue(lds_addr + stg * SBYTES, wave);
        lb.issue(lds_addr + stg * SBYTES + ABYTES, wave);
    };

    const int nk = p.K / KB;
    // prologue: k-steps 0 .. NS-1 into stages 0 .. NS-1, then wait for k-step 0
#pragma unroll
    for (int s = 0; s < NS; s++)
        if (s < nk) issue(s);
    wait_vm_stages<NS - 1, LPS>(min(NS - 1, nk - 1));
    __syncthreads();
    read_frags(lds, 0, 0);

    int st = 0;   // stage holding k-step kt
    for (int kt = 0; kt < nk; kt++) {
        const G9_LDS unsigned char *cur = lds + st * SBYTES;
        const int nst = st + 1 == NS ? 0 : st + 1;
#pragma unroll
        for (int s = 0; s < NSUB; s++) {
            if (s + 1 < NSUB) {
                read_frags(cur, s + 1, (s + 1) & 1);
            } else if (kt + 1 < nk) {
                // Before the last substep: k-step kt+1 must be in LDS (this wave's loads: at most min(NS-2, nk-2-kt)
                // later stages still in flight; the other waves': the barrier), and every wave must be done reading
                // stage st (its fragments are in registers: lgkmcnt(0), then the barrier) before the stage is
                // reloaded with k-step kt+NS.
                wait_vm_stages<NS - 2, LPS>(min(NS - 2, nk - 2 - kt));
                wait_lgkm0();
                __syncthreads();
                if (kt + NS < nk) issue(st);
                read_frags(lds + nst * SBYTES, 0, 0);
            }
            mfmas(s & 1);
        }
        st = nst;
    }

    // lane holds D[n][m]: m = lane % 32 of MFMA tile j, n in runs of 4 (rows 8q + 4·(lane/32) .. +3 of tile i)
    const float alpha = p.alpha, beta = p.beta;
#pragma unroll
    for (int i = 0; i < TN; i++)
#pragma unroll
        for (int j = 0; j < TM; j++) {
            const int m = m0 + wm * WTM + j * 32 + (lane & 31);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int n = n0 + wn * WTN + i * 32 + 8 * q + 4 * (lane >> 5);
                f16 *c = C + (long long)m * p.ldc + n;
                union { u32x2 w; f16 e[4]; } o, v;
                if (beta != 0.f) o.w = *reinterpret_cast<const u32x2 *>(c);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float x = alpha * acc[i][j][4 * q + e];
                    v.e[e] = (f16)(beta != 0.f ? __builtin_fmaf(beta, (float)o.e[e], x) : x);
                }
                *reinterpret_cast<u32x2 *>(c) = v.w;
            }
        }
}

}  // namespace hg
}  // namespace g9
