// FP16 GEMM kernel for gfx950 with direct global→LDS loads: C = alpha·op(A)·op(B) + beta·C, FP32 accumulation on
// v_mfma_f32_16x16x32_f16, result rounded once to FP16.
//
// Semantics are those of the reference's FP16 GEMM (reference: lib/kernels/hgemm.cl:838-898 hgemm_v / hgemm_kc_v,
// lib/kernels/hgemm.cl:558-564 gen9blas_epilog_b): every C element is the sum over k of the A·B products, then
// alpha·sum + beta·C in FP32 (C not read when beta = 0), rounded once to FP16. The MFMA accumulates in FP32, which
// gives both reference modes (FP16 chains, or FP32 partial sums every 32 products) at least their accuracy.
//
// This kernel serves products whose tiles are all full (M % BM = N % BN = K % KB = 0) with 16-byte aligned
// operands; the general FP16 kernel in gemm_kernel.h takes every other shape. Design:
// - the matrix-core instruction is v_mfma_f32_16x16x32_f16. It moves a quarter of the accumulator bytes per flop of
//   v_mfma_f32_32x32x16_f16 (4 instead of 16 FP32 per lane per instruction), and large FP16 products on random data
//   run at the board's power limit, so the energy per flop sets the rate: a loop of it sustains 1627 TFLOP/s on
//   MI355X against 1580 for the 32x32x16 form, and this kernel went from 1166-1176 to 1314-1324 TFLOP/s at n = 4096
//   (NN, sustained) when it moved from 32x32x16 to 16x16x32 tiles;
// - operand tiles go from global memory straight into LDS with global_load_lds_dwordx4 (no register staging, no
//   LDS write instructions): lane L of one instruction writes the 16 bytes at LDS offset base + 16·L, so each lane
//   is given the global address whose data belongs at that LDS position;
// - NS LDS stages of KB = 64 k each form a ring: the loads for k-step t+NS are issued as soon as stage t is free, so
//   a load has about NS-1 k-steps to arrive;
// - one barrier per k-step, placed before the last k32 substep: after it the wave issues the next stage's loads and
//   its first fragment reads, then runs the last substep's MFMAs, so neither the barrier nor the first LDS reads of
//   a k-step leave the matrix cores idle for long;
// - a k-contiguous operand (A not transposed, B transposed) is held as rows of KB k and read with ds_read_b128,
//   one 16-byte fragment per lane. Chunk c (k = 8c .. 8c+7) of row r sits at physical chunk c ^ kswz(r): the 16
//   lanes that one LDS cycle serves read 16 rows at one logical chunk, and the swizzle spreads them over all 64
//   banks;
// - an mn-contiguous operand (A transposed, B not transposed) is held as KB rows of k, each BM (or BN) elements
//   long, and read with ds_read_b64_tr_b16, which transposes 16-lane groups: lane j of a group reads 4 consecutive
//   mn of one k-row, and lane i receives the i-th mn of the group's reads for 4 k-rows. Chunk c of row k sits at
//   c ^ mnswz(k): 4·(k & 3) for rows of 128 or more mn, 4·((k >> 1) & 1) for rows of 64 (8 chunks, two k-rows per
//   256-byte bank row), so the four rows a group reads fall on distinct banks. A, when both operands are
//   mn-contiguous (TN), takes xor 2·((k >> 3) & 1) on top: then the two groups one LDS cycle serves (k-rows 8g + 0..3
//   and 8g + 8..11) read distinct banks too;
// - operands are swapped in the MFMA (the B fragment is the first input), so each lane ends with runs of 4
//   consecutive n of one row of C. n tiles come in pairs whose 16 fragment rows interleave in groups of 4 (rows
//   4q..4q+3 of the even tile are n 8q..8q+3 of the pair, of the odd tile n 8q+4..8q+7), so a lane's outputs of the
//   two tiles are 8 consecutive n: one 16-byte store, no lane exchange;
// - the workgroup → tile mapping gives each XCD a contiguous range of tiles, ordered in groups of 4 tile rows, so
//   one XCD's L2 serves the A and B panels its tiles share.
#pragma once
#include "internal.h"
#include "lds_dma.h"
#include <type_traits>

namespace g9 {
namespace hg {

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Physical chunk of logical chunk 0 in k-contiguous LDS row r (rows of KB k, CPRK chunks of 8 k): chunk c lives at
// c ^ kswz(r). 16 rows read together (16 consecutive rows, or the rows {0-3, 8-11, 16-19, 24-27} (+4) of a paired
// 16x16x32 fragment) land on distinct 16-byte bank groups; kswz(r + 32) = kswz(r).
template <int KB> __device__ __forceinline__ int kswz(int r) {
    constexpr int CPRK = KB / 8, RK = 128 / KB;
    return ((r / RK) ^ (((r >> 4) & 1) * (CPRK / 4))) % CPRK;
}

struct Params {
    const f16 *A, *B;
    f16 *C;
    long long lda, ldb, ldc, sA, sB, sC;
    int M, N, K, tiles_m, tiles_n;
    float alpha, beta;
};

// Global → LDS loads of one operand tile: RT rows (m or n) × KB k, RT·KB·2 bytes, issued by NW waves (counted in FP16
// elements; the FP32 kernel views its operands as FP16 pairs).
// KC: stored k-contiguous (element (mn, k) at X[mn·ld + k]); otherwise mn-contiguous (element (mn, k) at X[k·ld + mn]).
// MS: the mn-contiguous swizzle, chunk c of k-row k at c ^ mnswz<RT, false>(k) for the FP16 transposing reads
// (MS = 0), c ^ mnswz<RT, true>(k) for those of A in the TN layout (MS = 2), or at c ^ (8·((k >> 2) & 1)) for the
// FP32 reads of k-rows k and k + 4 by the two halves of a wave (MS = 1).
// Each lane's byte offset from the tile origin is fixed for the whole kernel; the wave-uniform origin advances.
// X3: xor 2·bit 3 of k as well, so that lane groups 0 and 1 of a transposing read (k-rows 8g + 0..3), which one LDS
// cycle serves together, use the two halves of the banks when each lane reads 8 bytes of 16 consecutive mn. Measured
// for A in the TN layout (n = 1024 365 → 387, n = 2048 812-828 → 843-850 TFLOP/s, n = 4096 the same); in TT
// (n = 4096 1321 → 1308) and for the paired n tiles of B, whose lanes read the first or the second 8 bytes of 4
// chunks, so that their groups share banks either way (NN n = 1024 401 → 393-395), it is not used.
template <int RT, bool X3 = false> __device__ __forceinline__ int mnswz(int k) {
    static_assert(RT >= 64, "an mn-contiguous row holds at least 8 chunks");
    return (RT >= 128 ? 4 * (k & 3) : 4 * ((k >> 1) & 1)) ^ (X3 ? 2 * ((k >> 3) & 1) : 0);
}
template <int RT, int KB, int NW, bool KC, int MS = 0>
struct Loader {
    static constexpr int NINST = RT * KB * 2 / 1024;       // 1 KiB instructions per tile
    static constexpr int NI = NINST / NW;                  // per wave
    static constexpr int CPRK = KB / 8, RPIK = 512 / KB, RK = 128 / KB;   // k-contiguous: chunks per row, rows per
                                                                          // instruction, rows per 256 bytes
    static constexpr int CPR = RT / 8, RPI = 512 / RT;                    // mn-contiguous: chunks per row, rows per
                                                                          // instruction
    static_assert(NINST % NW == 0, "tile instructions must divide over the waves");
    static_assert(!KC || (RPIK * NW) % 32 == 0, "k-contiguous swizzle must repeat over a wave's instructions");
    static_assert(KC || ((RT >= 128 || (RT == 64 && MS != 1)) && (RPI * NW) % (MS == 2 ? 16 : MS ? 8 : 4) == 0),
                  "mn-contiguous swizzle must repeat over a wave's instructions");
    const char *org;      // wave-uniform: tile origin at the next k-step to load
    unsigned voff;        // this lane's byte offset for instruction 0
    long long step_i;     // bytes between consecutive instructions of this wave
    long long step_k;     // bytes per k-step

    __device__ __forceinline__ void init(const f16 *X, long long ld, int mn0, int wave, int lane) {
        if constexpr (KC) {
            // instruction j = wave + NW·i covers rows RPIK·j ..; lane L: row RPIK·j + L / CPRK, physical chunk L % CPRK
            const int r = RPIK * wave + lane / CPRK;
            const int c = (lane % CPRK) ^ kswz<KB>(r);
            org = reinterpret_cast<const char *>(X + (long long)mn0 * ld);
            voff = (unsigned)(((long long)r * ld + 8 * c) * 2);
            step_i = (long long)RPIK * NW * ld * 2;
            step_k = KB * 2;
        } else {
            // instruction j covers k rows RPI·j ..; lane L: row RPI·j + L / CPR, physical chunk L % CPR
            const int k = RPI * wave + lane / CPR;
            const int c = (lane % CPR) ^ (MS == 1 ? 8 * ((k >> 2) & 1) : mnswz<RT, MS == 2>(k));
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

// Fragment reads of one operand for a wave's TT MFMA tiles (16 rows of m or n each, starting at wave row w0): per
// tile and k32 substep one 16-byte fragment per lane, row lane % 16 and k 8·(lane / 16) .. +7. PAIRED (the first MFMA
// input, n): tiles 2p and 2p+1 cover n 32p .. 32p+31 of the wave, fragment row r of tile t being n
// 32·(t/2) + 4·(t%2) + 8·(r/4) + r%4; otherwise row r of tile t is 16t + r.
template <int RT, int KB, int TT, bool KC, bool PAIRED, bool X3 = false>
struct Frags {
    static constexpr int NSUB = KB / 32;
    static constexpr int NOFF = KC ? 2 * NSUB : TT;
    unsigned off[NOFF];   // per-lane byte offsets: k-contiguous per tile parity and substep, else per tile
    __device__ __forceinline__ void init(int w0, int lane) {
        const int g = lane >> 4, i = lane & 15;
        if constexpr (KC) {
#pragma unroll
            for (int par = 0; par < 2; par++) {
                const int r = w0 + (PAIRED ? 4 * par + 8 * (i >> 2) + (i & 3) : 16 * par + i);   // + 32·(t/2)
                const int sw = kswz<KB>(r);
#pragma unroll
                for (int s = 0; s < NSUB; s++) off[par * NSUB + s] = r * (KB * 2) + (((4 * s + g) ^ sw) << 4);
            }
        } else {
            // ds_read_b64_tr_b16: in each 16-lane group (k group g), lane j reads 4 consecutive mn at k-row 8g + j/4
            // (+ 4 for the second read) from block P(j % 4); lane i then holds mn P(i/4) + i%4 of those 4 k-rows
            const int q = i >> 2, c = i & 3;
#pragma unroll
            for (int t = 0; t < TT; t++) {
                const int P = w0 + (PAIRED ? 32 * (t >> 1) + 4 * (t & 1) + 8 * c : 16 * t + 4 * c);
                // k-row 8g + q (+4, +32·s: the same swizzle)
                off[t] = (8 * g + q) * (RT * 2) + (((P >> 3) ^ mnswz<RT, X3>(8 * g + q)) << 4) + 2 * (P & 7);
            }
        }
    }
    // 16-byte fragment of tile t, substep s from the stage at `base`.
    __device__ __forceinline__ u32x4 read(const G9_LDS unsigned char *base, int t, int s) const {
        if constexpr (KC) {
            return *reinterpret_cast<const G9_LDS u32x4 *>(base + off[(t & 1) * NSUB + s] + (t >> 1) * 32 * (KB * 2));
        } else {
            const G9_LDS unsigned char *b = base + off[t] + 32 * s * (RT * 2);
            const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((G9_LDS i16x4 *)(b));                // k-rows +0..3
            const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((G9_LDS i16x4 *)(b + 4 * (RT * 2)));  // +4..7
            const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
            return u32x4{l2[0], l2[1], h2[0], h2[1]};
        }
    }
};

__device__ __forceinline__ f32x4 mma(u32x4 b, u32x4 a, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, b), __builtin_bit_cast(f16x8, a), c, 0, 0, 0);
}

// RA (read-ahead): the main loop reads each k-step's fragments one k-step early (for small wave tiles, whose few
// MFMAs per k-step cannot cover the LDS read latency inside the k-step).
template <int BM, int BN, int WM, int WN, int KB, int NS, bool AK, bool BKC, bool RA = false>
__global__ void __launch_bounds__(WM *WN * 64) hgemm_kernel(Params p) {
    constexpr int NW = WM * WN;
    constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 16, TN = WTN / 16;
    constexpr int ABYTES = BM * KB * 2, BBYTES = BN * KB * 2, SBYTES = ABYTES + BBYTES;
    constexpr int NSUB = KB / 32;
    constexpr bool AX3 = !AK && !BKC;   // TN: A's transposing reads take the bit-3 swizzle term
    using LA = Loader<BM, KB, NW, AK, AX3 ? 2 : 0>;
    using LB = Loader<BN, KB, NW, BKC>;
    constexpr int LPS = LA::NI + LB::NI;   // loads per stage per wave
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32 (n tiles come in pairs)");
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
    Frags<BM, KB, TM, AK, false, AX3> fa;
    Frags<BN, KB, TN, BKC, true> fb;
    fa.init(wm * WTM, lane);
    fb.init(wn * WTN, lane);

    f32x4 acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; i++)
#pragma unroll
        for (int j = 0; j < TM; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

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

    if constexpr (RA) {
        // Read-ahead: the fragments of a whole k-step are read one k-step before its MFMAs use them (two register
        // sets, alternating), so each k-step's LDS reads have all of the previous k-step's MFMAs to arrive. One
        // barrier per k-step, at its start: after it, k-step kt+1 is in LDS (every wave waited for its own loads
        // first) and every wave has finished reading k-step kt's stage (its reads were waited for), which then takes
        // the loads of k-step kt+NS. The k-step loop is unrolled by two so that the register sets are indexed by
        // constants.
        u32x4 fa2[2][NSUB][TM], fb2[2][NSUB][TN];
#pragma unroll
        for (int s = 0; s < NSUB; s++) {
#pragma unroll
            for (int j = 0; j < TM; j++) fa2[0][s][j] = fa.read(lds, j, s);
#pragma unroll
            for (int i = 0; i < TN; i++) fb2[0][s][i] = fb.read(lds + ABYTES, i, s);
        }
        constexpr int NMF = NSUB * TM * TN, NRD = NSUB * (TM + TN), NIT = NRD + LPS, PER = (NIT + NMF - 1) / NMF;
        int st = 0;   // stage holding k-step kt
        auto step = [&](auto cur_c, int kt) {
            constexpr int cur = decltype(cur_c)::value, nxt = cur ^ 1;
            const int nst = st + 1 == NS ? 0 : st + 1;
            wait_vm<(NS - 2) * LPS>();
            wait_lgkm0();
            __syncthreads();
            // the last k-step reads its successor's stage too (unused values, no branch in the schedule)
            const G9_LDS unsigned char *nx = lds + nst * SBYTES;
            const unsigned dsta = lds_addr + st * SBYTES, dstb = dsta + ABYTES;
#pragma unroll
            for (int t = 0; t < NMF; t++) {
                const int sub = t / (TM * TN), i = (t % (TM * TN)) / TM, j = t % TM;
                acc[i][j] = mma(fb2[cur][sub][i], fa2[cur][sub][j], acc[i][j]);
#pragma unroll
                for (int q = t * PER; q < (t + 1) * PER && q < NIT; q++) {   // reads in order of first use, then loads
                    if (q < NRD) {
                        const int rs = q / (TM + TN), w = q % (TM + TN);
                        if (w == 0) fb2[nxt][rs][0] = fb.read(nx + ABYTES, 0, rs);
                        else if (w <= TM) fa2[nxt][rs][w - 1] = fa.read(nx, w - 1, rs);
                        else fb2[nxt][rs][w - TM] = fb.read(nx + ABYTES, w - TM, rs);
                    } else if (q - NRD < LA::NI) {
                        la.one(q - NRD, dsta, wave);
                    } else {
                        lb.one(q - NRD - LA::NI, dstb, wave);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            const bool more = kt + NS + 1 < nk;   // the next issue loads k-step kt+NS+1, if it exists
            la.advance(more);
            lb.advance(more);
            st = nst;
        };
        for (int kt = 0; kt < nk; kt += 2) {
            step(std::integral_constant<int, 0>{}, kt);
            if (kt + 1 < nk) step(std::integral_constant<int, 1>{}, kt + 1);
        }
    } else {
        u32x4 ra[2][TM], rb[2][TN];
        auto read_frags = [&](const G9_LDS unsigned char *stg, int s, int buf) {
#pragma unroll
            for (int j = 0; j < TM; j++) ra[buf][j] = fa.read(stg, j, s);
#pragma unroll
            for (int i = 0; i < TN; i++) rb[buf][i] = fb.read(stg + ABYTES, i, s);
        };
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
                    acc[i][j] = mma(rb[s & 1][i], ra[s & 1][j], acc[i][j]);
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
            // the substep after the barrier runs at raised wave priority, so the MFMAs of the wave that leaves the
            // barrier first issue ahead of the other wave's (n = 4096 1343-1350 → 1356-1358, n = 2048 860-863 →
            // 869-872 TFLOP/s; raised before the barrier instead, or for the whole k-step: 1335-1348)
            __builtin_amdgcn_s_setprio(1);
            {
                constexpr int s = NSUB - 1;
                const G9_LDS unsigned char *nxt = lds + nst * SBYTES;
                const unsigned dsta = lds_addr + st * SBYTES, dstb = dsta + ABYTES;
                constexpr int NIT = NRF + NLD, PER = (NIT + NMF - 1) / NMF;
#pragma unroll
                for (int t = 0; t < NMF; t++) {
                    const int i = t / TM, j = t % TM;
                    acc[i][j] = mma(rb[s & 1][i], ra[s & 1][j], acc[i][j]);
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
            __builtin_amdgcn_s_setprio(0);
            st = nst;
        }
    }
    wait_vm<0>();   // the loads into stages nobody reads have landed before the wave ends

    // Epilogue. Lane l holds D[n][m] for m = lane % 16 of MFMA tile j and, in the n-tile pair p, n = 32p + 8·(l / 16)
    // + e from tile 2p (e = 0..3) and + 4 + e from tile 2p + 1: 8 consecutive n, one 16-byte store (alpha·acc +
    // beta·C in FP32, rounded once). The stores are non-temporal: C is not read again by this kernel, and every
    // workgroup stores its tile at about the same time at the end (n = 2048: 832 → 856 TFLOP/s, n = 4096:
    // 1330 → 1350, in alternating runs of both builds; the FP32 kernel's stores lose with it, 87.5 → 84.3 at
    // n = 1024).
    const float alpha = p.alpha, beta = p.beta;
    const int g = lane >> 4;
#pragma unroll
    for (int pp = 0; pp < TN / 2; pp++)
#pragma unroll
        for (int j = 0; j < TM; j++) {
            const int m = m0 + wm * WTM + j * 16 + (lane & 15);
            f16 *cp = C + (long long)m * p.ldc + n0 + wn * WTN + 32 * pp + 8 * g;
            union { u32x4 w; f16 e[8]; } o, v;
            if (beta != 0.f) o.w = *reinterpret_cast<const u32x4 *>(cp);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float x = alpha * acc[2 * pp + (e >> 2)][j][e & 3];
                v.e[e] = (f16)(beta != 0.f ? __builtin_fmaf(beta, (float)o.e[e], x) : x);
            }
            __builtin_nontemporal_store(v.w, reinterpret_cast<u32x4 *>(cp));
        }
}

}  // namespace hg
}  // namespace g9
