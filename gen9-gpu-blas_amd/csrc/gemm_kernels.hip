// Host side of the MFMA GEMM: tile configuration per type and dispatch over the transpose layouts.
// The kernel templates and their design notes are in gemm_kernel.h (every shape and type), hgemm_kernel.h (FP16,
// whole tiles, direct global→LDS loads) and sgemm_kernel.h (FP32, whole tiles, direct global→LDS loads).
#include "gemm_kernel.h"
#include "hgemm_kernel.h"
#include "sgemm_kernel.h"
#include <stdlib.h>
#include <string.h>
#include <algorithm>

namespace g9 {

// ---------------- host side ----------------
// Tile configurations, per element type and layout, from a sweep on MI355X at n = 4096 (every variant checked against
// a float64 reference). Big: the steady-state configuration. Small: smaller tiles for products whose big tiles
// would leave most of the 256 CUs idle.
//   FP16 256×256, 8 waves (4×2): NN 794, NT 950 TFLOP/s. FP64 256×128, 8 waves (4×2): 70.6 TFLOP/s.
//   FP32 with A k-contiguous: small tiles with 4 waves, many workgroups per CU. NN 64×128: 123 TFLOP/s at n = 4096,
//   117 at n = 2048 (256×128: 117 / 105; 128×128, 64×64, 128×64, 64×256 and 2- or 8-wave variants: 74-118). NT
//   64×64: 126 at n = 4096, 119 on the odd shape 3000×11008×4096 (128×128: 128 / 97, the odd shape's 2064 tiles
//   being four rounds of 512 workgroups and a nearly empty fifth). Transposed A: TN 128×128 125 (256×128: 117),
//   TT 128×64 120 (256×128: 117).
//   Small at n = 1024 (NN): FP32 64×64 (256 tiles, no split) 69 TFLOP/s against 62 for 128×128 split four ways;
//   FP64 64×128 split two ways 43, 64×64 41. Both are beaten by 64×64 tiles with two k groups (launch_layout).
struct TileCfg { int BM, BN, WM, WN; };
// Layouts whose staging needs more registers than a wave has at 2 waves per SIMD (transposed A, unaligned
// operands) keep FP16 at 4 waves (512 registers per wave), which compiles without spills.
template <class T, bool AK, bool BKC, bool VEC> struct Cfg;
// small_div: the small tile is taken when the big tiles times small_div are fewer than the CUs.
template <bool AK, bool BKC, bool VEC> struct Cfg<f16, AK, BKC, VEC> {
    static constexpr TileCfg big = (AK && VEC) ? TileCfg{256, 256, 4, 2} : TileCfg{256, 256, 2, 2};
    static constexpr TileCfg small{128, 128, 2, 2};
    static constexpr int small_div = 2;
};
template <bool AK, bool BKC, bool VEC> struct Cfg<float, AK, BKC, VEC> {
    static constexpr TileCfg big = !AK ? (BKC ? TileCfg{128, 64, 2, 2} : TileCfg{128, 128, 2, 2})
                                       : (BKC ? TileCfg{64, 64, 2, 2} : TileCfg{64, 128, 2, 2});
    static constexpr TileCfg small{64, 64, 2, 2};
    static constexpr int small_div = 1;
};
template <bool AK, bool BKC, bool VEC> struct Cfg<double, AK, BKC, VEC> {
    static constexpr TileCfg big{256, 128, 4, 2}, small{64, 128, 2, 2};
    static constexpr int small_div = 2;
};

// GEN9BLAS_SPLITK=n forces n split-K slices (0 or 1: none) and turns the two-k-group tiles off, so that the
// summation order no longer depends on the shape; -1 when unset.
static int splitk_forced() {
    static int forced = -2;
    if (forced == -2) {
        const char *e = getenv("GEN9BLAS_SPLITK");
        forced = e ? std::max(atoi(e), 0) : -1;
    }
    return forced;
}

// Split-K slices for a single product of `tiles` tiles: doubled while the slices still leave at most one workgroup
// per CU and each slice keeps at least 4 k-steps, up to 8. Without a forced split, s > 1 implies tiles · s ≤ CUs.
// Splitting changes only the FP32 (FP64) summation order: each slice sums its k-range, the slices are then added in
// order, and alpha/beta and the rounding to the element type are applied once.
static int splitk_slices(long long tiles, int K, int BK, int count) {
    const int forced = splitk_forced();
    if (count != 1) return 1;
    if (forced >= 0) return forced < 1 ? 1 : forced > 64 ? 64 : forced;
    int s = 1;
    while (s < 8 && tiles * s * 2 <= num_cus && K / (s * 2) >= 4 * BK) s *= 2;
    return s;
}

template <class T, TileCfg C, bool AK, bool BKC, bool VEC, int KG = 1>
static int launch_t(GemmParams<typename Mma<T>::Sum> p, int count) {
    using S = typename Mma<T>::Sum;
    constexpr int BK = 128 / (int)sizeof(T);
    p.tiles_m = (p.M + C.BM - 1) / C.BM;
    p.tiles_n = (p.N + C.BN - 1) / C.BN;
    if ((long long)p.tiles_m * p.tiles_n > 0x7fffffffLL || count > 65535)
        G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "gemm grid too large (%d × %d tiles, batch %d)", p.tiles_m, p.tiles_n, count);
    const long long tiles = (long long)p.tiles_m * p.tiles_n;
    const int split = KG > 1 ? 1 : splitk_slices(tiles, p.K, BK, count);
    const dim3 block(C.WM * C.WN * 64 * KG);
    if (split > 1) {
        static_assert((size_t)C.BM * C.BN * sizeof(S) <= SPLITK_TILE_BYTES_MAX, "split tile beyond the work-space bound");
        p.kper = ((p.K + split - 1) / split + BK - 1) / BK * BK;
        const int ns = (p.K + p.kper - 1) / p.kper;
        void *P;
        G9_TRY(scratch(SLOT_P, (size_t)ns * p.M * p.N * sizeof(S), &P));
        p.P = reinterpret_cast<S *>(P);
        p.vec_p = p.N % 4 == 0;
        hipLaunchKernelGGL((gemm_kernel<T, C.BM, C.BN, C.WM, C.WN, AK, BKC, VEC, true, true>), dim3((unsigned)tiles, (unsigned)ns),
                           block, 0, stream, p);
        G9_HIP(hipGetLastError());
        const long long mn = (long long)p.M * p.N;
        const bool v4 = p.vec_c && p.N % 4 == 0;
        const long long work = v4 ? mn / 4 : mn;
        const unsigned blocks = (unsigned)std::min<long long>((work + 255) / 256, (long long)num_cus * 8);
        T *Cp = reinterpret_cast<T *>(p.C);
        if (v4) hipLaunchKernelGGL((splitk_reduce<T, S, true>), dim3(blocks), dim3(256), 0, stream, p.P, Cp, p.ldc, p.M, p.N, ns, p.alpha, p.beta);
        else hipLaunchKernelGGL((splitk_reduce<T, S, false>), dim3(blocks), dim3(256), 0, stream, p.P, Cp, p.ldc, p.M, p.N, ns, p.alpha, p.beta);
        G9_HIP(hipGetLastError());
        return 0;
    }
    const dim3 grid((unsigned)tiles, (unsigned)count);
    hipLaunchKernelGGL((gemm_kernel<T, C.BM, C.BN, C.WM, C.WN, AK, BKC, VEC, true, false, 0, 0, KG>), grid, block, 0, stream, p);
    G9_HIP(hipGetLastError());
    return 0;
}

template <class T, bool AK, bool BKC, bool VEC>
static int launch_layout(const GemmParams<typename Mma<T>::Sum> &p, int count) {
    using CF = Cfg<T, AK, BKC, VEC>;
    const long long big_tiles = (long long)((p.M + CF::big.BM - 1) / CF::big.BM) * ((p.N + CF::big.BN - 1) / CF::big.BN) * count;
    if (big_tiles * CF::small_div < num_cus) {
        // 64×64 tiles with two k groups of 4 waves (8 waves per workgroup, the groups' sums added through LDS), when
        // they give at least num_cus / 2 tiles: two waves per SIMD hide each other's barrier and load waits without a
        // split-K pass. Measured (TFLOP/s, against the small tiles with split-K): FP32 NN n = 1024 71 → 82, TN 68 → 77,
        // n = 1000 38 → 56, 1024² × K 4096 81 → 98; FP64 n = 1024 44 → 52, n = 1536 38 → 48, 128×4096×128 (the
        // triangular solve's block products) 8.6 → 15.8. FP32 above num_cus tiles loses (n = 1280: 74 → 70), FP64
        // does not. Other FP64 shapes measured at n = 1024 / 1536 against 53.6 / 48.1: four k groups of 2×2 waves
        // 54.0 / 45.1, four of one 64×64 wave 41.9 / 34.9, two of 1×2 waves 48.7, four of 2×1 waves 51.1.
        // A batch (count > 1) cannot split K, so it takes these tiles from num_cus / 4 of them: FP64 128³ × 16 (the
        // triangular solve's 256-row compositions) 12.7 → 8.2 µs on 64 workgroups of 8 waves instead of 32 of 64×128,
        // DTRSM n = 4096 1.458 → 1.443 ms.
        if constexpr (sizeof(T) >= 4) {
            const long long t64 = (long long)((p.M + 63) / 64) * ((p.N + 63) / 64) * count;
            const long long need = count > 1 ? (num_cus + 3) / 4 : (num_cus + 1) / 2;
            if (splitk_forced() < 0 && t64 >= need && (sizeof(T) == 8 || t64 <= num_cus))
                return launch_t<T, TileCfg{64, 64, 2, 2}, AK, BKC, VEC, 2>(p, count);
        }
        return launch_t<T, CF::small, AK, BKC, VEC>(p, count);
    }
    // FP64 whose big tiles are exactly half the CUs (K would be split in two, with a reduction pass after): the small
    // tiles instead, when they fill the CUs. MI355X, µs (TFLOP/s): 1024×4096×1024 with beta = 1 (the triangular
    // solve's update of 1024 rows) 152.9 → 141.5 (56.2 → 60.7), 2048³ 268.4 → 258.3 (64.0 → 66.5); DTRSM n = 4096
    // 1.613 → 1.565 ms. 64×64 tiles with two k groups there: 142.8 and 265.9.
    if constexpr (sizeof(T) == 8) {
        const long long ts = (long long)((p.M + CF::small.BM - 1) / CF::small.BM) *
                             ((p.N + CF::small.BN - 1) / CF::small.BN) * count;
        if (splitk_forced() < 0 && count == 1 && big_tiles * 2 == num_cus && ts >= num_cus)
            return launch_t<T, CF::small, AK, BKC, VEC>(p, count);
    }
    // FP32 with B k-contiguous has 64×64 big tiles, so a product of exactly num_cus of them lands here: the same
    // two-k-group tiles (NT n = 1024)
    if constexpr (sizeof(T) == 4) {
        const long long t64 = (long long)((p.M + 63) / 64) * ((p.N + 63) / 64) * count;
        if (splitk_forced() < 0 && t64 * 2 >= num_cus && t64 <= num_cus)
            return launch_t<T, TileCfg{64, 64, 2, 2}, AK, BKC, VEC, 2>(p, count);
    }
    // FP32: 128×128 tiles with two k groups of 2×2 waves (64×64 per wave, 147 KiB of LDS: one workgroup per CU) when
    // their count fills whole rounds of num_cus workgroups (the last round at least 95 % full). Measured (TFLOP/s,
    // against the big tiles above): n = 4096 NN 123 → 125.5, TN 110 → 127.5, NT 123 → 132, n = 2048 NN 118 → 121.5;
    // the odd shape 3000×11008 (2064 tiles, nine rounds with a nearly empty last one) would fall from 117 to 97.
    if constexpr (sizeof(T) == 4) {
        const long long t128 = (long long)((p.M + 127) / 128) * ((p.N + 127) / 128) * count;
        const long long rounds = (t128 + num_cus - 1) / num_cus;
        if (splitk_forced() < 0 && t128 >= num_cus && t128 * 20 >= rounds * num_cus * 19)
            return launch_t<T, TileCfg{128, 128, 2, 2}, AK, BKC, VEC, 2>(p, count);
    }
    return launch_t<T, CF::big, AK, BKC, VEC>(p, count);
}

// ---------------- FP16 whole-tile kernel ----------------
// Configurations from sweeps on MI355X with N(0,1) FP16 inputs, timed after 1.5 s of the same load (the clock
// settles under the board's power limit; shorter runs see its ramp), every variant bit-exact on small integers:
// - products with at least one 256×256 tile per CU: 256×256 tiles, 8 waves of 128×64 (2×4), two stages of KB = 64.
//   n = 4096 NN 1314-1324 TFLOP/s (8 waves of 64×128: 1276-1286; 4 waves of 128×128: 1243-1246, at 2.03 GHz against
//   1.79-1.81; the same 8 waves on 32x32x16 MFMAs: 1166-1176); TN 1249, NT 1339, TT 1267 (32x32x16: 1180-1188);
// - at least one 128×128 tile per CU: 128×128, 8 waves of 64×32 (2×4), three stages. n = 2048 NN 835 (4 waves of
//   64×64 with 3 or 4 stages: 798-807; 32x32x16 tiles: 795), NT 845 (767), TN and TT 800-804 (800-802);
// - fewer 128×128 tiles than CUs, with A k-contiguous: 64×64 tiles (below); before them 32×128 tiles, 4 waves of
//   32×32, three stages, fragments read one k-step ahead: n = 1024 NN 385-386, NT 385 (reading inside the k-step:
//   369-371 and 363; four stages 359-370,
//   two 288-312; two k groups of 4 waves on separate rings, their sums added through LDS: 335-340; 32x32x16: 346).
//   Time per call against K at M = N = 1024 is about 2-3 µs plus 0.26 µs per k-step of 64 (8 MFMAs per wave), so
//   the k-step's latency chain (LDS reads, barrier), not its MFMAs, sets the rate; the read-ahead takes the LDS
//   reads off that chain.
//   At n = 2048 (128×128 tiles) the read-ahead gives nothing (841-849 against 849-853): that size runs at the power
//   limit (1.8-2.0 GHz).
// - the same small products on 64×64 tiles, 4 waves of 32×32, three stages, read-ahead: NT n = 1024 399.9 against
//   385.9 for 32×128 (four stages 390.6, two 303.6, no read-ahead 378.1); NN 400.7 against 382.8 (four stages 394.2),
//   its 64-wide mn-contiguous B rows swizzled by mnswz (hgemm_kernel.h). Per k-step a CU moves 16 KiB from L2 into
//   LDS instead of 20 KiB for the same flops; at n = 1024 the 256 CUs together pull about 20 TB/s.
template <int BM, int BN, int WM, int WN, int KB, int NS, bool AK, bool BKC, bool RA = false>
static int launch_hg(const hg::Params &p0, int count) {
    hg::Params p = p0;
    p.tiles_m = p.M / BM;
    p.tiles_n = p.N / BN;
    const dim3 grid((unsigned)(p.tiles_m * p.tiles_n), (unsigned)count), block(WM * WN * 64);
    hipLaunchKernelGGL((hg::hgemm_kernel<BM, BN, WM, WN, KB, NS, AK, BKC, RA>), grid, block, 0, stream, p);
    G9_HIP(hipGetLastError());
    return 0;
}
template <bool AK, bool BKC>
static int launch_hg_layout(const hg::Params &p, int count) {
    if ((long long)(p.M / 256) * (p.N / 256) * count >= num_cus && p.M % 256 == 0 && p.N % 256 == 0)
        return launch_hg<256, 256, 2, 4, 64, 2, AK, BKC>(p, count);
    // below one 128×128 tile per CU: 64×64 tiles, every layout. With A k-contiguous they move 20 % fewer L2 → LDS bytes
    // per flop than the 32×128 tiles of the same count (n = 1024 NN 382.8 → 400.7, NT 386 → 400 TFLOP/s); with A
    // transposed they replace 128×128 tiles, 64 of them for 256 CUs at n = 1024 (TN 212.6 → 365.5, TT 215.3 → 393.1)
    if ((long long)(p.M / 128) * (p.N / 128) * count < num_cus) return launch_hg<64, 64, 2, 2, 64, 3, AK, BKC, true>(p, count);
    return launch_hg<128, 128, 2, 4, 64, 3, AK, BKC>(p, count);
}
// The whole-tile FP16 kernel applies when every operand is 16-byte aligned with 16-byte row strides, M and N are
// multiples of 128, K of 64 (the k-step of every tile configuration), and the grid fits. GEN9BLAS_HGEMM=generic forces the general kernel.
static bool hgemm_tiles_apply(const GemmCall &c) {
    static int generic = -1;
    if (generic < 0) {
        const char *e = getenv("GEN9BLAS_HGEMM");
        generic = e && !strcmp(e, "generic");
    }
    if (generic || c.M % 128 || c.N % 128 || c.K % 64 || c.count > 65535) return false;
    const long long es = 2;
    // each lane's byte offset inside a 256-row (or 64-k-row) tile is 32-bit: rows of up to 8 Mi elements
    if (c.lda * es * 256 >= (1LL << 32) || c.ldb * es * 256 >= (1LL << 32)) return false;
    return (uintptr_t)c.A % 16 == 0 && (uintptr_t)c.B % 16 == 0 && (uintptr_t)c.C % 16 == 0 && (c.lda * es) % 16 == 0 &&
           (c.ldb * es) % 16 == 0 && (c.ldc * es) % 16 == 0 &&
           (c.count == 1 || ((c.sA * es) % 16 == 0 && (c.sB * es) % 16 == 0 && (c.sC * es) % 16 == 0));
}
static int launch_hgemm_tiles(const GemmCall &c) {
    hg::Params p;
    p.A = reinterpret_cast<const hg::f16 *>(c.A);
    p.B = reinterpret_cast<const hg::f16 *>(c.B);
    p.C = reinterpret_cast<hg::f16 *>(c.C);
    p.lda = c.lda; p.ldb = c.ldb; p.ldc = c.ldc;
    p.sA = c.sA; p.sB = c.sB; p.sC = c.sC;
    p.M = c.M; p.N = c.N; p.K = c.K;
    p.tiles_m = p.tiles_n = 0;
    p.alpha = (float)c.alpha;
    p.beta = (float)c.beta;
    const bool ak = !c.tA, bk = c.tB;
    if (ak && bk) return launch_hg_layout<true, true>(p, c.count);
    if (ak) return launch_hg_layout<true, false>(p, c.count);
    if (bk) return launch_hg_layout<false, true>(p, c.count);
    return launch_hg_layout<false, false>(p, c.count);
}

// ---------------- FP32 whole-tile kernel ----------------
// Classes, largest tile first; a product takes the first class whose whole tiles fill the CUs (128×128: twice over,
// else the 64×64 tiles of several rounds finish sooner: 2048³ 129 → 125 µs, 2048×2048×1024 68 → 66, the triangular
// solve's 1024×4096×1024 with beta = 1 70.3 → 67.1) and cover at least 90 % of C. Measured on MI355X (TFLOP/s,
// sustained, against the general kernel of gemm_kernel.h in the same runs):
// - 128×256 tiles, 8 waves of 64×64, two stages, sums blocked per 128 k: n = 4096 NN 144.9 (124.6), NT 144.3
//   (130.8); 8192×8192×2048 144.1 (123.4); 2944×11008×4096 NT β = 0.5 140.0 (127.9). Three stages 142.6, blocks of
//   32 k 134.3, of 64 k 140.3, of 256 k 142.6; 256×128 tiles 142.7;
// - 128×128 tiles, 8 waves of 64×32, three stages, 128-k blocks: n = 2048 134.4 (121.4; 4 waves of 64×64: 129.7;
//   64×64 tiles: 132.4; a later build read 133.0 against 137.2 for the 64×64 tiles, which n = 2048 now takes);
// - 64×64 tiles, 4 waves of 32×32, four stages, 256-k blocks: n = 1024 102.6 (87.7; 128-k blocks 101.9, 32-k blocks
//   90.9; three stages 94.0, six 93.0, eight 92.2).
// The rows and columns beyond the whole tiles (an M or N that is not a multiple of the tile) go to the general
// kernel, each C element still computed by exactly one of the launches; a bottom strip of r rows over a width that is
// a multiple of 64 instead takes 64×64 whole tiles on the last ⌈r/64⌉·64 rows, storing only its own r rows
// (3000×11008×4096 NT β = 0.5: 2.04 → 1.99 ms, the 56-row strip about 146 → 99 µs).
template <class T> static int launch_typed(const GemmCall &c);
struct SgClass { int BM, BN; };
static constexpr SgClass SG_CLASSES[] = {{128, 256}, {128, 128}, {64, 64}};
template <int BM, int BN, int WM, int WN, int NS, int BLK, bool AK, bool BKC>
static int launch_sg(const sg::Params &p0, int count) {
    sg::Params p = p0;
    p.tiles_m = p.M / BM;
    p.tiles_n = p.N / BN;
    const dim3 grid((unsigned)(p.tiles_m * p.tiles_n), (unsigned)count), block(WM * WN * 64);
    hipLaunchKernelGGL((sg::sgemm_kernel<BM, BN, WM, WN, NS, AK, BKC, BLK>), grid, block, 0, stream, p);
    G9_HIP(hipGetLastError());
    return 0;
}
template <bool AK, bool BKC>
static int launch_sg_layout(const sg::Params &p, int count, int cls) {
    if (cls == 0) return launch_sg<128, 256, 2, 4, 2, 4, AK, BKC>(p, count);
    if (cls == 1) return launch_sg<128, 128, 2, 4, 3, 4, AK, BKC>(p, count);
    return launch_sg<64, 64, 2, 2, 4, 8, AK, BKC>(p, count);
}
// The FP32 whole-tile kernel applies to 16-byte aligned operands with 16-byte row strides and K a multiple of 32,
// unless GEN9BLAS_SGEMM=generic or a forced split-K (GEN9BLAS_SPLITK) asks for the general kernel.
static bool sgemm_tiles_ok(const GemmCall &c) {
    static int generic = -1;
    if (generic < 0) {
        const char *e = getenv("GEN9BLAS_SGEMM");
        generic = e && !strcmp(e, "generic");
    }
    if (generic || splitk_forced() >= 0 || c.K % 32 || c.count > 65535) return false;
    const long long es = 4;
    // each lane's byte offset inside a tile is 32-bit
    if (c.lda * es * 256 >= (1LL << 32) || c.ldb * es * 256 >= (1LL << 32)) return false;
    return (uintptr_t)c.A % 16 == 0 && (uintptr_t)c.B % 16 == 0 && (uintptr_t)c.C % 16 == 0 && (c.lda * es) % 16 == 0 &&
           (c.ldb * es) % 16 == 0 && (c.ldc * es) % 16 == 0 &&
           (c.count == 1 || ((c.sA * es) % 16 == 0 && (c.sB * es) % 16 == 0 && (c.sC * es) % 16 == 0));
}
// Workgroups of KERN (threads each) that one CU holds at once, from the runtime's occupancy query (1 if it fails).
template <auto KERN> static int wgs_per_cu(int threads) {
    static const int occ = [threads] {
        int o = 0;
        return hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, KERN, threads, 0) == hipSuccess && o > 0 ? o : 1;
    }();
    return occ;
}
// k-limited tiles in the paired order: more tiles than CUs, all of them resident at once with two per CU (so that
// workgroups i and i + tiles / 2 run side by side on one CU, each long range beside a short one). With fewer per CU
// the later half starts as CUs free up, and the longest-first order balances better.
static int klim_pair(long long tiles, int per_cu) { return tiles > num_cus && tiles <= 2LL * num_cus && per_cu >= 2; }

// Triangle (TRI) and k-limited (KLIM) modes of the FP32 whole-tile kernel for SYRK / SYR2K / TRMM: one product,
// whole tiles (the callers check), `tiles` workgroups.
template <int BM, int BN, int WM, int WN, int NS, int BLK, bool AK, bool BKC, int TRI, int KLIM>
static int launch_sg_mode(const sg::Params &p0, long long tiles, int count = 1) {
    constexpr auto kern = sg::sgemm_kernel<BM, BN, WM, WN, NS, AK, BKC, BLK, TRI, KLIM>;
    sg::Params p = p0;
    p.tiles_m = p.M / BM;
    p.tiles_n = p.N / BN;
    if constexpr (KLIM != 0) p.kpair = count == 1 && klim_pair(tiles, wgs_per_cu<kern>(WM * WN * 64));
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles, (unsigned)count), dim3(WM * WN * 64), 0, stream, p);
    G9_HIP(hipGetLastError());
    return 0;
}
static sg::Params sg_params(const GemmCall &c) {
    sg::Params p;
    p.A = reinterpret_cast<const float *>(c.A);
    p.B = reinterpret_cast<const float *>(c.B);
    p.C = reinterpret_cast<float *>(c.C);
    p.lda = c.lda; p.ldb = c.ldb; p.ldc = c.ldc;
    p.sA = c.sA; p.sB = c.sB; p.sC = c.sC;
    p.M = c.M; p.N = c.N; p.K = c.K;
    p.tiles_m = p.tiles_n = 0;
    p.alpha = (float)c.alpha;
    p.beta = (float)c.beta;
    return p;
}
// Triangle of an FP32 square product on the whole-tile kernel (NT or TN): 128×128 or 64×64 tiles, whichever fills
// its last round of one workgroup per CU better (n = 4096: 528 tiles of 128×128 are 2.06 rounds, SYRK 90 TFLOP/s;
// 2080 of 64×64 fill 90 % of 9 rounds), when the triangle has at least one such tile per CU. Returns false (nothing
// launched) when neither applies; *rc is the launch's status otherwise.
template <int TRI, bool AK, bool BKC>
static bool sg_tri_layout(const GemmCall &c, int *rc) {
    const sg::Params p = sg_params(c);
    const long long t128 = (long long)(c.M / 128) * (c.M / 128 + 1) / 2, t64 = (long long)(c.M / 64) * (c.M / 64 + 1) / 2;
    const auto fill = [](long long t) { return (double)t / (double)(((t + num_cus - 1) / num_cus) * num_cus); };
    const bool ok128 = c.M % 128 == 0 && t128 >= num_cus, ok64 = c.M % 64 == 0 && t64 >= num_cus;
    if (ok128 && (!ok64 || fill(t128) >= fill(t64))) *rc = launch_sg_mode<128, 128, 2, 4, 3, 4, AK, BKC, TRI, 0>(p, t128);
    else if (ok64) *rc = launch_sg_mode<64, 64, 2, 2, 4, 8, AK, BKC, TRI, 0>(p, t64);
    else return false;
    return true;
}
static bool sg_tri(const GemmCall &c, bool lower, int *rc) {
    if (c.M != c.N || c.count != 1 || !sgemm_tiles_ok(c)) return false;
    if (!c.tA && c.tB) return lower ? sg_tri_layout<1, true, true>(c, rc) : sg_tri_layout<2, true, true>(c, rc);
    if (c.tA && !c.tB) return lower ? sg_tri_layout<1, false, false>(c, rc) : sg_tri_layout<2, false, false>(c, rc);
    return false;
}
// k-limited FP32 NN product (or strided batch of them) on the whole-tile kernel (TRMM, the triangular solves): the
// plain products' classes, whole tiles only. A batch takes the big classes only with two tiles per CU or more, so
// that tiles of long and short k ranges share the CUs (TRSV's E_q = inv(D_q)·C_q, 512³ × 31: 128×128 tiles 80 µs
// in a kernel trace; on 64×64 tiles the n = 16384 solve takes 385 against 400 µs).
template <int KLIM>
static bool sg_klim_mode(const GemmCall &c, int *rc) {
    const sg::Params p = sg_params(c);
    const long long t0 = (long long)(c.M / 128) * (c.N / 256), t1 = (long long)(c.M / 128) * (c.N / 128),
                    t2 = (long long)(c.M / 64) * (c.N / 64), nb = c.count;
    const long long want = nb > 1 ? 2LL * num_cus : num_cus;
    if (c.M % 128 == 0 && c.N % 256 == 0 && t0 * nb >= want)
        *rc = launch_sg_mode<128, 256, 2, 4, 2, 4, true, false, 0, KLIM>(p, t0, c.count);
    else if (c.M % 128 == 0 && c.N % 128 == 0 && t1 * nb >= want)
        *rc = launch_sg_mode<128, 128, 2, 4, 3, 4, true, false, 0, KLIM>(p, t1, c.count);
    else if (c.M % 64 == 0 && c.N % 64 == 0 && t2 * nb >= num_cus)
        *rc = launch_sg_mode<64, 64, 2, 2, 4, 8, true, false, 0, KLIM>(p, t2, c.count);
    else return false;
    return true;
}
static bool sg_klim(const GemmCall &c, int klim, int *rc) {
    // the k range of every tile is non-empty only when K spans the triangular operand's order
    if (c.count < 1 || c.tA || c.tB || !sgemm_tiles_ok(c) || (klim <= 2 ? c.K != c.M : c.K != c.N)) return false;
    switch (klim) {
    case 1: return sg_klim_mode<1>(c, rc);
    case 2: return sg_klim_mode<2>(c, rc);
    case 3: return sg_klim_mode<3>(c, rc);
    case 4: return sg_klim_mode<4>(c, rc);
    }
    return false;
}

// The part of an FP32 product in rows [m0, m0 + M) and columns [n0, n0 + N) of C, as a product of its own.
static GemmCall sub_call(const GemmCall &c, int m0, int M, int n0, int N) {
    GemmCall s = c;
    const float *A = reinterpret_cast<const float *>(c.A), *B = reinterpret_cast<const float *>(c.B);
    s.A = A + (c.tA ? (long long)m0 : (long long)m0 * c.lda);
    s.B = B + (c.tB ? (long long)n0 * c.ldb : (long long)n0);
    s.C = reinterpret_cast<float *>(c.C) + (long long)m0 * c.ldc + n0;
    s.M = M;
    s.N = N;
    return s;
}
static int launch_sgemm(const GemmCall &c) {
    if (!sgemm_tiles_ok(c)) return launch_typed<float>(c);
    int cls = -1, Mi = 0, Ni = 0;
    for (int k = 0; k < 3 && cls < 0; k++) {
        const int mi = c.M / SG_CLASSES[k].BM * SG_CLASSES[k].BM, ni = c.N / SG_CLASSES[k].BN * SG_CLASSES[k].BN;
        const long long tiles = (long long)(mi / SG_CLASSES[k].BM) * (ni / SG_CLASSES[k].BN) * c.count;
        if (tiles >= (k == 1 ? 2LL : 1LL) * num_cus && tiles <= 0x7fffffffLL && (double)mi * ni >= 0.9 * (double)c.M * c.N) {
            cls = k;
            Mi = mi;
            Ni = ni;
        }
    }
    if (cls < 0) return launch_typed<float>(c);
    sg::Params p;
    p.A = reinterpret_cast<const float *>(c.A);
    p.B = reinterpret_cast<const float *>(c.B);
    p.C = reinterpret_cast<float *>(c.C);
    p.lda = c.lda; p.ldb = c.ldb; p.ldc = c.ldc;
    p.sA = c.sA; p.sB = c.sB; p.sC = c.sC;
    p.M = Mi; p.N = Ni; p.K = c.K;
    p.tiles_m = p.tiles_n = 0;
    p.alpha = (float)c.alpha;
    p.beta = (float)c.beta;
    const bool ak = !c.tA, bk = c.tB;
    if (ak && bk) G9_TRY((launch_sg_layout<true, true>(p, c.count, cls)));
    else if (ak) G9_TRY((launch_sg_layout<true, false>(p, c.count, cls)));
    else if (bk) G9_TRY((launch_sg_layout<false, true>(p, c.count, cls)));
    else G9_TRY((launch_sg_layout<false, false>(p, c.count, cls)));
    if (Ni < c.N) G9_TRY(launch_typed<float>(sub_call(c, 0, Mi, Ni, c.N - Ni)));   // right strip
    if (Mi < c.M) {   // bottom strip, full width
        const int r = c.M - Mi, Ms = (r + 63) / 64 * 64;
        // shifted 64×64 whole tiles when the width is whole 64-column tiles and the shift keeps A 16-byte aligned
        if (Ni == c.N && c.N % 64 == 0 && Ms <= c.M && (!c.tA || (c.M - Ms) % 4 == 0)) {
            const GemmCall sc = sub_call(c, c.M - Ms, Ms, 0, c.N);
            sg::Params ps = p;
            ps.A = reinterpret_cast<const float *>(sc.A);
            ps.C = reinterpret_cast<float *>(sc.C);
            ps.M = Ms;
            ps.N = c.N;
            ps.m_skip = Ms - r;
            ps.tiles_m = Ms / 64;
            ps.tiles_n = c.N / 64;
            const dim3 grid((unsigned)(ps.tiles_m * ps.tiles_n), (unsigned)c.count), block(256);
            if (ak && bk) hipLaunchKernelGGL((sg::sgemm_kernel<64, 64, 2, 2, 4, true, true, 8, 0, 0, true>), grid, block, 0, stream, ps);
            else if (ak) hipLaunchKernelGGL((sg::sgemm_kernel<64, 64, 2, 2, 4, true, false, 8, 0, 0, true>), grid, block, 0, stream, ps);
            else if (bk) hipLaunchKernelGGL((sg::sgemm_kernel<64, 64, 2, 2, 4, false, true, 8, 0, 0, true>), grid, block, 0, stream, ps);
            else hipLaunchKernelGGL((sg::sgemm_kernel<64, 64, 2, 2, 4, false, false, 8, 0, 0, true>), grid, block, 0, stream, ps);
            G9_HIP(hipGetLastError());
        } else {
            G9_TRY(launch_typed<float>(sub_call(c, Mi, r, 0, c.N)));
        }
    }
    return 0;
}

template <class T>
static int launch_typed(const GemmCall &c) {
    using S = typename Mma<T>::Sum;
    GemmParams<S> p;
    p.A = c.A; p.B = c.B; p.C = c.C;
    p.lda = c.lda; p.ldb = c.ldb; p.ldc = c.ldc;
    p.sA = c.sA; p.sB = c.sB; p.sC = c.sC;
    p.M = c.M; p.N = c.N; p.K = c.K;
    p.alpha = (S)c.alpha;
    p.beta = (S)c.beta;
    p.tiles_m = p.tiles_n = 0;
    p.P = nullptr;
    p.kper = p.vec_p = 0;
    const long long es = sizeof(T);
    const long long cal = es * 4 < 16 ? es * 4 : 16;   // alignment of a 4-element group of C
    p.vec_c = ((uintptr_t)c.C % cal == 0) && (c.ldc * es) % cal == 0 && (c.count == 1 || (c.sC * es) % cal == 0);
    const bool vec = ((uintptr_t)c.A % 16 == 0) && ((uintptr_t)c.B % 16 == 0) && (c.lda * es) % 16 == 0 &&
                     (c.ldb * es) % 16 == 0 && (c.count == 1 || ((c.sA * es) % 16 == 0 && (c.sB * es) % 16 == 0));
    const bool ak = !c.tA, bk = c.tB;   // k-contiguous A: not transposed; k-contiguous B: transposed (stored N×K)
    const int sel = (ak ? 4 : 0) | (bk ? 2 : 0) | (vec ? 1 : 0);
    switch (sel) {
    case 0: return launch_layout<T, false, false, false>(p, c.count);
    case 1: return launch_layout<T, false, false, true>(p, c.count);
    case 2: return launch_layout<T, false, true, false>(p, c.count);
    case 3: return launch_layout<T, false, true, true>(p, c.count);
    case 4: return launch_layout<T, true, false, false>(p, c.count);
    case 5: return launch_layout<T, true, false, true>(p, c.count);
    case 6: return launch_layout<T, true, true, false>(p, c.count);
    default: return launch_layout<T, true, true, true>(p, c.count);
    }
}

// Triangle of a square product (SYRK, SYR2K): alpha·op(A)·op(B) + beta·C written on the lower (upper) triangle of C
// only. One launch over the T(T+1)/2 square tiles that meet the triangle (T tiles per side), diagonal tiles masked per
// element, each C element rounded once; the two layouts those routines use: A and B both k-contiguous, or both
// mn-contiguous. FP32 and FP64 take 64×64 tiles: at n = 4096 their 2080 tiles keep every CU busy to the end (FP32
// SYRK 0.71 ms, FP64 1.21), where 128×128 tiles (528) left a nearly empty last round (1.02, 1.58).
template <class T, int TRI, bool AK, bool BKC, bool VEC>
static int launch_tri_t(GemmParams<typename Mma<T>::Sum> p) {
    constexpr TileCfg C = sizeof(T) == 2 ? TileCfg{128, 128, 2, 2} : TileCfg{64, 64, 2, 2};
    p.tiles_m = p.tiles_n = (p.M + C.BM - 1) / C.BM;
    const long long tiles = (long long)p.tiles_m * (p.tiles_m + 1) / 2;
    if (tiles > 0x7fffffffLL) G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "triangle product too large (%d tiles per side)", p.tiles_m);
    hipLaunchKernelGGL((gemm_kernel<T, C.BM, C.BN, C.WM, C.WN, AK, BKC, VEC, true, false, TRI>), dim3((unsigned)tiles),
                       dim3(C.WM * C.WN * 64), 0, stream, p);
    G9_HIP(hipGetLastError());
    return 0;
}
template <class T, bool AK, bool BKC>
static int launch_tri_layout(const GemmParams<typename Mma<T>::Sum> &p, bool vec, bool lower) {
    if (vec) return lower ? launch_tri_t<T, 1, AK, BKC, true>(p) : launch_tri_t<T, 2, AK, BKC, true>(p);
    return lower ? launch_tri_t<T, 1, AK, BKC, false>(p) : launch_tri_t<T, 2, AK, BKC, false>(p);
}
template <class T>
static int launch_tri_typed(const GemmCall &c, bool lower) {
    using S = typename Mma<T>::Sum;
    GemmParams<S> p;
    p.A = c.A; p.B = c.B; p.C = c.C;
    p.lda = c.lda; p.ldb = c.ldb; p.ldc = c.ldc;
    const bool batch = c.count > 1;
    p.sA = batch ? c.sA : 0; p.sB = batch ? c.sB : 0; p.sC = batch ? c.sC : 0;
    p.M = c.M; p.N = c.N; p.K = c.K;
    p.alpha = (S)c.alpha;
    p.beta = (S)c.beta;
    p.tiles_m = p.tiles_n = 0;
    p.P = nullptr;
    p.kper = p.vec_p = 0;
    const long long es = sizeof(T);
    const long long cal = es * 4 < 16 ? es * 4 : 16;
    p.vec_c = ((uintptr_t)c.C % cal == 0) && (c.ldc * es) % cal == 0 && (p.sC * es) % cal == 0;
    const bool vec = ((uintptr_t)c.A % 16 == 0) && ((uintptr_t)c.B % 16 == 0) && (c.lda * es) % 16 == 0 && (c.ldb * es) % 16 == 0 &&
                     (p.sA * es) % 16 == 0 && (p.sB * es) % 16 == 0;
    if (!c.tA && c.tB) return launch_tri_layout<T, true, true>(p, vec, lower);
    if (c.tA && !c.tB) return launch_tri_layout<T, false, false>(p, vec, lower);
    G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "triangle product: layout tA=%d tB=%d", c.tA, c.tB);
}
int launch_gemm_tri(const GemmCall &c, bool lower) {
    if (c.M != c.N || c.count != 1) G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "triangle product: %d×%d, batch %d", c.M, c.N, c.count);
    switch (c.type) {
    case GEN9BLAS_H:
    case GEN9BLAS_HS: return launch_tri_typed<f16>(c, lower);
    case GEN9BLAS_S: {
        int rc = 0;
        return sg_tri(c, lower, &rc) ? rc : launch_tri_typed<float>(c, lower);
    }
    case GEN9BLAS_D: return launch_tri_typed<double>(c, lower);
    }
    G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "type %d unavailable", c.type);
}

// Product with a triangular operand (TRMM on the explicit triangular matrix, TRSM's leaf products): each tile's k
// range is cut to where the triangle is non-zero (klim as gemm_kernel's KLIM), one launch over every tile of C,
// longest ranges dispatched first; the small tiles when the big ones are fewer than the CUs. Layout NN only (both
// operands as stored), one product.
template <class T, TileCfg C, int KLIM, bool VEC>
static int launch_klim_t(GemmParams<typename Mma<T>::Sum> p, int count) {
    p.tiles_m = (p.M + C.BM - 1) / C.BM;
    p.tiles_n = (p.N + C.BN - 1) / C.BN;
    const long long tiles = (long long)p.tiles_m * p.tiles_n;
    if (tiles > 0x7fffffffLL) G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "gemm grid too large (%d × %d tiles)", p.tiles_m, p.tiles_n);
    constexpr auto kern = gemm_kernel<T, C.BM, C.BN, C.WM, C.WN, true, false, VEC, true, false, 0, KLIM>;
    p.kpair = count == 1 && klim_pair(tiles, wgs_per_cu<kern>(C.WM * C.WN * 64));
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles, (unsigned)count), dim3(C.WM * C.WN * 64), 0, stream, p);
    G9_HIP(hipGetLastError());
    return 0;
}
template <class T>
static int launch_klim_typed(const GemmCall &c, int klim) {
    using S = typename Mma<T>::Sum;
    GemmParams<S> p;
    p.A = c.A; p.B = c.B; p.C = c.C;
    p.lda = c.lda; p.ldb = c.ldb; p.ldc = c.ldc;
    const bool batch = c.count > 1;
    p.sA = batch ? c.sA : 0; p.sB = batch ? c.sB : 0; p.sC = batch ? c.sC : 0;
    p.M = c.M; p.N = c.N; p.K = c.K;
    p.alpha = (S)c.alpha;
    p.beta = (S)c.beta;
    p.tiles_m = p.tiles_n = 0;
    p.P = nullptr;
    p.kper = p.vec_p = 0;
    const long long es = sizeof(T);
    const long long cal = es * 4 < 16 ? es * 4 : 16;
    p.vec_c = ((uintptr_t)c.C % cal == 0) && (c.ldc * es) % cal == 0 && (p.sC * es) % cal == 0;
    const bool vec = ((uintptr_t)c.A % 16 == 0) && ((uintptr_t)c.B % 16 == 0) && (c.lda * es) % 16 == 0 && (c.ldb * es) % 16 == 0 &&
                     (p.sA * es) % 16 == 0 && (p.sB * es) % 16 == 0;
    // tile class: FP16 the big tiles when they are at least the CUs; FP32 / FP64 the first of big, small and (FP64)
    // 64×64 that makes two workgroups per CU or more, so that long and short k ranges can share the CUs
    const auto by_cfg = [&](auto vc) -> int {
        constexpr bool V = decltype(vc)::value;
        using CF = Cfg<T, true, false, V>;
        constexpr TileCfg tiny{64, 64, 2, 2};
        const auto ntiles = [&](TileCfg t) {
            return (long long)((c.M + t.BM - 1) / t.BM) * ((c.N + t.BN - 1) / t.BN) * c.count;
        };
        constexpr bool half = sizeof(T) == 2, dbl = sizeof(T) == 8;
        const long long want = half ? num_cus : 2LL * num_cus;
        const int cls = ntiles(CF::big) >= want ? 0 : (!dbl || ntiles(CF::small) >= want) ? 1 : 2;
        const auto go = [&](auto kc) -> int {
            constexpr int K = decltype(kc)::value;
            if (cls == 0) return launch_klim_t<T, CF::big, K, V>(p, c.count);
            if constexpr (dbl) {
                if (cls == 2) return launch_klim_t<T, tiny, K, V>(p, c.count);
            }
            return launch_klim_t<T, CF::small, K, V>(p, c.count);
        };
        switch (klim) {
        case 1: return go(std::integral_constant<int, 1>());
        case 2: return go(std::integral_constant<int, 2>());
        case 3: return go(std::integral_constant<int, 3>());
        case 4: return go(std::integral_constant<int, 4>());
        }
        G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "k-limited product: mode %d", klim);
    };
    return vec ? by_cfg(std::true_type()) : by_cfg(std::false_type());
}
int launch_gemm_klim(const GemmCall &c, int klim) {
    if (c.tA || c.tB || c.count < 1) G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "k-limited product: layout tA=%d tB=%d, batch %d", c.tA, c.tB, c.count);
    switch (c.type) {
    case GEN9BLAS_H:
    case GEN9BLAS_HS: return launch_klim_typed<f16>(c, klim);
    case GEN9BLAS_S: {
        int rc = 0;
        return sg_klim(c, klim, &rc) ? rc : launch_klim_typed<float>(c, klim);
    }
    case GEN9BLAS_D: return launch_klim_typed<double>(c, klim);
    }
    G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "type %d unavailable", c.type);
}

int launch_gemm(const GemmCall &c) {
    switch (c.type) {
    case GEN9BLAS_H:
    case GEN9BLAS_HS: return hgemm_tiles_apply(c) ? launch_hgemm_tiles(c) : launch_typed<f16>(c);
    case GEN9BLAS_S: return launch_sgemm(c);
    case GEN9BLAS_D: return launch_typed<double>(c);
    }
    G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "type %d unavailable", c.type);
}

}  // namespace g9
