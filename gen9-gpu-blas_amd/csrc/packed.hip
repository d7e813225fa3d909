// Packed B kept on the GPU: gen9blas_pack_b / gen9blas_gemm_pb / gen9blas_packed_b_free.
//
// Contract of the reference (reference: lib/src/packed.c:70-89 pack_b, :168-172 packed_b_free, :174-213 gemm_pb):
// pack_b copies op(B) (K×N; transB: B stored N×K) once into memory the library owns, so that later products
// C = alpha·op(A)·Bp + beta·C do not move B again; the original B may change or go away after packing. A type or
// size error returns NULL with the status set; gemm_pb on NULL returns INVALID_ARG; packed_b_free waits for queued
// work before releasing the buffer.
//
// MI355X layout: the packed form is op(B)ᵀ, an N×K row-major matrix in device memory whose rows start 128-byte
// aligned (leading dimension K rounded up to 64 elements, the padding zero-filled). It is the layout both hot kernels
// read fastest: the skinny kernels stream weight rows k-contiguous (so gemm_pb with M ≤ 16 is a decode step on
// resident weights), and it is the k-contiguous B ("NT") of the whole-tile FP16 kernel. gemm_pb is then gen9blas_gemm
// with transB = 1 on that matrix. The reference's padded tile layouts, packing bands and spare-buffer pool answer
// i915 constraints (page zeroing, preemption) that do not exist here.
#include "internal.h"
#include "gen9blas_ml.h"
#include "lds_dma.h"
#include "wave.h"
#include <new>

struct gen9blas_packed_b {
    int type;
    int K, N;
    long long ld;   // row stride of the packed N×K matrix (elements)
    void *buf;      // device memory, N·ld elements
};

namespace g9 {

// P[n][k] = op(B)[k][n] for k < K and 0 for K ≤ k < ld. Tiles of 32 n × 32 k through LDS; a block of 32×8 threads.
// transB: B is N×K (P is a row copy); otherwise B is K×N and the tile is transposed on its way through LDS.
template <class T>
__global__ void __launch_bounds__(256) pack_bt_kernel(const T *__restrict__ B, long long ldb, int transB, int K, int N,
                                                      T *__restrict__ P, long long ld) {
    __shared__ T tile[32][33];
    const int tx = threadIdx.x, ty = threadIdx.y;
    const long long k0 = (long long)blockIdx.x * 32, n0 = (long long)blockIdx.y * 32;
    for (int r = ty; r < 32; r += 8) {
        if (transB) {   // row n0 + r of B, k0 + tx
            const long long n = n0 + r, k = k0 + tx;
            tile[r][tx] = (n < N && k < K) ? B[n * ldb + k] : T(0);
        } else {        // row k0 + r of B, n0 + tx
            const long long k = k0 + r, n = n0 + tx;
            tile[tx][r] = (n < N && k < K) ? B[k * ldb + n] : T(0);
        }
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const long long n = n0 + r, k = k0 + tx;
        if (n < N && k < ld) P[n * ld + k] = tile[r][tx];
    }
}

// ---------------- small batches on packed FP16 weights with FP32 activations ----------------
// C (M×N) = A (M×K) · Bpᵀ for M ≤ 16 with FP32 activations, FP32 products and sums, FP32 result (reference:
// lib/src/packed.c:307-329, lib/kernels/hgemm.cl:1392-1436). On the VALU every 16 bytes of weights would cost 8·M FP32
// FMAs, more than the weight stream leaves time for at M = 16; the FP32 matrix cores take the product instead
// (FP16 → FP32 is exact, products and sums are FP32). A workgroup of SPW waves owns 16 weight rows and its waves
// split K in steps of 32. In a step lane l loads 16 bytes of weight row n0 + l%16 (8 k from 8·(l/16)) and the same 8 k
// of activation row l%16 (zero past M or K); 8 v_mfma_f32_16x16x4_f32 add the step to
// the wave's 16×16 accumulators, MFMA e taking k = 8·q + e from lane group q (each k of the step once) into chain
// e % 4 (four independent chains keep the matrix cores busy). A lane then holds D[4·q + r][n0 + l%16], r = 0..3.
// The chains are added, the waves' sums added in LDS in wave order, and wave 0 writes C, setting *flag for a
// non-finite result.
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4p __attribute__((ext_vector_type(4)));
constexpr int SPW = 16;  // waves per workgroup
constexpr int SPB = 8;   // steps per batch: all their loads are issued before the first MFMA
__global__ void __launch_bounds__(SPW * 64) skinny_pb_kernel(int M, int N, int K, const float *__restrict__ A,
                                                             long long lda, int avec, const _Float16 *__restrict__ W,
                                                             long long ldw, int spw, float *__restrict__ C,
                                                             long long ldc, int *flag) {
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i = lane & 15, q = lane >> 4, n = blockIdx.x * 16 + i;
    const bool wrow = n < N, arow = i < M;
    const _Float16 *wr = W + (long long)(wrow ? n : 0) * ldw;
    const float *ar = A + (long long)(arow ? i : 0) * lda;
    floatx4 acc[4];   // four independent chains of MFMAs, added at the end
#pragma unroll
    for (int c = 0; c < 4; c++) acc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int s0 = w * spw;
    for (int sb = s0; sb < s0 + spw; sb += SPB) {
        u32x4p wq[SPB];
        float av[SPB][8];
#pragma unroll
        for (int b = 0; b < SPB; b++) {
            const int k = (sb + b) * 32 + 8 * q;
            const u32x4p z = {0u, 0u, 0u, 0u};
            // packed rows hold ldw ≥ K elements (zeros past K, ldw a multiple of 64): k < ldw keeps k + 7 inside
            wq[b] = wrow && k < ldw ? *reinterpret_cast<const u32x4p *>(wr + k) : z;
            if (avec && arow && k + 8 <= K) {
                const u32x4p a0 = *reinterpret_cast<const u32x4p *>(ar + k);
                const u32x4p a1 = *reinterpret_cast<const u32x4p *>(ar + k + 4);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const unsigned x0 = a0[e], x1 = a1[e];
                    av[b][e] = __builtin_bit_cast(float, x0);
                    av[b][e + 4] = __builtin_bit_cast(float, x1);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) av[b][e] = arow && k + e < K ? ar[k + e] : 0.f;
            }
        }
#pragma unroll
        for (int b = 0; b < SPB; b++) {
            float we[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const unsigned h2 = wq[b][e / 2];
                const unsigned short h = e % 2 ? (unsigned short)(h2 >> 16) : (unsigned short)(h2 & 0xffffu);
                we[e] = (float)__builtin_bit_cast(_Float16, h);
            }
#pragma unroll
            for (int e = 0; e < 8; e++) acc[e % 4] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[b][e], we[e], acc[e % 4], 0, 0, 0);
        }
    }
    __shared__ float part[SPW][4][64];
#pragma unroll
    for (int r = 0; r < 4; r++) part[w][r][lane] = (acc[0][r] + acc[1][r]) + (acc[2][r] + acc[3][r]);
    __syncthreads();
    if (w != 0 || !wrow) return;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int m = 4 * q + r;
        if (m >= M) continue;
        float t = part[0][r][lane];
#pragma unroll
        for (int v = 1; v < SPW; v++) t += part[v][r][lane];
        C[(long long)m * ldc + n] = t;
        if (!__builtin_isfinite(t)) *flag = 1;   // every writer stores the same value
    }
}

// The same product with the weight and activation tiles streamed through LDS (K % GK == 0, 16-byte aligned
// activation rows): a workgroup of SKS waves owns 16 weight rows; its waves take groups of GK = 64 or 128 k round
// robin, and each wave streams its groups through a private NSP-stage LDS ring with global_load_lds_dwordx4: per group
// 16·GK·2 / 1024 copies of 1 KiB bring 16 weight rows × 2·GK bytes (1024 / (2·GK) rows per copy, contiguous in
// memory) and ⌈MT / rows per copy⌉ copies bring MT activation rows × 4·GK bytes. Chunk c (16 bytes) of weight row r
// sits at position c ^ wsw(r), wsw(r) = (r / rows per 256 bytes) mod chunks per row, and of activation row r at
// c ^ (r % 16), so the 16 lanes that read one chunk of 16 rows hit distinct banks. Per 32 k, lane (i = l%16, q = l/16)
// reads 8 FP16 weights of row n0 + i and 8 FP32 activations of row i at k = 8·q .. 8·q+7, and 8
// v_mfma_f32_16x16x4_f32 add them (MFMA e takes k = 8·q + e from lane group q) into chain e % 4 of four independent
// chains. A wave reads only what it copied itself, so no barrier is needed until the waves' 16×16 sums are added in
// LDS in wave order. The 64-k groups halve a stage, so 8 waves (two per SIMD, hiding each other's ring and LDS waits)
// with three stages fit beside 16 activation rows.
template <int MT, int SKS, int NSP, int GK = 128>
__global__ void __launch_bounds__(SKS * 64) skinny_pb_lds_kernel(int M, int N, int K, const float *__restrict__ A,
                                                                 long long lda, const _Float16 *__restrict__ W,
                                                                 long long ldw, float *__restrict__ C, long long ldc,
                                                                 int *flag) {
    static_assert(GK == 64 || GK == 128, "groups of 64 or 128 k");
    constexpr int WROW = GK * 2, AROW = GK * 4;               // bytes of a weight / activation row per group
    constexpr int CPR = WROW / 16, RPC = 1024 / WROW, RPB = 256 / WROW;   // weight chunks per row, rows per copy,
                                                                          // rows per 256 bytes
    constexpr int CPRA = AROW / 16, RPCA = 1024 / AROW;
    constexpr int NWC = 16 / RPC, NAC = (MT + RPCA - 1) / RPCA;   // copies per group
    constexpr int NSUB = GK / 32;
    constexpr int WB = 16 * WROW, SB = WB + NAC * 1024, LPG = NWC + NAC;
    static_assert((NSP - 1) * LPG < 64, "copies in flight must fit vmcnt");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[SKS * NSP * SB];
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i = lane & 15, q = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const unsigned lbase = (unsigned)(uintptr_t)smem + wv * NSP * SB;
    const G9_LDS unsigned char *lds = (const G9_LDS unsigned char *)smem + wv * NSP * SB;
    const int G = K / GK, ng = G > wv ? (G - wv + SKS - 1) / SKS : 0;
    auto wsw = [](int r) { return (r / RPB) % CPR; };
    // weight copy c: row RPC·c + L / CPR, position L % CPR; activation copy c: row RPCA·c + L / CPRA, position
    // L % CPRA. Rows past N (M) load the last valid row: their results are not stored (activations: zeroed before use).
    unsigned woff[NWC], aoff[NAC];
#pragma unroll
    for (int c = 0; c < NWC; c++) {
        const int r = RPC * c + lane / CPR, rr = min(n0 + r, N - 1) - n0;
        woff[c] = (unsigned)((long long)rr * ldw * 2 + (((lane % CPR) ^ wsw(r)) << 4));
    }
#pragma unroll
    for (int c = 0; c < NAC; c++) {
        const int r = RPCA * c + lane / CPRA, rr = min(r, M - 1);
        aoff[c] = (unsigned)((long long)rr * lda * 4 + (((lane % CPRA) ^ (r & 15)) << 4));
    }
    const char *wb = reinterpret_cast<const char *>(W + (long long)n0 * ldw);
    const char *ab = reinterpret_cast<const char *>(A);
    // every workgroup reads the same rows of A: each wave starts its walk over its k groups at an offset given by the
    // workgroup's place on its XCD (dispatch slot / 8), so an XCD's workgroups read different columns of A at once
    const int rot = ng > 1 ? (int)((blockIdx.x >> 3) % (unsigned)ng) : 0;
    auto issue = [&](int j, int st) {   // group wv + SKS·((j + rot) mod ng) into stage st
        const int gg = wv + SKS * (j + rot < ng ? j + rot : j + rot - ng);
        const unsigned dst = lbase + st * SB;
#pragma unroll
        for (int c = 0; c < NWC; c++) lds_dma16(wb + (long long)gg * WROW, woff[c], dst + c * 1024);
#pragma unroll
        for (int c = 0; c < NAC; c++) lds_dma16(ab + (long long)gg * AROW, aoff[c], dst + WB + c * 1024);
    };
    floatx4 acc[4];
#pragma unroll
    for (int c = 0; c < 4; c++) acc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
    // rows of D past M come from duplicated activation rows: they are computed and never stored
    const int arow = i < MT ? i : 0;
#pragma unroll
    for (int st = 0; st < NSP; st++)
        if (st < ng) issue(st, st);
    int st = 0;
    for (int j = 0; j < ng; j++) {
        wait_vm_stages<NSP - 1, LPG>(min(NSP - 1, ng - 1 - j));   // group j has landed
        const G9_LDS unsigned char *sg = lds + st * SB;
        u32x4p wf[NSUB], af0[NSUB], af1[NSUB];
#pragma unroll
        for (int t = 0; t < NSUB; t++) {
            const int c = 4 * t + q;   // 16-byte weight chunk of the row; activation chunks 2c, 2c + 1
            wf[t] = *reinterpret_cast<const G9_LDS u32x4p *>(sg + i * WROW + ((c ^ wsw(i)) << 4));
            af0[t] = *reinterpret_cast<const G9_LDS u32x4p *>(sg + WB + arow * AROW + (((2 * c) ^ (arow & 15)) << 4));
            af1[t] = *reinterpret_cast<const G9_LDS u32x4p *>(sg + WB + arow * AROW + (((2 * c + 1) ^ (arow & 15)) << 4));
        }
        __builtin_amdgcn_sched_barrier(0);   // all fragment reads are issued before the first MFMA
#pragma unroll
        for (int t = 0; t < NSUB; t++) {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const unsigned h2 = wf[t][e / 2];
                const unsigned short h = e % 2 ? (unsigned short)(h2 >> 16) : (unsigned short)(h2 & 0xffffu);
                const unsigned ab32 = e < 4 ? af0[t][e] : af1[t][e - 4];
                // consecutive MFMAs go to different chains, so none waits for the one before
                acc[e % 4] = __builtin_amdgcn_mfma_f32_16x16x4f32(__builtin_bit_cast(float, ab32),
                                                                  (float)__builtin_bit_cast(_Float16, h), acc[e % 4], 0, 0, 0);
            }
        }
        wait_lgkm0();   // the stage is refilled next: its reads must be done
        if (j + NSP < ng) issue(j + NSP, st);
        st = st + 1 == NSP ? 0 : st + 1;
    }
    // lane holds D[m = 4q + r][n0 + i]; sum the chains, then the waves' tiles in wave order
    __syncthreads();
    float *part = reinterpret_cast<float *>(smem);   // [SKS][4][64]
#pragma unroll
    for (int r = 0; r < 4; r++) part[(wv * 4 + r) * 64 + lane] = (acc[0][r] + acc[1][r]) + (acc[2][r] + acc[3][r]);
    __syncthreads();
    const int n = n0 + i;
    if (wv != 0 || n >= N) return;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int m = 4 * q + r;
        if (m >= M) continue;
        float t = part[r * 64 + lane];
#pragma unroll
        for (int v = 1; v < SKS; v++) t += part[(v * 4 + r) * 64 + lane];
        C[(long long)m * ldc + n] = t;
        if (!__builtin_isfinite(t)) *flag = 1;
    }
}

// The same product on the VALU for small M: on the matrix cores a v_mfma_f32_16x16x4_f32 multiplies 16 activation
// rows whatever M is (N·K/16 of them per call, about 4 µs of issue per SIMD at N = K = 4096), while FP32 FMAs cost
// N·K·M. Shaped like the FP16 dot-product skinny kernel: a workgroup of KS waves owns RW consecutive weight rows, its
// waves split K in chunks of 8 k per lane (16 bytes of each weight row, nontemporal, and 32 bytes of each activation
// row, re-read from L2), every load of NC chunks issued before the first product; each weight is converted to FP32
// once and multiplied into the MT activation rows (rows past M repeat the last one and are not stored). The RW·MT
// sums of a lane are reduced across the wave by a transposing butterfly, the KS waves' sums added in LDS in wave
// order. Requires K % 8 == 0 and 16-byte aligned activation rows (the launcher checks); packed rows hold zeros past
// K up to their stride.
template <int MT, int RW, int KS, int NC>
__global__ void __launch_bounds__(KS * 64) skinny_pb_valu_kernel(int M, int N, int K, const float *__restrict__ A,
                                                                  long long lda, const _Float16 *__restrict__ W,
                                                                  long long ldw, float *__restrict__ C, long long ldc,
                                                                  int *flag) {
    constexpr int NV = RW * MT;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int n0 = blockIdx.x * RW;
    const _Float16 *wr[RW];
    const float *ar[MT];
#pragma unroll
    for (int r = 0; r < RW; r++) wr[r] = W + (long long)min(n0 + r, N - 1) * ldw;
#pragma unroll
    for (int m = 0; m < MT; m++) ar[m] = A + (long long)min(m, M - 1) * lda;
    float v[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) v[i] = 0.f;
    constexpr int SUPER = NC * KS * 64 * 8;   // chunk j of lane l: k = k0 + ((j·KS + wv)·64 + l)·8 .. +7
    const u32x4p zero = {0u, 0u, 0u, 0u};
    for (int k0 = 0; k0 < K; k0 += SUPER) {
        u32x4p wq[NC][RW], aq[NC][MT][2];
#pragma unroll
        for (int j = 0; j < NC; j++) {
            const int k = k0 + ((j * KS + wv) * 64 + lane) * 8;
            const bool in = k < K;
#pragma unroll
            for (int r = 0; r < RW; r++)
                wq[j][r] = in ? __builtin_nontemporal_load(reinterpret_cast<const u32x4p *>(wr[r] + k)) : zero;
#pragma unroll
            for (int m = 0; m < MT; m++) {
                aq[j][m][0] = in ? *reinterpret_cast<const u32x4p *>(ar[m] + k) : zero;
                aq[j][m][1] = in ? *reinterpret_cast<const u32x4p *>(ar[m] + k + 4) : zero;
            }
        }
#pragma unroll
        for (int j = 0; j < NC; j++)
#pragma unroll
            for (int r = 0; r < RW; r++)
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const unsigned h2 = wq[j][r][e / 2];
                    const float we = (float)__builtin_bit_cast(_Float16, (unsigned short)(e % 2 ? h2 >> 16 : h2 & 0xffffu));
#pragma unroll
                    for (int m = 0; m < MT; m++) {
                        const unsigned ab = aq[j][m][e / 4][e % 4];
                        v[r * MT + m] = __builtin_fmaf(we, __builtin_bit_cast(float, ab), v[r * MT + m]);
                    }
                }
    }
    int base = 0;
    butterfly<0, NV>(v, lane, base);
    constexpr int NF = Butterfly<NV>::per_lane;
    const bool writer = (lane & (Butterfly<NV>::dup - 1)) == 0;
    __shared__ float part[KS][NV];
    if (writer)
#pragma unroll
        for (int i = 0; i < NF; i++) part[wv][base + i] = v[i];
    __syncthreads();
    for (int t = threadIdx.x; t < NV; t += KS * 64) {
        const int n = n0 + t / MT, m = t % MT;
        if (n >= N || m >= M) continue;
        float s = part[0][t];
#pragma unroll
        for (int q = 1; q < KS; q++) s += part[q][t];
        C[(long long)m * ldc + n] = s;
        if (!__builtin_isfinite(s)) *flag = 1;   // every writer stores the same value
    }
}

constexpr int PB_VALU_MAX_M = 4;   // largest M on skinny_pb_valu_kernel
template <int MT, int RW, int KS, int NC>
static void launch_pb_valu(int M, int N, int K, const float *A, long long lda, const _Float16 *W, long long ldw, float *C,
                           long long ldc, int *flag) {
    hipLaunchKernelGGL((skinny_pb_valu_kernel<MT, RW, KS, NC>), dim3((unsigned)((N + RW - 1) / RW)), dim3(KS * 64), 0,
                       stream, M, N, K, A, lda, W, ldw, C, ldc, flag);
}

}  // namespace g9

using namespace g9;

extern "C" {

gen9blas_packed_b *gen9blas_pack_b(int type, int transB, int K, int N, const void *B, int ldb) {
    if (begin()) return nullptr;
    if (type < 0 || type > 3) {
        fail(GEN9BLAS_ERR_UNSUPPORTED, "type %d unavailable", type);
        return nullptr;
    }
    if (K <= 0 || N <= 0) {
        fail(GEN9BLAS_ERR_INVALID_ARG, "pack_b: K = %d, N = %d", K, N);
        return nullptr;
    }
    if (!B || ldb < (transB ? K : N)) {
        fail(GEN9BLAS_ERR_INVALID_ARG, "pack_b: %s (ldb %d)", B ? "leading dimension too small" : "NULL B", ldb);
        return nullptr;
    }
    const int es = elem_size(type);
    const long long ld = ((long long)K + 63) / 64 * 64;
    Operand ob;
    ob.host = B;
    ob.es = es;
    ob.rows = transB ? N : K;
    ob.cols = transB ? K : N;
    ob.caller_ld = ldb;
    if (resolve(ob, SLOT_B, true, false, true)) return nullptr;
    void *buf = nullptr;
    const hipError_t e = hipMalloc(&buf, (size_t)N * ld * es);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        fail(GEN9BLAS_ERR_OUT_OF_MEMORY, "pack_b: hipMalloc(%zu): %s", (size_t)((size_t)N * ld * es), hipGetErrorString(e));
        return nullptr;
    }
    const dim3 grid((unsigned)(ld / 32), (unsigned)((N + 31) / 32)), block(32, 8);
    if (es == 2)
        hipLaunchKernelGGL((pack_bt_kernel<uint16_t>), grid, block, 0, stream, (const uint16_t *)ob.dev, ob.ld, transB != 0,
                           K, N, (uint16_t *)buf, ld);
    else if (es == 4)
        hipLaunchKernelGGL((pack_bt_kernel<uint32_t>), grid, block, 0, stream, (const uint32_t *)ob.dev, ob.ld, transB != 0,
                           K, N, (uint32_t *)buf, ld);
    else
        hipLaunchKernelGGL((pack_bt_kernel<uint64_t>), grid, block, 0, stream, (const uint64_t *)ob.dev, ob.ld, transB != 0,
                           K, N, (uint64_t *)buf, ld);
    // synchronous, as the reference: the caller may reuse B (and the staging buffer is reused) after the return
    hipError_t ke = hipGetLastError();
    if (ke == hipSuccess) ke = hipStreamSynchronize(stream);
    if (ke != hipSuccess) {
        hip_fail(ke, "pack_b", __FILE__, __LINE__);
        (void)hipFree(buf);
        return nullptr;
    }
    gen9blas_packed_b *P = new (std::nothrow) gen9blas_packed_b;
    if (!P) {
        (void)hipFree(buf);
        fail(GEN9BLAS_ERR_OUT_OF_MEMORY, "pack_b: out of host memory");
        return nullptr;
    }
    P->type = type;
    P->K = K;
    P->N = N;
    P->ld = ld;
    P->buf = buf;
    return P;
}

int gen9blas_gemm_pb(int transA, int M, double alpha, const void *A, int lda, const gen9blas_packed_b *Bp, double beta,
                     void *C, int ldc) {
    G9_TRY(begin());
    if (!Bp) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "gemm_pb: no packed B");
    return gemm_impl(Bp->type, transA, 1, M, Bp->N, Bp->K, alpha, A, lda, 0, Bp->buf, (int)Bp->ld, 0, beta, C, ldc, 0, 1);
}

// Small batches on HS-packed weights (reference: lib/src/packed.c:307-329): DECLINED outside 1 ≤ M ≤ 16, a B not
// packed as GEN9BLAS_HS is INVALID_ARG. Always waits: *nonfinite is known only after the kernel. The non-finite flag
// is a word of pinned, coherent host memory that the kernel writes directly (only for a non-finite result); it is
// zero at the start of every call (the host clears it after a call that set it), so no copy is needed to read it.
int gen9blas_gemm_pb_skinny(int M, const float *A, int lda, const gen9blas_packed_b *Bp, float *C, int ldc,
                            int *nonfinite) {
    const double t0 = now_s();
    G9_TRY(begin());
    if (!Bp || Bp->type != GEN9BLAS_HS) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "gemm_pb_skinny: needs B packed as GEN9BLAS_HS");
    if (M < 1 || M > 16) return GEN9BLAS_DECLINED;
    if (!A || !C || !nonfinite) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "gemm_pb_skinny: NULL pointer");
    const int K = Bp->K, N = Bp->N;
    if (lda < K || ldc < N) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "gemm_pb_skinny: lda %d < K %d or ldc %d < N %d", lda, K, ldc, N);
    *nonfinite = 0;
    static volatile int *flag;
    if (!flag) {
        void *h = nullptr;
        G9_HIP(hipHostMalloc(&h, 256, hipHostMallocCoherent));
        flag = (volatile int *)h;
        *flag = 0;
    }
    Operand o[2];
    o[0].host = A; o[0].es = 4; o[0].rows = M; o[0].cols = K; o[0].caller_ld = lda;
    o[1].host = C; o[1].es = 4; o[1].rows = M; o[1].cols = N; o[1].caller_ld = ldc;
    G9_TRY(resolve(o[0], SLOT_A, true, false, true));
    G9_TRY(resolve(o[1], SLOT_C, ldc != N, true, true));
    const int steps = (K + 31) / 32;
    int spw = (steps + SPW - 1) / SPW;
    spw = (spw + SPB - 1) / SPB * SPB;
    const bool avec = (uintptr_t)o[0].dev % 16 == 0 && o[0].ld % 4 == 0;
    prof_begin();
    const dim3 grid((unsigned)((N + 15) / 16));
    const float *ad = (const float *)o[0].dev;
    const _Float16 *wd = (const _Float16 *)Bp->buf;
    float *cd = (float *)o[1].dev;
    // small M on the VALU (whole 8-k chunks, 16-byte activation rows). MI355X, 32 packed 4096² copies rotated, µs per
    // synchronous call against the matrix-core kernel below: M = 1 19.0 against 21.6 (2 rows per workgroup, 4 waves;
    // 1-8 rows, 2-8 waves, 1-4 chunks swept), M = 2 20.0 against 21.6 (4 rows, 8 waves), M = 4 21.5 against 21.9
    // (8 rows, 8 waves); M = 8 on the VALU 25.9-44 against 22.5
    if (M <= PB_VALU_MAX_M && K % 8 == 0 && avec) {
        if (M <= 1) launch_pb_valu<1, 2, 4, 1>(M, N, K, ad, o[0].ld, wd, Bp->ld, cd, o[1].ld, (int *)flag);
        else if (M <= 2) launch_pb_valu<2, 4, 8, 1>(M, N, K, ad, o[0].ld, wd, Bp->ld, cd, o[1].ld, (int *)flag);
        else launch_pb_valu<4, 8, 8, 1>(M, N, K, ad, o[0].ld, wd, Bp->ld, cd, o[1].ld, (int *)flag);
    } else if (K % 64 == 0 && avec && 16LL * (Bp->ld * 2 + o[0].ld * 4) < (1LL << 32)) {
        // the LDS-streaming kernel: whole 64-k groups, 16-byte activation rows, 32-bit per-lane offsets
        // MI355X, 32 packed 4096² copies rotated, µs per synchronous call (the wait for the call is about 6-8 µs of
        // it): 8 waves on 64-k groups, three stages at M ≤ 8 and two at M > 8: M = 8 18.2, M = 12 17.7-19.1, M = 16
        // 18.4-19.7 against 18.9, 19.8 and 20.0-20.5 for 128-k groups (8 waves with two stages at M ≤ 8, 4 waves with
        // two above, the largest that fit); 4 waves with four 64-k stages 19.9-21.0. Before that: M = 1 and 4 on
        // 128-k groups, 8 waves with two stages 21.7-21.9 (three: 22.4-22.9; 4 waves with three, five: 23.1-24.3;
        // 2 waves with four, eight: 29-31). Two waves per SIMD hide each other's ring and LDS waits.
        if (M <= 4) hipLaunchKernelGGL((skinny_pb_lds_kernel<4, 8, 3, 64>), grid, dim3(8 * 64), 0, stream, M, N, K, ad, o[0].ld, wd, Bp->ld, cd, o[1].ld, (int *)flag);
        else if (M <= 8) hipLaunchKernelGGL((skinny_pb_lds_kernel<8, 8, 3, 64>), grid, dim3(8 * 64), 0, stream, M, N, K, ad, o[0].ld, wd, Bp->ld, cd, o[1].ld, (int *)flag);
        else hipLaunchKernelGGL((skinny_pb_lds_kernel<16, 8, 2, 64>), grid, dim3(8 * 64), 0, stream, M, N, K, ad, o[0].ld, wd, Bp->ld, cd, o[1].ld, (int *)flag);
    } else {
        hipLaunchKernelGGL(skinny_pb_kernel, grid, dim3(SPW * 64), 0, stream, M, N, K, ad, o[0].ld, (int)avec, wd, Bp->ld,
                           spw, cd, o[1].ld, (int *)flag);
    }
    G9_HIP(hipGetLastError());
    prof_end();
    const int saved = nowait;
    nowait = 0;   // the flag is read after the kernel
    const int r = finish(o, 2);
    nowait = saved;
    G9_TRY(r);
    if (*flag) {
        *nonfinite = 1;
        *flag = 0;
    }
    prof_collect(t0);
    return 0;
}

void gen9blas_packed_b_free(gen9blas_packed_b *Bp) {
    if (!Bp) return;
    (void)hipStreamSynchronize(stream);   // queued products may still read it
    (void)hipFree(Bp->buf);
    delete Bp;
}

}  // extern "C"
