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

void gen9blas_packed_b_free(gen9blas_packed_b *Bp) {
    if (!Bp) return;
    (void)hipStreamSynchronize(stream);   // queued products may still read it
    (void)hipFree(Bp->buf);
    delete Bp;
}

}  // extern "C"
