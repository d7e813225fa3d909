// gen9blas MI355X additions: the HIP stream, device memory and asynchronous ("no-wait") calls.
//
// These entry points have no counterpart in the reference's BLAS header, except the no-wait pair, which mirrors
// gen9blas_set_nowait / gen9blas_flush of the reference's ML header (reference: lib/gen9blas_ml.h:56-69) and is
// extended here to every BLAS call whose operands are all device memory.
#pragma once
#include <stddef.h>
#include "gen9blas.h"
#ifdef __cplusplus
extern "C" {
#endif

// gfx architecture number of the open device (950 for MI355X), 0 without a device.
GEN9BLAS_API int gen9blas_device_arch(void);
// The library's HIP stream (a hipStream_t). Every kernel of the library is launched on it. The stream synchronizes
// with the legacy default stream, so work queued on the null stream by the caller is ordered before library calls.
GEN9BLAS_API void *gen9blas_hip_stream(void);
// Device memory (hipMalloc). Pointers into it are used in place by every entry point.
GEN9BLAS_API void *gen9blas_device_alloc(size_t bytes);
GEN9BLAS_API void gen9blas_device_free(void *p);
// 1 when [p, p+bytes) lies in one HIP device (or managed) allocation, which kernels use in place; 0 for host memory,
// NULL, or without a device. The BLAS shim uses it to keep device operands off the CPU BLAS.
GEN9BLAS_API int gen9blas_is_device(const void *p, size_t bytes);
// Copy between any two of host / pinned host / device memory, synchronous on the library stream.
GEN9BLAS_API int gen9blas_memcpy(void *dst, const void *src, size_t bytes);
// No-wait mode: while on, a call whose operands are all device memory queues its kernels and returns without waiting
// (results written by the kernels are ready after gen9blas_flush). Calls that touch host memory, and calls that
// return a value through a host pointer (dot, asum, nrm2, iamax), still wait.
GEN9BLAS_API void gen9blas_set_nowait(int on);
// Waits until all queued work of the library has finished; returns 0 or the error of a failed kernel.
GEN9BLAS_API int gen9blas_flush(void);
// gen9blas_gemm that allocates nothing. No counterpart in the reference: it is for callers that cannot allocate
// device memory (tight serving loops, harnesses that forbid hipMalloc). Same arguments, kernels and results as
// gen9blas_gemm, but A, B and C must be device memory (an operand in host memory would need staging buffers:
// INVALID_ARG before anything runs), and the work space is a static 64 MiB device array per GPU: enough for the
// split-K slices of every default dispatch on MI355X (CUs × the largest split tile) and for the skinny products
// (min(M, N) ≤ 16: a transposed small operand gathered, M·K elements; the K-split partial sums of weights stored
// K×N, at most 4 MiB). A product that would need more (a split forced by GEN9BLAS_SPLITK, or a skinny product whose
// M·K·element size passes about 60 MiB) gives INVALID_ARG before any launch. It runs on the library stream like every call and
// is not meant for HIP graph capture. Call gen9blas_init first: the first call of the library opens the device. All
// calls on one GPU share the array, so calls that overlap on one GPU (from several threads) race.
GEN9BLAS_API int gen9blas_gemm_noalloc(int type, int transA, int transB, int M, int N, int K, double alpha,
                                       const void *A, int lda, const void *B, int ldb, double beta, void *C, int ldc);

#ifdef __cplusplus
}
#endif
