// gen9blas for AMD Instinct MI355X (gfx950): BLAS levels 1-3 in FP16, FP32 and FP64 on hand-written HIP kernels.
//
// This header is the drop-in C ABI. Every declaration keeps the signature, the argument meaning and the status
// codes of the reference library's public header (reference: lib/gen9blas.h:20-166), so programs, the ctypes module
// and the Rust/ggml bindings written against that header link against libgen9blas.so unchanged.
//
// Rules shared by every entry point
// - Matrices are row-major. Elements are passed as void*: uint16_t holds FP16 bit patterns, then float, double.
// - A pointer may be host memory (pageable or pinned) or HIP device memory. Device memory is used in place by the
//   kernels ("zero-copy"); host memory is copied to a device work buffer and results are copied back.
// - Return value: 0 success, < 0 an error (text: gen9blas_error()), GEN9BLAS_DECLINED (1) "not handled, nothing
//   written" for functions documented to decline. Functions returning pointers return NULL on error and set
//   gen9blas_last_status().
// - Process-wide state (work buffers, the last error, the HIP stream): the caller serializes calls. gen9blas_error()
//   stays valid until the next call.
// - Non-positive dimensions make a call a no-op that returns 0.
// MI355X-only additions (HIP stream, device memory, no-wait mode) are declared in gen9blas_hip.h.
#pragma once
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

// ABI version 0.2.0 (reference: lib/gen9blas.h:20-23). The ctypes module accepts 0.2.x only.
#define GEN9BLAS_VERSION_MAJOR 0
#define GEN9BLAS_VERSION_MINOR 2
#define GEN9BLAS_VERSION_PATCH 0
#define GEN9BLAS_VERSION (GEN9BLAS_VERSION_MAJOR * 10000 + GEN9BLAS_VERSION_MINOR * 100 + GEN9BLAS_VERSION_PATCH)
#ifndef GEN9BLAS_API
#define GEN9BLAS_API __attribute__((visibility("default")))
#endif

// Element types (reference: lib/gen9blas.h:28-31). On MI355X both FP16 types run on FP16 MFMA with FP32
// accumulation; GEN9BLAS_HS keeps the guarantee "FP32 partial sums at least every GEN9BLAS_KC products".
enum { GEN9BLAS_H = 0, GEN9BLAS_S = 1, GEN9BLAS_HS = 2, GEN9BLAS_D = 3 };
#define GEN9BLAS_KC 32
enum { GEN9BLAS_NO_TRANS = 0, GEN9BLAS_TRANS = 1 };
enum { GEN9BLAS_LEFT = 0, GEN9BLAS_RIGHT = 1 };
enum { GEN9BLAS_LOWER = 0, GEN9BLAS_UPPER = 1 };
enum { GEN9BLAS_NON_UNIT = 0, GEN9BLAS_UNIT = 1 };

// Status codes (reference: lib/gen9blas.h:38-46).
typedef enum {
    GEN9BLAS_OK = 0,
    GEN9BLAS_DECLINED = 1,
    GEN9BLAS_ERR = -1,                 // HIP runtime / kernel error
    GEN9BLAS_ERR_UNSUPPORTED = -2,     // type, layout or function not available in this build
    GEN9BLAS_ERR_INVALID_ARG = -3,     // bad leading dimension, increment, handle, ...
    GEN9BLAS_ERR_OUT_OF_MEMORY = -4,   // device or pinned host allocation failed
    GEN9BLAS_ERR_NO_DEVICE = -5,       // no usable gfx950 device; permanent for the process
} gen9blas_status;

// ---- Library (reference: lib/gen9blas.h:48-78) ----
// gen9blas_version: reference lib/gen9blas.h:50, implemented in lib/src/core.c:385-392
GEN9BLAS_API int gen9blas_version(void);
// Opens the GPU once per process; later calls return the first result (a failure is final).
// gen9blas_init: reference lib/gen9blas.h:53, implemented in lib/src/core.c:205-219
GEN9BLAS_API int gen9blas_init(void);
// 9 when a supported device is open (the reference's "full feature set" value, kept so callers testing for it keep
// working), 0 when there is none. gen9blas_hip.h: gen9blas_device_arch() gives the gfx number (950).
// gen9blas_device_gen: reference lib/gen9blas.h:55
GEN9BLAS_API int gen9blas_device_gen(void);
enum {
    GEN9BLAS_FEAT_FP16 = 0,
    GEN9BLAS_FEAT_FP32,
    GEN9BLAS_FEAT_FP64,
    GEN9BLAS_FEAT_SKINNY_PB,
    GEN9BLAS_FEAT_EPILOG_EXT,
    GEN9BLAS_FEAT_NORM_PACK,
    GEN9BLAS_FEAT_ROPE_MULTI,
    GEN9BLAS_FEAT_CPY,
    GEN9BLAS_FEAT_SET_ROWS,
};
// gen9blas_has: reference lib/gen9blas.h:68
GEN9BLAS_API int gen9blas_has(int feature);        // 1 available, 0 not (also for unknown features)
// gen9blas_error: reference lib/gen9blas.h:69
GEN9BLAS_API const char *gen9blas_error(void);
// gen9blas_last_status: reference lib/gen9blas.h:70
GEN9BLAS_API int gen9blas_last_status(void);
// GEN9BLAS_PROFILE=1: device time of the main kernel(s) of the last call (HIP events); else the whole call.
// gen9blas_last_time_ms: reference lib/gen9blas.h:71
GEN9BLAS_API double gen9blas_last_time_ms(void);
// Level 3 calls: bit 1 = A, 2 = B, 4 = C was used in place (device memory), 0 = staged through a work buffer.
// gen9blas_last_zero_copy: reference lib/gen9blas.h:72
GEN9BLAS_API int gen9blas_last_zero_copy(void);

// Host memory the GPU can DMA without an intermediate copy (pinned, 4096-byte aligned). Kernels still run on device
// copies: on a discrete GPU, reading host memory from a kernel would be bound by the host link.
// gen9blas_alloc: reference lib/gen9blas.h:76, implemented in lib/src/core.c:288-297
GEN9BLAS_API void *gen9blas_alloc(size_t bytes);
// gen9blas_free: reference lib/gen9blas.h:77, implemented in lib/src/core.c:288-297
GEN9BLAS_API void gen9blas_free(void *p);
// gen9blas_is_usm: reference lib/gen9blas.h:78, implemented in lib/src/core.c:288-297
GEN9BLAS_API int gen9blas_is_usm(const void *p, size_t bytes);   // 1: [p, p+bytes) inside one gen9blas_alloc block

// ---- Level 3 (reference: lib/gen9blas.h:80-117) ----
// C = alpha·op(A)·op(B) + beta·C; op(A) M×K (transA: A stored K×M), op(B) K×N (transB: B stored N×K).
// beta = 0: C is not read. alpha and beta are rounded to float for GEN9BLAS_H/HS/S.
// gen9blas_gemm: reference lib/gen9blas.h:82, implemented in lib/src/gemm.c:177-180
GEN9BLAS_API int gen9blas_gemm(int type, int transA, int transB, int M, int N, int K, double alpha, const void *A, int lda,
                               const void *B, int ldb, double beta, void *C, int ldc);
// Strided batch: matrix b uses A + b·sA, B + b·sB, C + b·sC (strides in elements); one launch for the batch.
// gen9blas_gemm_batched: reference lib/gen9blas.h:86, implemented in lib/src/gemm.c:5-74
GEN9BLAS_API int gen9blas_gemm_batched(int type, int transA, int transB, int M, int N, int K, double alpha,
                                       const void *A, int lda, int64_t sA, const void *B, int ldb, int64_t sB,
                                       double beta, void *C, int ldc, int64_t sC, int count);
// Packed B kept on the device (reference: lib/gen9blas.h:89-97).
typedef struct gen9blas_packed_b gen9blas_packed_b;
// gen9blas_pack_b: reference lib/gen9blas.h:94
GEN9BLAS_API gen9blas_packed_b *gen9blas_pack_b(int type, int transB, int K, int N, const void *B, int ldb);
// gen9blas_gemm_pb: reference lib/gen9blas.h:95
GEN9BLAS_API int gen9blas_gemm_pb(int transA, int M, double alpha, const void *A, int lda, const gen9blas_packed_b *Bp,
                                  double beta, void *C, int ldc);
// gen9blas_packed_b_free: reference lib/gen9blas.h:97
GEN9BLAS_API void gen9blas_packed_b_free(gen9blas_packed_b *Bp);
// gen9blas_symm: reference lib/gen9blas.h:99
GEN9BLAS_API int gen9blas_symm(int type, int side, int uplo, int M, int N, double alpha, const void *A, int lda,
                               const void *B, int ldb, double beta, void *C, int ldc);
// gen9blas_syrk: reference lib/gen9blas.h:102
GEN9BLAS_API int gen9blas_syrk(int type, int uplo, int trans, int N, int K, double alpha, const void *A, int lda,
                               double beta, void *C, int ldc);
// gen9blas_syr2k: reference lib/gen9blas.h:105
GEN9BLAS_API int gen9blas_syr2k(int type, int uplo, int trans, int N, int K, double alpha, const void *A, int lda,
                                const void *B, int ldb, double beta, void *C, int ldc);
// gen9blas_trmm: reference lib/gen9blas.h:108
GEN9BLAS_API int gen9blas_trmm(int type, int side, int uplo, int transA, int diag, int M, int N, double alpha,
                               const void *A, int lda, void *B, int ldb);
// gen9blas_trsm: reference lib/gen9blas.h:111
GEN9BLAS_API int gen9blas_trsm(int type, int side, int uplo, int transA, int diag, int M, int N, double alpha,
                               const void *A, int lda, void *B, int ldb);
// gen9blas_hgemm: reference lib/gen9blas.h:114, implemented in lib/src/gemm.c:181-182
GEN9BLAS_API int gen9blas_hgemm(int M, int N, int K, double alpha, const uint16_t *A, int lda, const uint16_t *B, int ldb,
                                double beta, uint16_t *C, int ldc);
// gen9blas_sgemm: reference lib/gen9blas.h:116, implemented in lib/src/gemm.c:183-184
GEN9BLAS_API int gen9blas_sgemm(int M, int N, int K, double alpha, const float *A, int lda, const float *B, int ldb,
                                double beta, float *C, int ldc);

// ---- Levels 1-2 (reference: lib/gen9blas.h:119-148). type: GEN9BLAS_S, _D or _H (_HS = _H).
// FP16 computes in FP32; dot/asum/nrm2 accumulate in FP64. Vectors: n elements inc apart (inc != 0; inc < 0: the
// pointer is the lowest address, element 0 is at the end, as in BLAS).
// gen9blas_axpy: reference lib/gen9blas.h:121, implemented in lib/src/level12.c:45-52
GEN9BLAS_API int gen9blas_axpy(int type, int n, double a, const void *x, int incx, void *y, int incy);
// gen9blas_scal: reference lib/gen9blas.h:122
GEN9BLAS_API int gen9blas_scal(int type, int n, double a, void *x, int incx);
// gen9blas_copy: reference lib/gen9blas.h:123
GEN9BLAS_API int gen9blas_copy(int type, int n, const void *x, int incx, void *y, int incy);
// gen9blas_swap: reference lib/gen9blas.h:124
GEN9BLAS_API int gen9blas_swap(int type, int n, void *x, int incx, void *y, int incy);
// gen9blas_rot: reference lib/gen9blas.h:125
GEN9BLAS_API int gen9blas_rot(int type, int n, void *x, int incx, void *y, int incy, double c, double s);
// gen9blas_rotm: reference lib/gen9blas.h:126
GEN9BLAS_API int gen9blas_rotm(int type, int n, void *x, int incx, void *y, int incy, const double *param);
// gen9blas_rotg: reference lib/gen9blas.h:127
GEN9BLAS_API void gen9blas_rotg(float *a, float *b, float *c, float *s);
// gen9blas_rotmg: reference lib/gen9blas.h:128
GEN9BLAS_API void gen9blas_rotmg(float *d1, float *d2, float *x1, float y1, float *param);
// gen9blas_dot: reference lib/gen9blas.h:129, implemented in lib/src/level12.c:171-188
GEN9BLAS_API int gen9blas_dot(int type, int n, const void *x, int incx, const void *y, int incy, double *result);
// gen9blas_asum: reference lib/gen9blas.h:130
GEN9BLAS_API int gen9blas_asum(int type, int n, const void *x, int incx, double *result);
// gen9blas_nrm2: reference lib/gen9blas.h:131
GEN9BLAS_API int gen9blas_nrm2(int type, int n, const void *x, int incx, double *result);
// gen9blas_iamax: reference lib/gen9blas.h:132
GEN9BLAS_API int gen9blas_iamax(int type, int n, const void *x, int incx, int64_t *result);
// y = alpha·op(A)·x + beta·y, A M×N (trans: x has length M, y length N). beta = 0: y is not read.
// gen9blas_gemv: reference lib/gen9blas.h:134, implemented in lib/src/level12.c:215-265
GEN9BLAS_API int gen9blas_gemv(int type, int trans, int M, int N, double alpha, const void *A, int lda, const void *x, int incx,
                               double beta, void *y, int incy);
// gen9blas_symv: reference lib/gen9blas.h:137
GEN9BLAS_API int gen9blas_symv(int type, int uplo, int n, double alpha, const void *A, int lda, const void *x, int incx,
                               double beta, void *y, int incy);
// gen9blas_trmv: reference lib/gen9blas.h:140
GEN9BLAS_API int gen9blas_trmv(int type, int uplo, int trans, int diag, int n, const void *A, int lda, void *x, int incx);
// gen9blas_trsv: reference lib/gen9blas.h:141
GEN9BLAS_API int gen9blas_trsv(int type, int uplo, int trans, int diag, int n, const void *A, int lda, void *x, int incx);
// gen9blas_syr: reference lib/gen9blas.h:143
GEN9BLAS_API int gen9blas_syr(int type, int uplo, int n, double alpha, const void *x, int incx, void *A, int lda);
// gen9blas_syr2: reference lib/gen9blas.h:144
GEN9BLAS_API int gen9blas_syr2(int type, int uplo, int n, double alpha, const void *x, int incx, const void *y, int incy,
                               void *A, int lda);
// gen9blas_ger: reference lib/gen9blas.h:147
GEN9BLAS_API int gen9blas_ger(int type, int M, int N, double alpha, const void *x, int incx, const void *y, int incy,
                              void *A, int lda);

// ---- Level 2 banded and packed, CBLAS RowMajor layout (reference: lib/gen9blas.h:150-166) ----
// gen9blas_gbmv: reference lib/gen9blas.h:154
GEN9BLAS_API int gen9blas_gbmv(int type, int trans, int M, int N, int KL, int KU, double alpha, const void *A, int lda,
                               const void *x, int incx, double beta, void *y, int incy);
// gen9blas_sbmv: reference lib/gen9blas.h:156
GEN9BLAS_API int gen9blas_sbmv(int type, int uplo, int N, int K, double alpha, const void *A, int lda, const void *x, int incx,
                               double beta, void *y, int incy);
// gen9blas_tbmv: reference lib/gen9blas.h:158
GEN9BLAS_API int gen9blas_tbmv(int type, int uplo, int trans, int diag, int N, int K, const void *A, int lda, void *x, int incx);
// gen9blas_tbsv: reference lib/gen9blas.h:159
GEN9BLAS_API int gen9blas_tbsv(int type, int uplo, int trans, int diag, int N, int K, const void *A, int lda, void *x, int incx);
// gen9blas_spmv: reference lib/gen9blas.h:160
GEN9BLAS_API int gen9blas_spmv(int type, int uplo, int N, double alpha, const void *Ap, const void *x, int incx, double beta,
                               void *y, int incy);
// gen9blas_tpmv: reference lib/gen9blas.h:162
GEN9BLAS_API int gen9blas_tpmv(int type, int uplo, int trans, int diag, int N, const void *Ap, void *x, int incx);
// gen9blas_tpsv: reference lib/gen9blas.h:163
GEN9BLAS_API int gen9blas_tpsv(int type, int uplo, int trans, int diag, int N, const void *Ap, void *x, int incx);
// gen9blas_spr: reference lib/gen9blas.h:164
GEN9BLAS_API int gen9blas_spr(int type, int uplo, int N, double alpha, const void *x, int incx, void *Ap);
// gen9blas_spr2: reference lib/gen9blas.h:165
GEN9BLAS_API int gen9blas_spr2(int type, int uplo, int N, double alpha, const void *x, int incx, const void *y, int incy,
                               void *Ap);

#ifdef __cplusplus
}
#endif
