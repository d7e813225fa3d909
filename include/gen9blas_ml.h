// gen9blas MI355X: the part of the reference's ML header that lies on the packed-weight decode path.
//
// The reference's lib/gen9blas_ml.h declares its ggml operator set (norms, RoPE, attention, packed activations,
// fused FFN, copies). Of it, this build provides the small-batch product on packed FP16 weights with FP32
// activations, and the queued-work pair gen9blas_set_nowait / gen9blas_flush (declared with the MI355X additions in
// gen9blas_hip.h, included here). The other operators are not part of this library.
#pragma once
#include "gen9blas.h"
#include "gen9blas_hip.h"
#ifdef __cplusplus
extern "C" {
#endif

// C (M×N, FP32, row stride ldc) = A (M×K, FP32, row stride lda) · op(B) for 1 <= M <= 16, with Bp packed by
// gen9blas_pack_b as GEN9BLAS_HS (K×N; FP16 weights): FP32 products and sums, FP32 result, A read as it lies.
// *nonfinite = 1 if any result is infinite or NaN, else 0. Returns 0, GEN9BLAS_DECLINED (1, nothing done) for M
// outside 1..16, GEN9BLAS_ERR_INVALID_ARG for a B not packed as GEN9BLAS_HS, or another error status.
// gen9blas_gemm_pb_skinny: reference lib/gen9blas_ml.h:25-28, lib/src/packed.c:307-329
GEN9BLAS_API int gen9blas_gemm_pb_skinny(int M, const float *A, int lda, const gen9blas_packed_b *Bp, float *C, int ldc,
                                         int *nonfinite);

#ifdef __cplusplus
}
#endif
