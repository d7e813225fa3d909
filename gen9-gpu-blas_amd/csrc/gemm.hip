// Level 3 entry points: gen9blas_gemm / _gemm_batched / _hgemm / _sgemm.
//
// Dispatch follows the reference (reference: lib/src/gemm.c:5-74, 177-263):
// - type check first (UNSUPPORTED), then non-positive dimensions return 0 without work;
// - a single product with min(M, N) ≤ the skinny threshold (16 by default, GEN9BLAS_SKINNY=n overrides, never for
//   FP64) takes the skinny kernel, with the roles of A and B swapped when N < M (Cᵀ = op(B)ᵀ·op(A)ᵀ, C written
//   through swapped strides) — here when both streamed operands are K-contiguous, otherwise the MFMA kernel;
// - everything else runs the MFMA kernel. It reads every transpose layout directly and fuses alpha/beta, so the
//   reference's pack kernels, padded work buffers and separate epilogue have no counterpart here;
// - GEN9BLAS_MAX_LAUNCH_MS (opt-in; the reference's default of 100 ms guarded against i915 preemption resets, which
//   do not exist on MI355X) splits a long product into bands of rows, each estimated below that time.
#include "internal.h"
#include <stdlib.h>

namespace g9 {

static int skinny_threshold(int type) {
    static int forced = -2;
    if (forced == -2) {
        const char *e = getenv("GEN9BLAS_SKINNY");
        forced = e ? atoi(e) : -1;
    }
    if (type == GEN9BLAS_D) return 0;
    return forced >= 0 ? forced : 16;
}

static double max_launch_ms() {
    static double v = -1;
    if (v < 0) {
        const char *e = getenv("GEN9BLAS_MAX_LAUNCH_MS");
        v = e && atof(e) > 0 ? atof(e) : 0;   // 0: no banding
    }
    return v;
}

// Conservative sustained rate of the MFMA kernels (TFLOP/s) for band planning.
static double est_ms(int type, double M, double N, double K) {
    const double tf = type == GEN9BLAS_D ? 20 : type == GEN9BLAS_S ? 40 : 400;
    return 2 * M * N * K / (tf * 1e9);
}

// One product (or a batch) on resolved device operands, split into row bands when planned.
static int run_gemm(GemmCall c) {
    const double lim = max_launch_ms();
    if (lim <= 0) return launch_gemm(c);
    const int parts = (int)(est_ms(c.type, c.M, c.N, c.K) * c.count / lim) + 1;
    if (parts <= 1) return launch_gemm(c);
    const int es = elem_size(c.type);
    const int mb = ((c.M + parts - 1) / parts + 255) / 256 * 256;
    for (int b = 0; b < c.count; b++)
        for (int i0 = 0; i0 < c.M; i0 += mb) {
            GemmCall s = c;
            s.count = 1;
            s.M = c.M - i0 < mb ? c.M - i0 : mb;
            s.A = (const char *)c.A + ((long long)b * c.sA + (c.tA ? i0 : (long long)i0 * c.lda)) * es;
            s.B = (const char *)c.B + (long long)b * c.sB * es;
            s.C = (char *)c.C + ((long long)b * c.sC + (long long)i0 * c.ldc) * es;
            G9_TRY(launch_gemm(s));
        }
    return 0;
}

// Operand description for resolve(): one matrix (re-pitched when staged) or, for a batch, its whole span.
static void describe(Operand &o, const void *p, long long rows, long long cols, long long ld, long long stride, int count,
                     int es) {
    o.host = p;
    o.es = es;
    if (count == 1) {
        o.rows = rows;
        o.cols = cols;
        o.caller_ld = ld;
    } else {
        o.rows = 1;
        o.cols = (long long)(count - 1) * stride + (rows - 1) * ld + cols;
        o.caller_ld = o.cols;
    }
}

int gemm_impl(int type, int tA, int tB, int M, int N, int K, double alpha, const void *A, int lda, long long sA,
                     const void *B, int ldb, long long sB, double beta, void *C, int ldc, long long sC, int count) {
    const double t0 = now_s();
    G9_TRY(begin());
    if (type < 0 || type > 3) G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "type %d unavailable", type);
    if (M <= 0 || N <= 0 || K <= 0 || count <= 0) return 0;
    tA = tA != 0;
    tB = tB != 0;
    if (!A || !B || !C) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "gemm: NULL matrix pointer");
    if (lda < (tA ? M : K) || ldb < (tB ? K : N) || ldc < N)
        G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "gemm: leading dimension too small (lda %d, ldb %d, ldc %d)", lda, ldb, ldc);
    if (count > 1 && (sA < 0 || sB < 0 || sC < 0)) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "gemm_batched: negative stride");
    const int es = elem_size(type);

    Operand ops[3];
    describe(ops[0], A, tA ? K : M, tA ? M : K, lda, sA, count, es);
    describe(ops[1], B, tB ? N : K, tB ? K : N, ldb, sB, count, es);
    describe(ops[2], C, M, N, ldc, sC, count, es);
    // A staged batch span of C is copied in when it has gaps the copy back must preserve.
    const bool c_gaps = count > 1 && (ldc != N || sC != (long long)M * ldc);
    G9_TRY(resolve(ops[0], SLOT_A, true, false, count == 1));
    G9_TRY(resolve(ops[1], SLOT_B, true, false, count == 1));
    G9_TRY(resolve(ops[2], SLOT_C, beta != 0.0 || c_gaps, true, count == 1));
    last_zc = (ops[0].zc ? 1 : 0) | (ops[1].zc ? 2 : 0) | (ops[2].zc ? 4 : 0);
    const long long Ld = count == 1 ? ops[0].ld : lda, Bld = count == 1 ? ops[1].ld : ldb, Cld = count == 1 ? ops[2].ld : ldc;

    prof_begin();
    const int mn = M < N ? M : N;
    if (count == 1 && mn <= skinny_threshold(type) && !tA && tB) {
        // both streamed operands K-contiguous: C = alpha·a·wᵀ + beta·C with the small side as a
        SkinnyCall s;
        s.type = type;
        s.K = K;
        s.alpha = alpha;
        s.beta = beta;
        s.C = ops[2].dev;
        if (M <= N) {
            s.M = M; s.N = N;
            s.a = ops[0].dev; s.sam = Ld;
            s.w = ops[1].dev; s.swn = Bld;
            s.scm = Cld; s.scn = 1;
        } else {
            s.M = N; s.N = M;
            s.a = ops[1].dev; s.sam = Bld;
            s.w = ops[0].dev; s.swn = Ld;
            s.scm = 1; s.scn = Cld;
        }
        G9_TRY(launch_skinny(s));
    } else {
        GemmCall g;
        g.type = type;
        g.tA = tA; g.tB = tB;
        g.M = M; g.N = N; g.K = K;
        g.count = count;
        g.alpha = alpha;
        g.beta = beta;
        g.A = ops[0].dev; g.lda = Ld; g.sA = sA;
        g.B = ops[1].dev; g.ldb = Bld; g.sB = sB;
        g.C = ops[2].dev; g.ldc = Cld; g.sC = sC;
        G9_TRY(run_gemm(g));
    }
    prof_end();
    G9_TRY(finish(ops, 3));
    prof_collect(t0);
    return 0;
}

}  // namespace g9

using namespace g9;

extern "C" {

int gen9blas_gemm_batched(int type, int transA, int transB, int M, int N, int K, double alpha, const void *A, int lda,
                          int64_t sA, const void *B, int ldb, int64_t sB, double beta, void *C, int ldc, int64_t sC,
                          int count) {
    return gemm_impl(type, transA, transB, M, N, K, alpha, A, lda, sA, B, ldb, sB, beta, C, ldc, sC, count);
}

int gen9blas_gemm(int type, int transA, int transB, int M, int N, int K, double alpha, const void *A, int lda, const void *B,
                  int ldb, double beta, void *C, int ldc) {
    return gemm_impl(type, transA, transB, M, N, K, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0, 1);
}

int gen9blas_hgemm(int M, int N, int K, double alpha, const uint16_t *A, int lda, const uint16_t *B, int ldb, double beta,
                   uint16_t *C, int ldc) {
    return gemm_impl(GEN9BLAS_H, 0, 0, M, N, K, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0, 1);
}

int gen9blas_sgemm(int M, int N, int K, double alpha, const float *A, int lda, const float *B, int ldb, double beta, float *C,
                   int ldc) {
    return gemm_impl(GEN9BLAS_S, 0, 0, M, N, K, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0, 1);
}

}  // extern "C"
