// Level 3 entry points: gen9blas_gemm / _gemm_batched / _hgemm / _sgemm.
//
// Dispatch follows the reference (reference: lib/src/gemm.c:5-74, 177-263):
// - type check first (UNSUPPORTED), then non-positive dimensions return 0 without work;
// - a single product with min(M, N) ≤ the skinny threshold (16 by default, GEN9BLAS_SKINNY=n overrides, never for
//   FP64) takes the skinny kernel, with the roles of A and B swapped when N < M (Cᵀ = op(B)ᵀ·op(A)ᵀ, C written
//   through swapped strides), in every layout: weights contiguous along K or along N, the small operand transposed
//   or not;
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

// A single product whose C lies in pageable host memory and spans at least two pinned chunks (HGEMM n = 4096: 32 MiB)
// is computed in row panels of at most one chunk of C each, so that copies and kernels overlap: panel p's kernel
// runs while panel p + 1's inputs come in, and panel p's rows of C go back while the next inputs move and the host
// copies out the panel before. A comes in panel by panel when its panel rows are contiguous (not transposed,
// pageable, not re-pitched); B, and an A that is not, come in whole first. C comes in per panel when beta ≠ 0 or its
// rows have gaps, which the copy back must keep. Each panel is the product over a band of rows, as run_gemm's bands
// are, with the same kernels. With GEN9BLAS_PROFILE the reported time spans the panels' copies too. `taken` is false
// when the product does not qualify (nothing is done then).
constexpr size_t PANEL_MIN = 16u << 20;
static int gemm_panels(bool &taken, int type, int tA, int tB, int M, int N, int K, double alpha, const void *A, int lda,
                       const void *B, int ldb, double beta, void *C, int ldc, double t0) {
    taken = false;
    const size_t es = elem_size(type);
    const size_t cspan = ((size_t)(M - 1) * ldc + N) * es, cdense = (size_t)M * N * es;
    if (cspan < PANEL_MIN || cspan > 2 * cdense || mem_kind(C, cspan) != MEM_HOST) return 0;
    const size_t chunk = out_chunk(), rowb = (size_t)ldc * es;
    const long long pr = chunk ? (long long)(chunk / rowb) / 256 * 256 : 0;   // rows per panel
    if (pr < 256 || pr >= M) return 0;
    taken = true;
    const size_t aspan = tA ? 0 : ((size_t)(M - 1) * lda + K) * es;
    const bool pa = !tA && aspan <= 2 * (size_t)M * K * es && mem_kind(A, aspan) == MEM_HOST;
    const bool c_in = beta != 0.0 || ldc != N;

    Operand ops[3];
    describe(ops[0], A, tA ? K : M, tA ? M : K, lda, 0, 1, (int)es);
    describe(ops[1], B, tB ? N : K, tB ? K : N, ldb, 0, 1, (int)es);
    describe(ops[2], C, M, N, ldc, 0, 1, (int)es);
    G9_TRY(resolve(ops[0], SLOT_A, !pa, false, !pa));
    G9_TRY(resolve(ops[1], SLOT_B, true, false, true));
    G9_TRY(resolve(ops[2], SLOT_C, false, false, false));   // pageable, not re-pitched: ld = ldc, filled per panel
    last_zc = (ops[0].zc ? 1 : 0) | (ops[1].zc ? 2 : 0);
    char *Ad = (char *)ops[0].dev, *Cd = (char *)ops[2].dev;
    const long long Ald = ops[0].ld;
    auto rows_of = [&](long long p) { return M - p * pr < pr ? M - p * pr : pr; };
    auto cbytes = [&](long long p) { return ((size_t)(rows_of(p) - 1) * ldc + N) * es; };
    const long long np = (M + pr - 1) / pr;
    auto issue = [&](long long p) -> int {   // panel p: its inputs on the second stream, then its kernel
        const long long i0 = p * pr, rows = rows_of(p);
        const size_t co = (size_t)i0 * ldc * es;
        if (pa) {
            const size_t ao = (size_t)i0 * lda * es;
            G9_TRY(stage_in(Ad + ao, (const char *)A + ao, ((size_t)(rows - 1) * lda + K) * es));
        }
        if (c_in) G9_TRY(stage_in(Cd + co, (const char *)C + co, cbytes(p)));
        if (pa || c_in) G9_TRY(stage_in_ready());
        GemmCall g;
        g.type = type;
        g.tA = tA; g.tB = tB;
        g.M = (int)rows; g.N = N; g.K = K;
        g.count = 1;
        g.alpha = alpha;
        g.beta = beta;
        g.A = Ad + (size_t)(tA ? i0 : i0 * Ald) * es; g.lda = Ald; g.sA = 0;
        g.B = ops[1].dev; g.ldb = ops[1].ld; g.sB = 0;
        g.C = Cd + co; g.ldc = ldc; g.sC = 0;
        G9_TRY(run_gemm(g));
        return out_mark((int)(p & 1));
    };
    auto host_c = [&](long long p) { return (char *)C + (size_t)p * pr * ldc * es; };
    // Second stream: A0 A1 C0 A2 C1 A3 C2 C3 (each result queued behind the next panel's inputs, which do not wait
    // for its kernel); the host copies C(p - 1) out while C(p) and A(p + 1) move.
    auto run = [&]() -> int {
        prof_begin();
        G9_TRY(issue(0));
        for (long long p = 0; p < np; p++) {
            if (p + 1 < np) G9_TRY(issue(p + 1));
            G9_TRY(out_start((int)(p & 1), Cd + (size_t)p * pr * ldc * es, cbytes(p)));
            if (p > 0) G9_TRY(out_finish((int)((p - 1) & 1), host_c(p - 1), cbytes(p - 1)));
        }
        G9_TRY(out_finish((int)((np - 1) & 1), host_c(np - 1), cbytes(np - 1)));
        prof_end();
        return wait_stream();
    };
    const int r = run();
    if (r) {
        out_drain();
        return r;
    }
    prof_collect(t0);
    return 0;
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
    const int mn = M < N ? M : N;
    const bool skinny = count == 1 && mn <= skinny_threshold(type);
    if (count == 1 && !skinny) {
        bool taken;
        const int r = gemm_panels(taken, type, tA, tB, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, t0);
        if (taken) return r;
    }

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
    if (skinny) {
        // C = alpha·a·wᵀ + beta·C with the small side as a (reference: lib/src/gemm.c:207-221): a = op(A), w = op(B)ᵀ,
        // or for N < M a = op(B)ᵀ, w = op(A), C written through swapped strides
        SkinnyCall s;
        s.type = type;
        s.K = K;
        s.alpha = alpha;
        s.beta = beta;
        s.C = ops[2].dev;
        if (M <= N) {
            s.M = M; s.N = N;
            s.a = ops[0].dev; s.sam = tA ? 1 : Ld; s.sak = tA ? Ld : 1;        // op(A)[m][k]
            s.w = ops[1].dev; s.swn = tB ? Bld : 1; s.swk = tB ? 1 : Bld;      // op(B)[k][n]
            s.scm = Cld; s.scn = 1;
        } else {
            s.M = N; s.N = M;
            s.a = ops[1].dev; s.sam = tB ? Bld : 1; s.sak = tB ? 1 : Bld;      // op(B)ᵀ[n][k]
            s.w = ops[0].dev; s.swn = tA ? 1 : Ld; s.swk = tA ? Ld : 1;        // op(A)[m][k]
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
