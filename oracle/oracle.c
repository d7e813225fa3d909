/* Oracle: CPU restatement of the reference's arithmetic on the gen9blas hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (libgen9blas.so, libgen9blas_blas.so, gen9blas.py) links,
 * loads or calls this code; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the
 * checker. Built with -ffp-contract=off: every fused multiply-add below is an explicit fma()/fmaf().
 *
 * Every function restates, element by element, what the reference's kernels compute (file:line in each comment).
 * The products inside one 16-wide k block of the reference's FP16 kernels are summed in k order here; the Gen9
 * kernels visit them in their packed-layout order, which changes individual roundings but not the precision of the
 * accumulation (the quantity the parity bounds are written against).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ---------------- binary16 ---------------- */

/* Correctly rounded (nearest, ties to even) conversion of a double to binary16 bits; overflow to ±inf, NaN to a
 * quiet NaN. Works on the bits of the double: 53-bit significand, keep 11 bits (normal) or the multiples of 2^-24
 * (subnormal), round on the discarded remainder. */
uint16_t orc_f16_round(double x) {
    uint64_t b;
    memcpy(&b, &x, sizeof b);
    const uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
    b &= 0x7fffffffffffffffULL;
    const int ef = (int)(b >> 52);
    if (ef == 0x7ff) return sign | ((b & 0xfffffffffffffULL) ? 0x7e00 : 0x7c00);
    const int e = ef - 1023;                 /* |x| in [2^e, 2^(e+1)) */
    if (ef == 0 || e < -25) return sign;     /* below half of 2^-24 (or a double subnormal): ±0 */
    const uint64_t m = (b & 0xfffffffffffffULL) | (1ULL << 52);
    int shift, ebits;
    if (e >= -14) { shift = 42; ebits = e + 15; }   /* normal: 11 significant bits */
    else { shift = 28 - e; ebits = 0; }              /* subnormal: units of 2^-24 */
    uint64_t r = m >> shift;
    const uint64_t rem = m & ((1ULL << shift) - 1), half = 1ULL << (shift - 1);
    if (rem > half || (rem == half && (r & 1))) r++;
    if (ebits == 0) return sign | (uint16_t)r;       /* r = 1024 encodes the smallest normal, as it should */
    if (r == 2048) { r = 1024; ebits++; }
    if (ebits >= 31) return sign | 0x7c00;
    return sign | (uint16_t)((ebits << 10) | (r & 0x3ff));
}

double orc_f16_value(uint16_t h) {
    const int s = h >> 15, ef = (h >> 10) & 0x1f, mant = h & 0x3ff;
    double v;
    if (ef == 0x1f) v = mant ? NAN : INFINITY;
    else if (ef == 0) v = ldexp((double)mant, -24);
    else v = ldexp((double)(mant | 0x400), ef - 25);
    return s ? -v : v;
}

/* fma with a single rounding to binary16. The double sum is exact whenever it can matter: the product of two
 * binary16 values has at most 22 significant bits, and when the exponent span of product and addend exceeds the
 * 53 bits of a double the smaller term lies far below half an ulp of the binary16 result. */
static inline double h_fma(double a, double b, double c) { return orc_f16_value(orc_f16_round(a * b + c)); }

/* element (i, j) of op(X): trans ? X[j·ld + i] : X[i·ld + j] */
#define OP(X, t, i, j, ld) ((t) ? (X)[(long)(j) * (ld) + (i)] : (X)[(long)(i) * (ld) + (j)])

/* ---------------- level 3 ---------------- */

/* The reference's FP16 epilogue (reference: lib/kernels/hgemm.cl:558-564, gen9blas_epilog_b): FP32 arithmetic on
 * the FP16 result of the main kernel, alpha·Cp, + beta·C when beta ≠ 0, rounded to FP16. With alpha = 1 and beta = 0
 * it equals the direct write of the main kernel (reference: lib/src/gemm.c:38). */
static uint16_t h_epilogue(double cp, float alpha, float beta, uint16_t c) {
    float v = alpha * (float)cp;
    if (beta != 0.0f) v = v + beta * (float)orc_f16_value(c);
    return orc_f16_round((double)v);
}

/* GEN9BLAS_H: one FP16 accumulator per C element, fma with one rounding per product, k in order
 * (reference: lib/kernels/hgemm.cl:838-868, hgemm_v). */
void orc_gemm_h(int M, int N, int K, int tA, int tB, float alpha, const uint16_t *A, int lda, const uint16_t *B, int ldb,
                float beta, uint16_t *C, int ldc) {
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            double h = 0;
            for (int k = 0; k < K; k++) h = h_fma(orc_f16_value(OP(A, tA, i, k, lda)), orc_f16_value(OP(B, tB, k, j, ldb)), h);
            C[(long)i * ldc + j] = h_epilogue(h, alpha, beta, C[(long)i * ldc + j]);
        }
}

/* GEN9BLAS_HS: the FP16 accumulator runs for KC = 32 products, is added to an FP32 sum and restarts at zero; the
 * result is FP16(f + h) (reference: lib/kernels/hgemm.cl:870-898, hgemm_kc_v; KC: lib/gen9blas.h:32). */
void orc_gemm_hs(int M, int N, int K, int tA, int tB, float alpha, const uint16_t *A, int lda, const uint16_t *B, int ldb,
                 float beta, uint16_t *C, int ldc) {
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            float f = 0.0f;
            double h = 0;
            for (int k = 0; k < K; k++) {
                h = h_fma(orc_f16_value(OP(A, tA, i, k, lda)), orc_f16_value(OP(B, tB, k, j, ldb)), h);
                if ((k + 1) % 32 == 0) { f = f + (float)h; h = 0; }
            }
            const float s = f + (float)h;
            C[(long)i * ldc + j] = h_epilogue(orc_f16_value(orc_f16_round((double)s)), alpha, beta, C[(long)i * ldc + j]);
        }
}

/* GEN9BLAS_S: FP32 fma chain in k order, then alpha·acc (+ beta·C) in FP32 (reference: lib/kernels/sgemm.cl:192-230,
 * sgemm_v + gen9blas_epilog_fb). */
void orc_gemm_s(int M, int N, int K, int tA, int tB, float alpha, const float *A, int lda, const float *B, int ldb,
                float beta, float *C, int ldc) {
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            float acc = 0.0f;
            for (int k = 0; k < K; k++) acc = fmaf(OP(A, tA, i, k, lda), OP(B, tB, k, j, ldb), acc);
            float v = alpha * acc;
            if (beta != 0.0f) v = v + beta * C[(long)i * ldc + j];
            C[(long)i * ldc + j] = v;
        }
}

/* GEN9BLAS_D: FP64 fma chain in k order, FP64 epilogue (reference: lib/kernels/dgemm_core.cl:61-94, dgemm_v; the
 * epilogue is the FP64 copy of gen9blas_epilog_fb made by lib/gen_dgemm.py:30-38). */
void orc_gemm_d(int M, int N, int K, int tA, int tB, double alpha, const double *A, int lda, const double *B, int ldb,
                double beta, double *C, int ldc) {
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            double acc = 0.0;
            for (int k = 0; k < K; k++) acc = fma(OP(A, tA, i, k, lda), OP(B, tB, k, j, ldb), acc);
            double v = alpha * acc;
            if (beta != 0.0) v = v + beta * C[(long)i * ldc + j];
            C[(long)i * ldc + j] = v;
        }
}

/* Skinny C = alpha·A·op(B) + beta·C with FP32 accumulation of the products (exact for FP16 inputs), then
 * beta = 0 ? alpha·t : fma(alpha, t, beta·C), rounded to the element type (reference: lib/kernels/level12.cl:646-801,
 * skinny_k* / skinny_r*; selection lib/src/gemm.c:191-263). es = 2 (FP16 bits) or 4 (FP32). */
static double ld_el(const void *p, long i, int es) {
    return es == 2 ? orc_f16_value(((const uint16_t *)p)[i]) : (double)((const float *)p)[i];
}
static void st_el(void *p, long i, int es, float v) {
    if (es == 2) ((uint16_t *)p)[i] = orc_f16_round((double)v);
    else ((float *)p)[i] = v;
}
void orc_skinny(int es, int M, int N, int K, int tA, int tB, float alpha, const void *A, int lda, const void *B, int ldb,
                float beta, void *C, int ldc) {
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            float t = 0.0f;
            for (int k = 0; k < K; k++) {
                const long ia = tA ? (long)k * lda + i : (long)i * lda + k, ib = tB ? (long)j * ldb + k : (long)k * ldb + j;
                t = fmaf((float)ld_el(A, ia, es), (float)ld_el(B, ib, es), t);
            }
            const long ic = (long)i * ldc + j;
            st_el(C, ic, es, beta == 0.0f ? alpha * t : fmaf(alpha, t, beta * (float)ld_el(C, ic, es)));
        }
}

/* ---------------- levels 1-2 ---------------- */
/* Element i of a vector: p[o + i·inc], o = (n-1)·(-inc) for inc < 0 (reference: lib/src/level12.c:28-30). */
static long voff(int n, int inc) { return inc < 0 ? (long)(n - 1) * -inc : 0; }

/* y = fma(a, x, y): FP32 for FP32 and FP16 storage (FP16 rounded on store), FP64 for FP64
 * (reference: lib/kernels/level12.cl:133-139, axpy). */
void orc_axpy(int es, int n, double a, const void *x, int incx, void *y, int incy) {
    const long ox = voff(n, incx), oy = voff(n, incy);
    for (int i = 0; i < n; i++) {
        const long jx = ox + (long)i * incx, jy = oy + (long)i * incy;
        if (es == 8) ((double *)y)[jy] = fma(a, ((const double *)x)[jx], ((double *)y)[jy]);
        else st_el(y, jy, es, fmaf((float)a, (float)ld_el(x, jx, es), (float)ld_el(y, jy, es)));
    }
}

/* Σ x·y (mode 0), Σ|x| (1), sqrt(Σx²) (2), accumulated in FP64 (reference: lib/kernels/level12.cl:189-214, red;
 * lib/src/level12.c:171-190). */
double orc_reduce(int es, int mode, int n, const void *x, int incx, const void *y, int incy) {
    const long ox = voff(n, incx), oy = voff(n, incy);
    double s = 0.0;
    for (int i = 0; i < n; i++) {
        const long jx = ox + (long)i * incx;
        const double v = es == 8 ? ((const double *)x)[jx] : ld_el(x, jx, es);
        if (mode == 0) {
            const long jy = oy + (long)i * incy;
            s = fma(v, es == 8 ? ((const double *)y)[jy] : ld_el(y, jy, es), s);
        } else if (mode == 1) s += fabs(v);
        else s = fma(v, v, s);
    }
    return mode == 2 ? sqrt(s) : s;
}

/* y = alpha·op(A)·x + beta·y with the sum in the compute type (FP32 for FP16/FP32, FP64 for FP64), then
 * beta = 0 ? alpha·t : fma(alpha, t, beta·y) (reference: lib/kernels/level12.cl:243-423, gemv_n / gemv_t1 + gemv_t2). */
void orc_gemv(int es, int trans, int M, int N, double alpha, const void *A, int lda, const void *x, int incx, double beta,
              void *y, int incy) {
    const int nx = trans ? M : N, ny = trans ? N : M;
    const long ox = voff(nx, incx), oy = voff(ny, incy);
    for (int r = 0; r < ny; r++) {
        const long jy = oy + (long)r * incy;
        if (es == 8) {
            double t = 0.0;
            for (int c = 0; c < nx; c++) {
                const long ia = trans ? (long)c * lda + r : (long)r * lda + c;
                t = fma(((const double *)A)[ia], ((const double *)x)[ox + (long)c * incx], t);
            }
            double *yp = (double *)y + jy;
            *yp = beta == 0.0 ? alpha * t : fma(alpha, t, beta * *yp);
        } else {
            float t = 0.0f;
            for (int c = 0; c < nx; c++) {
                const long ia = trans ? (long)c * lda + r : (long)r * lda + c;
                t = fmaf((float)ld_el(A, ia, es), (float)ld_el(x, ox + (long)c * incx, es), t);
            }
            const float fa = (float)alpha, fb = (float)beta;
            st_el(y, jy, es, fb == 0.0f ? fa * t : fmaf(fa, t, fb * (float)ld_el(y, jy, es)));
        }
    }
}

/* Array helpers for the Python wrapper. */
void orc_f16_round_array(const double *x, uint16_t *h, long n) {
    for (long i = 0; i < n; i++) h[i] = orc_f16_round(x[i]);
}
void orc_f16_value_array(const uint16_t *h, double *x, long n) {
    for (long i = 0; i < n; i++) x[i] = orc_f16_value(h[i]);
}
