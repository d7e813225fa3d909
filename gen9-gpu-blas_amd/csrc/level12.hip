// Level 1-2 entry points (reference: lib/src/level12.c:10-265).
//
// Contract kept from the reference: the type is checked first (GEN9BLAS_HS counts as GEN9BLAS_H), an empty vector
// returns 0, a zero increment is INVALID_ARG, inc < 0 addresses the vector from its lowest address (element 0 at the
// end), gemv checks lda ≥ N and does not read y when beta = 0, reductions return FP64, iamax is 0-based (first
// maximum, NaN skipped). Every call runs one kernel (two for reductions and the transposed GEMV) and waits once.
#include "internal.h"
#include <math.h>

namespace g9 {

typedef long long ll;

// Element size of a level 1/2 type, or an error.
static int l12_es(int type, int *es) {
    G9_TRY(begin());
    if (type == GEN9BLAS_H || type == GEN9BLAS_HS) *es = 2;
    else if (type == GEN9BLAS_S) *es = 4;
    else if (type == GEN9BLAS_D) *es = 8;
    else G9_FAIL(GEN9BLAS_ERR_UNSUPPORTED, "type %d unavailable", type);
    return 0;
}

static void vec(Operand &o, const void *p, int n, int inc, int es) {
    o.host = p;
    o.es = es;
    o.rows = 1;
    o.cols = (ll)(n - 1) * (inc < 0 ? -(ll)inc : inc) + 1;
    o.caller_ld = o.cols;
}
static ll voff(int n, int inc) { return inc < 0 ? (ll)(n - 1) * -(ll)inc : 0; }

#define L12_BEGIN(n, bad_inc)                                                         \
    const double t0_ = now_s();                                                       \
    int es;                                                                           \
    G9_TRY(l12_es(type, &es));                                                        \
    if ((n) <= 0) return 0;                                                           \
    if (bad_inc) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "vector increment 0");

// Two-vector elementwise operation: x (read, or read+written), y (written).
static int two(int es, int n, const void *x, int incx, bool x_written, void *y, int incy, bool y_read, double t0, int op,
               double h11, double h12, double h21, double h22) {
    Operand o[2];
    vec(o[0], x, n, incx, es);
    vec(o[1], y, n, incy, es);
    // a strided y that is written is copied in even when not read: the copy back must keep the gaps
    G9_TRY(resolve(o[0], SLOT_A, true, x_written, false));
    G9_TRY(resolve(o[1], SLOT_B, y_read || (incy != 1 && incy != -1), true, false));
    prof_begin();
    if (op == 0) G9_TRY(launch_axpy(es, n, h11, o[0].dev, voff(n, incx), incx, o[1].dev, voff(n, incy), incy));
    else if (op == 2) G9_TRY(launch_copy(es, n, o[0].dev, voff(n, incx), incx, o[1].dev, voff(n, incy), incy));
    else G9_TRY(launch_rot(es, n, o[0].dev, voff(n, incx), incx, o[1].dev, voff(n, incy), incy, h11, h12, h21, h22, op == 4));
    prof_end();
    G9_TRY(finish(o, 2));
    prof_collect(t0);
    return 0;
}

static int reduction(int type, int mode, int n, const void *x, int incx, const void *y, int incy, double *result) {
    const double t0_ = now_s();
    int es;
    const int ok = l12_es(type, &es);
    // a host result is 0 until the sum is known, as in the reference (reference: lib/src/level12.c:172)
    const int rkind = ok == GEN9BLAS_ERR_NO_DEVICE ? MEM_HOST : mem_kind(result, sizeof(double));
    if (result && (rkind == MEM_HOST || rkind == MEM_PINNED)) *result = 0;
    G9_TRY(ok);
    if (n <= 0) return 0;
    if (!incx || (mode == 0 && !incy)) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "vector increment 0");
    if (!result) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "NULL result pointer");
    if (rkind == MEM_DEVICE_OVERRUN) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "result pointer runs past its device allocation");
    Operand o[2];
    vec(o[0], x, n, incx, es);
    G9_TRY(resolve(o[0], SLOT_A, true, false, false));
    int no = 1;
    if (mode == 0) {
        vec(o[1], y, n, incy, es);
        G9_TRY(resolve(o[1], SLOT_B, true, false, false));
        no = 2;
    }
    // A result pointer in device memory receives the sum in place (no wait in no-wait mode); a host pointer is
    // filled after the wait, from the pinned result slot the final kernel writes (else through a device word and a
    // copy).
    const bool dev_result = rkind == MEM_DEVICE;
    double *slot = dev_result ? nullptr : (double *)result_slot();
    void *res = dev_result ? result : slot;
    if (!res) G9_TRY(scratch(SLOT_Q, 64, &res));
    prof_begin();
    G9_TRY(launch_reduce(es, mode, n, o[0].dev, voff(n, incx), incx, mode == 0 ? o[1].dev : nullptr,
                         mode == 0 ? voff(n, incy) : 0, mode == 0 ? incy : 0, (double *)res));
    prof_end();
    if (dev_result) {
        G9_TRY(finish(o, no));
    } else {
        if (!slot) G9_HIP(hipMemcpyAsync(result, res, sizeof(double), hipMemcpyDeviceToHost, stream));
        const int saved = nowait;
        nowait = 0;   // the result goes through a host pointer: always wait
        const int r = finish(o, no, !slot);
        nowait = saved;
        G9_TRY(r);
        if (slot) *result = *(volatile double *)slot;
    }
    prof_collect(t0_);
    return 0;
}

}  // namespace g9

using namespace g9;

extern "C" {

int gen9blas_axpy(int type, int n, double a, const void *x, int incx, void *y, int incy) {
    L12_BEGIN(n, !incx || !incy);
    return two(es, n, x, incx, false, y, incy, true, t0_, 0, a, 0, 0, 0);
}

int gen9blas_scal(int type, int n, double a, void *x, int incx) {
    L12_BEGIN(n, !incx);
    Operand o[1];
    vec(o[0], x, n, incx, es);
    G9_TRY(resolve(o[0], SLOT_A, true, true, false));
    prof_begin();
    G9_TRY(launch_scal(es, n, a, o[0].dev, voff(n, incx), incx));
    prof_end();
    G9_TRY(finish(o, 1));
    prof_collect(t0_);
    return 0;
}

int gen9blas_copy(int type, int n, const void *x, int incx, void *y, int incy) {
    L12_BEGIN(n, !incx || !incy);
    return two(es, n, x, incx, false, y, incy, false, t0_, 2, 0, 0, 0, 0);
}

int gen9blas_swap(int type, int n, void *x, int incx, void *y, int incy) {
    L12_BEGIN(n, !incx || !incy);
    return two(es, n, x, incx, true, y, incy, true, t0_, 4, 0, 0, 0, 0);
}

int gen9blas_rot(int type, int n, void *x, int incx, void *y, int incy, double c, double s) {
    L12_BEGIN(n, !incx || !incy);
    return two(es, n, x, incx, true, y, incy, true, t0_, 3, c, s, -s, c);
}

// H from param (BLAS convention; reference: lib/src/level12.c:92-107): flag -1 full [h11 h12; h21 h22], 0 unit
// diagonal, 1 [h11 1; -1 h22], -2 identity. param[1..4] = h11, h21, h12, h22.
int gen9blas_rotm(int type, int n, void *x, int incx, void *y, int incy, const double *param) {
    if (!param) {
        int es;
        G9_TRY(l12_es(type, &es));
        G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "rotm: NULL param");
    }
    const double fl = param[0];
    if (fl == -2.0) return 0;   // identity: nothing to do
    double h11, h12, h21, h22;
    if (fl < 0) { h11 = param[1]; h21 = param[2]; h12 = param[3]; h22 = param[4]; }
    else if (fl == 0) { h11 = 1; h21 = param[2]; h12 = param[3]; h22 = 1; }
    else { h11 = param[1]; h21 = -1; h12 = 1; h22 = param[4]; }
    L12_BEGIN(n, !incx || !incy);
    return two(es, n, x, incx, true, y, incy, true, t0_, 3, h11, h12, h21, h22);
}

int gen9blas_dot(int type, int n, const void *x, int incx, const void *y, int incy, double *result) {
    return reduction(type, 0, n, x, incx, y, incy, result);
}
int gen9blas_asum(int type, int n, const void *x, int incx, double *result) {
    return reduction(type, 1, n, x, incx, nullptr, 0, result);
}
int gen9blas_nrm2(int type, int n, const void *x, int incx, double *result) {
    return reduction(type, 2, n, x, incx, nullptr, 0, result);
}

int gen9blas_iamax(int type, int n, const void *x, int incx, int64_t *result) {
    if (result) *result = -1;
    L12_BEGIN(n, !incx);
    if (!result) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "NULL result pointer");
    Operand o[1];
    vec(o[0], x, n, incx, es);
    G9_TRY(resolve(o[0], SLOT_A, true, false, false));
    // the final kernel writes the index into the pinned result slot (else a device word, copied after)
    long long *slot = (long long *)result_slot();
    void *res = slot;
    if (!res) G9_TRY(scratch(SLOT_Q, 64, &res));
    prof_begin();
    G9_TRY(launch_iamax(es, n, o[0].dev, voff(n, incx), incx, (long long *)res));
    prof_end();
    long long idx = 0;
    if (slot) {
        G9_TRY(wait_done());
        idx = *(volatile long long *)slot;
    } else {
        G9_HIP(hipMemcpyAsync(&idx, res, sizeof idx, hipMemcpyDeviceToHost, stream));
        G9_TRY(wait_stream());
    }
    *result = idx;
    prof_collect(t0_);
    return 0;
}

int gen9blas_gemv(int type, int trans, int M, int N, double alpha, const void *A, int lda, const void *x, int incx, double beta,
                  void *y, int incy) {
    L12_BEGIN(M < N ? M : N, !incx || !incy);
    if (lda < N) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "lda < N");
    trans = trans != 0;
    const int nx = trans ? M : N, ny = trans ? N : M;
    Operand o[3];
    o[0].host = A; o[0].es = es; o[0].rows = M; o[0].cols = N; o[0].caller_ld = lda;
    vec(o[1], x, nx, incx, es);
    vec(o[2], y, ny, incy, es);
    G9_TRY(resolve(o[0], SLOT_A, true, false, true));
    G9_TRY(resolve(o[1], SLOT_B, true, false, false));
    G9_TRY(resolve(o[2], SLOT_C, beta != 0.0 || (incy != 1 && incy != -1), true, false));
    prof_begin();
    G9_TRY(launch_gemv(es, trans, M, N, alpha, o[0].dev, o[0].ld, o[1].dev, voff(nx, incx), incx, beta, o[2].dev,
                       voff(ny, incy), incy));
    prof_end();
    G9_TRY(finish(o, 3));
    prof_collect(t0_);
    return 0;
}

int gen9blas_ger(int type, int M, int N, double alpha, const void *x, int incx, const void *y, int incy, void *A, int lda) {
    L12_BEGIN(M < N ? M : N, !incx || !incy);
    if (lda < N) G9_FAIL(GEN9BLAS_ERR_INVALID_ARG, "lda < N");
    Operand o[3];
    o[0].host = A; o[0].es = es; o[0].rows = M; o[0].cols = N; o[0].caller_ld = lda;
    vec(o[1], x, M, incx, es);
    vec(o[2], y, N, incy, es);
    G9_TRY(resolve(o[0], SLOT_A, true, true, true));
    G9_TRY(resolve(o[1], SLOT_B, true, false, false));
    G9_TRY(resolve(o[2], SLOT_C, true, false, false));
    prof_begin();
    G9_TRY(launch_ger(es, M, N, alpha, o[1].dev, voff(M, incx), incx, o[2].dev, voff(N, incy), incy, o[0].dev, o[0].ld));
    prof_end();
    G9_TRY(finish(o, 3));
    prof_collect(t0_);
    return 0;
}

// ROTG / ROTMG work on four numbers and run on the host, as in the reference (reference: lib/src/level12.c:109-162).
// ROTG follows the overflow-safe scaling of Netlib BLAS 3.10 (Anderson, "Algorithm 978: Safe scaling in the Level 1
// BLAS", 2017): r = ±scl·sqrt((a/scl)² + (b/scl)²) with scl clamped to [safmin, 1/safmin].
void gen9blas_rotg(float *a, float *b, float *c, float *s) {
    const float safmin = 1.17549435e-38f, safmax = 1.0f / safmin;
    const float av = *a, bv = *b, an = fabsf(av), bn = fabsf(bv);
    if (bn == 0) { *c = 1; *s = 0; *b = 0; return; }
    if (an == 0) { *c = 0; *s = 1; *a = bv; *b = 1; return; }
    const float big = an > bn ? an : bn;
    const float scl = big < safmin ? safmin : big > safmax ? safmax : big;
    const float sigma = an > bn ? copysignf(1.0f, av) : copysignf(1.0f, bv);
    const float ua = av / scl, ub = bv / scl;
    const float r = sigma * scl * sqrtf(ua * ua + ub * ub);
    *c = av / r;
    *s = bv / r;
    const float z = an > bn ? *s : (*c != 0 ? 1.0f / *c : 1.0f);
    *a = r;
    *b = z;
}

// ROTMG: the modified Givens construction of Lawson, Hanson, Kincaid and Krogh (ACM TOMS 5, 1979) with the rescaling
// by gamma = 4096 that keeps d1, d2 inside [1/gamma², gamma²]. param receives the flag and the entries of H.
void gen9blas_rotmg(float *d1, float *d2, float *x1, float y1, float *param) {
    const float gam = 4096.0f, gamsq = gam * gam, rgamsq = 1.0f / gamsq;
    float flag, h11 = 0, h12 = 0, h21 = 0, h22 = 0;
    if (*d1 < 0) {
        flag = -1;
        *d1 = *d2 = *x1 = 0;
    } else {
        const float p2 = *d2 * y1;
        if (p2 == 0) { param[0] = -2; return; }
        const float p1 = *d1 * *x1, q2 = p2 * y1, q1 = p1 * *x1;
        if (fabsf(q1) > fabsf(q2)) {
            h21 = -y1 / *x1;
            h12 = p2 / p1;
            const float u = 1 - h12 * h21;
            if (u > 0) {
                flag = 0;
                *d1 /= u;
                *d2 /= u;
                *x1 *= u;
            } else {
                flag = -1;
                h11 = h12 = h21 = h22 = 0;
                *d1 = *d2 = *x1 = 0;
            }
        } else if (q2 < 0) {
            flag = -1;
            h11 = h12 = h21 = h22 = 0;
            *d1 = *d2 = *x1 = 0;
        } else {
            flag = 1;
            h11 = p1 / p2;
            h22 = *x1 / y1;
            const float u = 1 + h11 * h22, t = *d2 / u;
            *d2 = *d1 / u;
            *d1 = t;
            *x1 = y1 * u;
        }
        // rescale d1 (and the first row of H) into range
        if (*d1 != 0)
            while (*d1 <= rgamsq || *d1 >= gamsq) {
                if (flag == 0) { h11 = 1; h22 = 1; }
                else if (flag > 0) { h21 = -1; h12 = 1; }
                flag = -1;
                if (*d1 <= rgamsq) { *d1 *= gamsq; *x1 /= gam; h11 /= gam; h12 /= gam; }
                else { *d1 /= gamsq; *x1 *= gam; h11 *= gam; h12 *= gam; }
            }
        if (*d2 != 0)
            while (fabsf(*d2) <= rgamsq || fabsf(*d2) >= gamsq) {
                if (flag == 0) { h11 = 1; h22 = 1; }
                else if (flag > 0) { h21 = -1; h12 = 1; }
                flag = -1;
                if (fabsf(*d2) <= rgamsq) { *d2 *= gamsq; h21 /= gam; h22 /= gam; }
                else { *d2 /= gamsq; h21 *= gam; h22 *= gam; }
            }
    }
    if (flag < 0) { param[1] = h11; param[2] = h21; param[3] = h12; param[4] = h22; }
    else if (flag == 0) { param[2] = h21; param[3] = h12; }
    else { param[1] = h11; param[4] = h22; }
    param[0] = flag;
}

}  // extern "C"
