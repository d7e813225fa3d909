"""ctypes bindings of libgen9blas_blas.so (the BLAS / CBLAS shim) shared by its CPU and GPU tests."""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.realpath(__file__)))
SHIM = os.path.join(ROOT, "gen9-gpu-blas_amd", "libgen9blas_blas.so")
ROW, COL, NT, T = 101, 102, 111, 112
OWN = {f"cblas_{p}{f}" for p in "sd" for f in ("gemm", "gemv", "ger", "axpy", "scal", "copy", "swap", "rot", "rotm",
                                               "dot", "asum", "nrm2")}
OWN |= {f"cblas_i{p}amax" for p in "sd"} | {f"{p}{f}_" for p in "sd" for f in ("gemm", "gemv", "ger")}
OWN |= {"cblas_sdsdot", "cblas_dsdot"}
L3 = ("symm", "syrk", "syr2k", "trmm", "trsm")
OWN |= {f"cblas_{p}{f}" for p in "sd" for f in L3} | {f"{p}{f}_" for p in "sd" for f in L3}
SIDE, UPLO, DIAG = {"L": 141, "R": 142}, {"U": 121, "L": 122}, {"N": 131, "U": 132}

i, f, d, p = ctypes.c_int, ctypes.c_float, ctypes.c_double, ctypes.c_void_p


def load():
    L = ctypes.CDLL(SHIM)
    for P, R in (("s", f), ("d", d)):
        getattr(L, f"cblas_{P}gemm").argtypes = [i, i, i, i, i, i, R, p, i, p, i, R, p, i]
        getattr(L, f"cblas_{P}gemv").argtypes = [i, i, i, i, R, p, i, p, i, R, p, i]
        getattr(L, f"cblas_{P}ger").argtypes = [i, i, i, R, p, i, p, i, p, i]
        getattr(L, f"cblas_{P}axpy").argtypes = [i, R, p, i, p, i]
        getattr(L, f"cblas_{P}scal").argtypes = [i, R, p, i]
        getattr(L, f"cblas_{P}dot").argtypes = [i, p, i, p, i]
        getattr(L, f"cblas_{P}dot").restype = R
        getattr(L, f"cblas_{P}asum").argtypes = [i, p, i]
        getattr(L, f"cblas_{P}asum").restype = R
        getattr(L, f"cblas_{P}nrm2").argtypes = [i, p, i]
        getattr(L, f"cblas_{P}nrm2").restype = R
        getattr(L, f"cblas_i{P}amax").argtypes = [i, p, i]
        getattr(L, f"cblas_i{P}amax").restype = ctypes.c_size_t
        getattr(L, f"cblas_{P}symm").argtypes = [i, i, i, i, i, R, p, i, p, i, R, p, i]
        getattr(L, f"cblas_{P}syrk").argtypes = [i, i, i, i, i, R, p, i, R, p, i]
        getattr(L, f"cblas_{P}syr2k").argtypes = [i, i, i, i, i, R, p, i, p, i, R, p, i]
        getattr(L, f"cblas_{P}trmm").argtypes = [i, i, i, i, i, i, i, R, p, i, p, i]
        getattr(L, f"cblas_{P}trsm").argtypes = [i, i, i, i, i, i, i, R, p, i, p, i]
        getattr(L, f"cblas_{P}symv").argtypes = [i, i, i, R, p, i, p, i, R, p, i]
    L.cblas_sdsdot.argtypes = [i, f, p, i, p, i]
    L.cblas_sdsdot.restype = f
    L.cblas_dsdot.argtypes = [i, p, i, p, i]
    L.cblas_dsdot.restype = d
    return L


def ptr(a):
    return ctypes.c_void_p(a.data_ptr() if hasattr(a, "data_ptr") else a.ctypes.data)


def ref_error(C, ref, scale):
    return float(np.max(np.abs(np.asarray(C, np.float64) - ref) / np.maximum(scale, 1e-300)))


def fortran_gemm(L, P, ta, tb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc):
    """Column-major Fortran ?gemm_ with arguments by reference."""
    R = f if P == "s" else d
    fn = getattr(L, f"{P}gemm_")
    args = [ctypes.c_char_p(ta.encode()), ctypes.c_char_p(tb.encode())] + [ctypes.byref(i(v)) for v in (M, N, K)]
    args += [ctypes.byref(R(alpha)), ptr(A), ctypes.byref(i(lda)), ptr(B), ctypes.byref(i(ldb)), ctypes.byref(R(beta)),
             ptr(C), ctypes.byref(i(ldc))]
    fn(*args)


# ---------------- level 3 beyond GEMM through the shim ----------------
def to_mem(X, order, torch=None):
    """A logical matrix X in the memory layout of `order` (ROW; COL or "F": column-major), on the device when torch is
    given: (object, leading dimension, function reading an object of that layout back as a logical float64 matrix)."""
    col = order != ROW
    m = np.array(X.T if col else X, order="C")   # always a copy: the call may write it
    ld = X.shape[0] if col else X.shape[1]
    if torch is not None:
        m = torch.from_numpy(m).cuda()

    def back(o):
        a = np.asarray(o.cpu().numpy() if hasattr(o, "cpu") else o, np.float64)
        return a.T if col else a
    return m, ld, back


def call_l3(L, P, order, op, opt, dims, alpha, beta, A, B, C):
    """One call of ?symm / ?syrk / ?syr2k / ?trmm / ?trsm: CBLAS in `order` (ROW or COL) or Fortran (order "F").
    opt: side, uplo, trans, diag letters as BLAS names them; dims: (M, N) or (N, K) for SYRK/SYR2K; A, B, C:
    (object, ld) pairs from to_mem (C unused by TRMM/TRSM, B unused by SYRK)."""
    R = f if P == "s" else d
    side, uplo, tr, dg = opt
    if order == "F":
        ch = lambda c: ctypes.c_char_p(c.encode())
        ri = lambda v: ctypes.byref(i(v))
        rr = lambda v: ctypes.byref(R(v))
        args = {"symm": lambda: [ch(side), ch(uplo), ri(dims[0]), ri(dims[1]), rr(alpha), ptr(A[0]), ri(A[1]),
                                 ptr(B[0]), ri(B[1]), rr(beta), ptr(C[0]), ri(C[1])],
                "syrk": lambda: [ch(uplo), ch(tr), ri(dims[0]), ri(dims[1]), rr(alpha), ptr(A[0]), ri(A[1]), rr(beta),
                                 ptr(C[0]), ri(C[1])],
                "syr2k": lambda: [ch(uplo), ch(tr), ri(dims[0]), ri(dims[1]), rr(alpha), ptr(A[0]), ri(A[1]), ptr(B[0]),
                                  ri(B[1]), rr(beta), ptr(C[0]), ri(C[1])],
                "trmm": lambda: [ch(side), ch(uplo), ch(tr), ch(dg), ri(dims[0]), ri(dims[1]), rr(alpha), ptr(A[0]),
                                 ri(A[1]), ptr(B[0]), ri(B[1])]}
        args["trsm"] = args["trmm"]
        getattr(L, f"{P}{op}_")(*args[op]())
        return
    t = T if tr == "T" else NT
    fn = getattr(L, f"cblas_{P}{op}")
    if op == "symm":
        fn(order, SIDE[side], UPLO[uplo], dims[0], dims[1], alpha, ptr(A[0]), A[1], ptr(B[0]), B[1], beta, ptr(C[0]),
           C[1])
    elif op == "syrk":
        fn(order, UPLO[uplo], t, dims[0], dims[1], alpha, ptr(A[0]), A[1], beta, ptr(C[0]), C[1])
    elif op == "syr2k":
        fn(order, UPLO[uplo], t, dims[0], dims[1], alpha, ptr(A[0]), A[1], ptr(B[0]), B[1], beta, ptr(C[0]), C[1])
    else:
        fn(order, SIDE[side], UPLO[uplo], t, DIAG[dg], dims[0], dims[1], alpha, ptr(A[0]), A[1], ptr(B[0]), B[1])


def l3_case(rng, dt, op, opt, dims):
    """Random operands of one level-3 call as logical matrices (A, B, C), TRSM's A well conditioned."""
    side, uplo, tr, dg = opt
    if op in ("syrk", "syr2k"):
        N, K = dims
        shape = (K, N) if tr == "T" else (N, K)
        return (rng.uniform(-1, 1, shape).astype(dt), rng.uniform(-1, 1, shape).astype(dt),
                rng.uniform(-1, 1, (N, N)).astype(dt))
    M, N = dims
    n = M if side == "L" else N
    A = rng.uniform(-1, 1, (n, n))
    if op == "trsm":
        A *= 1.0 / n
        A[np.diag_indices(n)] = 123.0 if dg == "U" else 1.0   # unit diagonal: the stored one is not read
    return A.astype(dt), rng.uniform(-1, 1, (M, N)).astype(dt), rng.uniform(-1, 1, (M, N)).astype(dt)


def l3_ref(op, opt, alpha, beta, A, B, C):
    """float64 closed form of a level-3 call on logical matrices: (result, scale, mask of the entries it defines).
    TRSM: scale is None (the check is on the solution error)."""
    side, uplo, tr, dg = opt
    A, B, C = (np.asarray(x, np.float64) for x in (A, B, C))
    tri = np.tril if uplo == "L" else np.triu
    if op == "symm":
        S = tri(A) + tri(A, -1 if uplo == "L" else 1).T
        P, Pa = (S @ B, np.abs(S) @ np.abs(B)) if side == "L" else (B @ S, np.abs(B) @ np.abs(S))
        return alpha * P + beta * C, abs(alpha) * Pa + abs(beta * C), None
    if op in ("syrk", "syr2k"):
        oA, oB = (A.T, B.T) if tr == "T" else (A, B)
        if op == "syrk":
            P, Pa = oA @ oA.T, np.abs(oA) @ np.abs(oA).T
        else:
            P = oA @ oB.T + oB @ oA.T
            Pa = np.abs(oA) @ np.abs(oB).T + np.abs(oB) @ np.abs(oA).T
        mask = tri(np.ones(C.shape, bool))
        return alpha * P + beta * C, abs(alpha) * Pa + abs(beta * C), mask
    Tm = tri(A)
    if dg == "U":
        np.fill_diagonal(Tm, 1.0)
    Tm = Tm.T if tr == "T" else Tm
    if op == "trmm":
        P, Pa = (Tm @ B, np.abs(Tm) @ np.abs(B)) if side == "L" else (B @ Tm, np.abs(B) @ np.abs(Tm))
        return alpha * P, abs(alpha) * Pa, None
    X = np.linalg.solve(Tm, alpha * B) if side == "L" else np.linalg.solve(Tm.T, alpha * B.T).T
    return X, None, None


def l3_error(op, got, ref, scale, mask):
    if scale is None:
        return float(np.abs(got - ref).max() / np.abs(ref).max())
    e = np.abs(got - ref) / np.maximum(scale, 1e-300)
    return float((e[mask] if mask is not None else e).max())


L3_OPTS = {"symm": [(s, u, "N", "N") for s in "LR" for u in "UL"],
           "syrk": [("L", u, t, "N") for u in "UL" for t in "NT"],
           "syr2k": [("L", u, t, "N") for u in "UL" for t in "NT"],
           "trmm": [(s, u, t, dg) for s in "LR" for u in "UL" for t in "NT" for dg in "NU"],
           "trsm": [(s, u, t, dg) for s in "LR" for u in "UL" for t in "NT" for dg in "NU"]}
L3_TOL = {"s": 1e-5, "d": 1e-12}   # BLAS results (normwise per entry); TRSM solution error: 1e-4 / 1e-12
L3_TRSM_TOL = {"s": 1e-4, "d": 1e-12}


# ---------------- level 2 on symmetric, triangular, band and packed matrices through the shim ----------------
L2_SYM = ("symv", "sbmv", "spmv")
L2_TRI = ("trmv", "trsv", "tbmv", "tbsv", "tpmv", "tpsv")
L2_RANK = ("syr", "syr2", "spr", "spr2")
L2 = L2_SYM + L2_TRI + L2_RANK + ("gbmv",)
OWN |= {f"cblas_{p}{f}" for p in "sd" for f in L2} | {f"{p}{f}_" for p in "sd" for f in L2}


def band_rows(D, KL, KU):
    """Row-major band array of D (element (r, c) at [r, KL + c − r])."""
    M, N = D.shape
    P = np.zeros((M, KL + KU + 1), D.dtype)
    for r in range(M):
        for c in range(max(0, r - KL), min(N, r + KU + 1)):
            P[r, KL + c - r] = D[r, c]
    return P


def packed_rows(T, uplo):
    return T[np.triu_indices(T.shape[0])] if uplo == "U" else T[np.tril_indices(T.shape[0])]


def l2_storage(op, D, uplo, K, KL, KU, order):
    """Memory of the matrix operand for `order` (ROW; COL or "F": column-major): the column-major storage of a
    matrix is the row-major storage of its transpose (band widths swapped, packed triangle flipped)."""
    col = order != ROW
    X = D.T if col else D
    fl = {"U": "L", "L": "U"}[uplo] if col else uplo
    if op in ("gbmv",):
        return band_rows(X, KU, KL) if col else band_rows(X, KL, KU), KL + KU + 1
    if op in ("sbmv", "tbmv", "tbsv"):
        lo, up = (K, 0) if fl == "L" else (0, K)
        return band_rows(X, lo, up), K + 1
    if op in ("spmv", "tpmv", "tpsv", "spr", "spr2"):
        return packed_rows(X, fl), 0
    return np.array(X, order="C"), D.shape[1]


def call_l2(L, P, order, op, o, m, n, K, KL, KU, alpha, beta, A, lda, x, incx, y, incy):
    """One level-2 call: CBLAS in `order` or Fortran ("F"); o = (uplo, trans, diag) letters; A, x, y device tensors
    or NumPy arrays (y unused where the routine has none)."""
    R = f if P == "s" else d
    uplo, tr, dg = o
    if order == "F":
        ch = lambda c: ctypes.c_char_p(c.encode())
        ri = lambda v: ctypes.byref(i(v))
        rr = lambda v: ctypes.byref(R(v))
        a = {"symv": [ch(uplo), ri(n), rr(alpha), ptr(A), ri(lda), ptr(x), ri(incx), rr(beta), ptr(y), ri(incy)],
             "sbmv": [ch(uplo), ri(n), ri(K), rr(alpha), ptr(A), ri(lda), ptr(x), ri(incx), rr(beta), ptr(y), ri(incy)],
             "spmv": [ch(uplo), ri(n), rr(alpha), ptr(A), ptr(x), ri(incx), rr(beta), ptr(y), ri(incy)],
             "trmv": [ch(uplo), ch(tr), ch(dg), ri(n), ptr(A), ri(lda), ptr(x), ri(incx)],
             "tbmv": [ch(uplo), ch(tr), ch(dg), ri(n), ri(K), ptr(A), ri(lda), ptr(x), ri(incx)],
             "tpmv": [ch(uplo), ch(tr), ch(dg), ri(n), ptr(A), ptr(x), ri(incx)],
             "syr": [ch(uplo), ri(n), rr(alpha), ptr(x), ri(incx), ptr(A), ri(lda)],
             "syr2": [ch(uplo), ri(n), rr(alpha), ptr(x), ri(incx), ptr(y), ri(incy), ptr(A), ri(lda)],
             "spr": [ch(uplo), ri(n), rr(alpha), ptr(x), ri(incx), ptr(A)],
             "spr2": [ch(uplo), ri(n), rr(alpha), ptr(x), ri(incx), ptr(y), ri(incy), ptr(A)],
             "gbmv": [ch(tr), ri(m), ri(n), ri(KL), ri(KU), rr(alpha), ptr(A), ri(lda), ptr(x), ri(incx), rr(beta),
                      ptr(y), ri(incy)]}
        a["trsv"], a["tbsv"], a["tpsv"] = a["trmv"], a["tbmv"], a["tpmv"]
        getattr(L, f"{P}{op}_")(*a[op])
        return
    u, t, dd = UPLO[uplo], T if tr == "T" else NT, DIAG[dg]
    c = lambda v: R(v)
    a = {"symv": [order, u, n, c(alpha), ptr(A), lda, ptr(x), incx, c(beta), ptr(y), incy],
         "sbmv": [order, u, n, K, c(alpha), ptr(A), lda, ptr(x), incx, c(beta), ptr(y), incy],
         "spmv": [order, u, n, c(alpha), ptr(A), ptr(x), incx, c(beta), ptr(y), incy],
         "trmv": [order, u, t, dd, n, ptr(A), lda, ptr(x), incx],
         "tbmv": [order, u, t, dd, n, K, ptr(A), lda, ptr(x), incx],
         "tpmv": [order, u, t, dd, n, ptr(A), ptr(x), incx],
         "syr": [order, u, n, c(alpha), ptr(x), incx, ptr(A), lda],
         "syr2": [order, u, n, c(alpha), ptr(x), incx, ptr(y), incy, ptr(A), lda],
         "spr": [order, u, n, c(alpha), ptr(x), incx, ptr(A)],
         "spr2": [order, u, n, c(alpha), ptr(x), incx, ptr(y), incy, ptr(A)],
         "gbmv": [order, t, m, n, KL, KU, c(alpha), ptr(A), lda, ptr(x), incx, c(beta), ptr(y), incy]}
    a["trsv"], a["tbsv"], a["tpsv"] = a["trmv"], a["tbmv"], a["tpmv"]
    getattr(L, f"cblas_{P}{op}")(*a[op])


def l2_opts(op):
    if op in L2_SYM or op in L2_RANK:
        return [(u, "N", "N") for u in "UL"]
    if op == "gbmv":
        return [("U", t, "N") for t in "NT"]
    return [(u, t, dg) for u in "UL" for t in "NT" for dg in "NU"]


def l2_case(rng, dt, op, o, n, K):
    """Logical operands of one call: (D, x, y, m, KL, KU). D is the logical matrix with the entries the routine reads
    (band / triangle applied); solves get a well-conditioned D."""
    uplo, tr, dg = o
    m, KL, KU = n, 0, 0
    if op == "gbmv":
        m, KL, KU = n + 7, 3, K
    D = rng.uniform(-1, 1, (m, n))
    ii, jj = np.indices(D.shape)
    if op == "gbmv":
        D *= (jj - ii >= -KL) & (jj - ii <= KU)
    elif op in ("sbmv", "tbmv", "tbsv"):
        D *= np.abs(jj - ii) <= K
    if op in ("trsv", "tbsv", "tpsv"):
        D = D / n
        D[np.diag_indices(n)] = 1.5 + rng.uniform(0, 1, n)
    nx = m if (op == "gbmv" and tr == "T") else n
    ny = n if (op == "gbmv" and tr == "T") else m
    return D.astype(dt), rng.uniform(-1, 1, nx).astype(dt), rng.uniform(-1, 1, ny).astype(dt), m, KL, KU


def l2_ref(op, o, alpha, beta, D, x, y):
    """float64 result and scale of one call on logical operands (solves: scale None)."""
    uplo, tr, dg = o
    D, X, Y = (np.asarray(v, np.float64) for v in (D, x, y))
    tri = np.tril if uplo == "L" else np.triu
    if op in L2_SYM:
        S = tri(D) + tri(D).T - np.diag(np.diag(D))
        return alpha * S @ X + beta * Y, abs(alpha) * np.abs(S) @ np.abs(X) + abs(beta * Y)
    if op == "gbmv":
        Op = D.T if tr == "T" else D
        return alpha * Op @ X + beta * Y, abs(alpha) * np.abs(Op) @ np.abs(X) + abs(beta * Y)
    if op in L2_TRI:
        Tm = tri(D)
        if dg == "U":
            np.fill_diagonal(Tm, 1.0)
        Op = Tm.T if tr == "T" else Tm
        if op in ("trmv", "tbmv", "tpmv"):
            return Op @ X, np.abs(Op) @ np.abs(X)
        from scipy.linalg import solve_triangular
        return solve_triangular(Op, X, lower=(uplo == "L") != (tr == "T")), None
    # rank updates: the full logical matrix after the update of the `uplo` triangle
    upd = np.outer(X, X) if op in ("syr", "spr") else np.outer(X, Y) + np.outer(Y, X)
    sc = np.outer(np.abs(X), np.abs(X)) if op in ("syr", "spr") else np.outer(np.abs(X), np.abs(Y)) * 2
    mask = tri(np.ones(D.shape, bool))
    return np.where(mask, D + alpha * upd, D), np.abs(D) + abs(alpha) * sc


def l2_result(op, o, order, A_mem, x_mem, y_mem, n, K, KL, KU, dt):
    """The logical result read back from memory: the vector (x or y) or, for rank updates, the logical matrix."""
    host = lambda v: np.asarray(v.cpu().numpy() if hasattr(v, "cpu") else v, np.float64)
    if op in L2_TRI:
        return host(x_mem)
    if op not in L2_RANK:
        return host(y_mem)
    a = host(A_mem)
    uplo = o[0]
    col = order != ROW
    fl = {"U": "L", "L": "U"}[uplo] if col else uplo
    if op in ("syr", "syr2"):
        return a.T if col else a
    Tm = np.zeros((n, n))
    Tm[np.triu_indices(n) if fl == "U" else np.tril_indices(n)] = a
    return Tm.T if col else Tm


def l2_run(L, P, op, o, order, n, K, rng, dt, torch=None, alpha=0.75, beta=-0.5):
    """One level-2 call through the shim on fresh operands: (error, routes checked by the caller). Solves: error of the
    solution relative to its max; rank updates: over the updated triangle (full storage: the whole matrix, since the
    other triangle must stay as it was)."""
    D, x, y, m, KL, KU = l2_case(rng, dt, op, o, n, K)
    A_mem, lda = l2_storage(op, D, o[0], K, KL, KU, order)
    A_mem = np.array(A_mem, dt)
    xm, ym = x.copy(), y.copy()
    if torch is not None:
        A_mem, xm, ym = (torch.from_numpy(v).cuda() for v in (A_mem, xm, ym))
    call_l2(L, P, order, op, o, m, n, K, KL, KU, alpha, beta, A_mem, lda, xm, 1, ym, 1)   # logical shape, any order
    if torch is not None:
        torch.cuda.synchronize()
    got = l2_result(op, o, order, A_mem, xm, ym, n, K, KL, KU, dt)
    ref, scale = l2_ref(op, o, alpha, beta, D, x, y)
    if scale is None:
        return float(np.abs(got - ref).max() / np.abs(ref).max())
    if op in ("spr", "spr2"):
        mask = (np.tril if o[0] == "L" else np.triu)(np.ones((n, n), bool))
        got, ref, scale = got[mask], ref[mask], scale[mask]
    return float((np.abs(got - ref) / np.maximum(scale, 1e-300)).max())


# ---------------- LD_PRELOAD interposition: an unmodified program linked against another BLAS ----------------
# stub "system BLAS" the program is linked against: its GEMMs write -1 everywhere, so results tell which library ran
STUB_BLAS_C = r"""
void cblas_sgemm(int o, int ta, int tb, int M, int N, int K, float al, const float *A, int lda, const float *B, int ldb,
                 float be, float *C, int ldc) {
    for (int i = 0; i < (o == 101 ? M : N); i++) for (int j = 0; j < (o == 101 ? N : M); j++) C[(long)i * ldc + j] = -1.f;
}
void sgemm_(const char *ta, const char *tb, const int *M, const int *N, const int *K, const float *al, const float *A,
            const int *lda, const float *B, const int *ldb, const float *be, float *C, const int *ldc) {
    for (int j = 0; j < *N; j++) for (int i = 0; i < *M; i++) C[(long)j * *ldc + i] = -1.f;
}
"""
# the program: a row-major CBLAS call and a column-major Fortran call, each checked against a float64 reference on
# every 32nd row; prints "<name> maxrel=<error>" per call
PROG_C = r"""
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
void cblas_sgemm(int, int, int, int, int, int, float, const float *, int, const float *, int, float, float *, int);
void sgemm_(const char *, const char *, const int *, const int *, const int *, const float *, const float *, const int *,
            const float *, const int *, const float *, float *, const int *);
static float rnd(unsigned *s) { *s = *s * 1664525u + 1013904223u; return (float)((*s >> 8) & 0xffff) / 32768.f - 1.f; }
int main(void) {
    unsigned s = 7;
    int M = 1024, N = 768, K = 640;   /* 2MNK just above the shim's 1e9-flop level-3 threshold */
    float *A = malloc(sizeof(float) * M * K), *B = malloc(sizeof(float) * K * N), *C = malloc(sizeof(float) * M * N);
    for (long i = 0; i < (long)M * K; i++) A[i] = rnd(&s);
    for (long i = 0; i < (long)K * N; i++) B[i] = rnd(&s);
    cblas_sgemm(101, 111, 111, M, N, K, 1.f, A, K, B, N, 0.f, C, N);
    double worst = 0;
    for (int i = 0; i < M; i += 32)
        for (int j = 0; j < N; j++) {
            double r = 0, a = 0;
            for (int k = 0; k < K; k++) { r += (double)A[(long)i * K + k] * B[(long)k * N + j]; a += fabs((double)A[(long)i * K + k] * B[(long)k * N + j]); }
            const double e = fabs(C[(long)i * N + j] - r) / a;
            if (e > worst) worst = e;
        }
    printf("cblas_sgemm maxrel=%.3e\n", worst);
    /* Fortran: column-major C (m x n) = A (m x k) * B (k x n) */
    int m = 800, n = 900, k = 700;
    float one = 1.f, zero = 0.f;
    float *a = malloc(sizeof(float) * m * k), *b = malloc(sizeof(float) * k * n), *c = malloc(sizeof(float) * m * n);
    for (long i = 0; i < (long)m * k; i++) a[i] = rnd(&s);
    for (long i = 0; i < (long)k * n; i++) b[i] = rnd(&s);
    sgemm_("N", "N", &m, &n, &k, &one, a, &m, b, &k, &zero, c, &m);
    worst = 0;
    for (int i = 0; i < m; i += 32)
        for (int j = 0; j < n; j++) {
            double r = 0, t = 0;
            for (int q = 0; q < k; q++) { r += (double)a[(long)q * m + i] * b[(long)j * k + q]; t += fabs((double)a[(long)q * m + i] * b[(long)j * k + q]); }
            const double e = fabs(c[(long)j * m + i] - r) / t;
            if (e > worst) worst = e;
        }
    printf("sgemm_ maxrel=%.3e\n", worst);
    return 0;
}
"""


def build_preload_program(tmp):
    """Compiles the stub BLAS (libstubblas.so) and the program linked against it (rpath to tmp) with gcc; returns the
    program's path."""
    import subprocess
    tmp = str(tmp)
    with open(os.path.join(tmp, "stub.c"), "w") as f:
        f.write(STUB_BLAS_C)
    with open(os.path.join(tmp, "prog.c"), "w") as f:
        f.write(PROG_C)
    subprocess.run(["gcc", "-O2", "-shared", "-fPIC", "-o", os.path.join(tmp, "libstubblas.so"),
                    os.path.join(tmp, "stub.c")], check=True)
    prog = os.path.join(tmp, "prog")
    subprocess.run(["gcc", "-O2", "-o", prog, os.path.join(tmp, "prog.c"), "-L" + tmp, "-lstubblas",
                    "-Wl,-rpath," + tmp, "-lm"], check=True)
    return prog


def run_preload_program(prog, preload, extra_env=None):
    """Runs the program (with the shim in LD_PRELOAD when `preload`); returns ({call: maxrel}, stderr)."""
    import subprocess
    env = dict(os.environ)
    env.pop("LD_PRELOAD", None)
    if preload:
        env["LD_PRELOAD"] = SHIM
        env["GEN9BLAS_BLAS_INFO"] = "1"
    env.update(extra_env or {})
    r = subprocess.run([prog], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    errs = {}
    for line in r.stdout.splitlines():
        name, val = line.split(" maxrel=")
        errs[name] = float(val)
    return errs, r.stderr
