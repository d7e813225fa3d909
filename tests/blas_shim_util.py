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
