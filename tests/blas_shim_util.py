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
