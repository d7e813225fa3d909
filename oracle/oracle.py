"""Oracle for the gen9blas hot path: the checker, never the thing measured or shipped.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg. The product
(libgen9blas.so, gen9blas.py, libgen9blas_blas.so) never imports or calls it.

Two parts:
- `liboracle.so` (oracle.c): the element-by-element restatement of the reference kernels' arithmetic (FP16 fma chains
  of the H and HS modes, FP32/FP64 fma chains, FP32-accumulated skinny products, FP64 reductions, GEMV). Each C
  function cites the reference file:line it follows.
- `cpu_path`: the reference's own CPU path. The reference's BLAS layer forwards to OpenBLAS (reference:
  lib/src/cblas.c:43-56, OpenBLAS 0.3.26 per README.md:48); here OpenBLAS is SciPy's bundled 0.3.29, reached through
  NumPy / scipy.linalg.blas. For FP16 the CPU path is NumPy FP32 math on the same FP16 inputs.

Also here: the reference's error metric e = |C − ref| / (|alpha|·Σ|a·b| + |beta·c|) (reference: lib/test_basic.py:53-56)
and the seeded input generators of the benchmark configurations.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.realpath(__file__))
_LIB_PATH = os.path.join(HERE, "liboracle.so")


def build():
    """Compiles liboracle.so (make -C oracle)."""
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    return _LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        i, d, f, p, l = ctypes.c_int, ctypes.c_double, ctypes.c_float, ctypes.c_void_p, ctypes.c_long
        L.orc_f16_round.restype = ctypes.c_uint16
        L.orc_f16_round.argtypes = [d]
        L.orc_f16_value.restype = d
        L.orc_f16_value.argtypes = [ctypes.c_uint16]
        L.orc_f16_round_array.argtypes = [p, p, l]
        L.orc_f16_value_array.argtypes = [p, p, l]
        for n in ("orc_gemm_h", "orc_gemm_hs"):
            getattr(L, n).argtypes = [i, i, i, i, i, f, p, i, p, i, f, p, i]
        L.orc_gemm_s.argtypes = [i, i, i, i, i, f, p, i, p, i, f, p, i]
        L.orc_gemm_d.argtypes = [i, i, i, i, i, d, p, i, p, i, d, p, i]
        L.orc_skinny.argtypes = [i, i, i, i, i, i, f, p, i, p, i, f, p, i]
        L.orc_axpy.argtypes = [i, i, d, p, i, p, i]
        L.orc_reduce.restype = d
        L.orc_reduce.argtypes = [i, i, i, p, i, p, i]
        L.orc_gemv.argtypes = [i, i, i, i, d, p, i, p, i, d, p, i]
        _lib = L
    return _lib


# ---------------- binary16 ----------------
def f16_round(x):
    """float64 array -> binary16 bit patterns (uint16), round to nearest even (oracle.c:orc_f16_round)."""
    x = np.ascontiguousarray(x, dtype=np.float64)
    h = np.empty(x.shape, np.uint16)
    lib().orc_f16_round_array(x.ctypes.data, h.ctypes.data, x.size)
    return h


def f16_value(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    x = np.empty(h.shape, np.float64)
    lib().orc_f16_value_array(h.ctypes.data, x.ctypes.data, h.size)
    return x


# ---------------- restatement of the reference kernels ----------------
def _stored(X, dt):
    """(contiguous array, ld) of a 2-D operand as stored."""
    X = np.ascontiguousarray(X, dtype=dt)
    return X, X.shape[1]


def gemm(kind, A, B, alpha=1.0, beta=0.0, C=None, tA=False, tB=False):
    """C = alpha·op(A)·op(B) + beta·C with the reference's accumulation for kind in {"H", "HS", "S", "D"}.
    A, B are the stored matrices (op = transpose when tA / tB). FP16 arrays may be float16 or uint16 bits."""
    dt = {"H": np.float16, "HS": np.float16, "S": np.float32, "D": np.float64}[kind]
    a, lda = _stored(A, dt)
    b, ldb = _stored(B, dt)
    M, K = (a.shape[1], a.shape[0]) if tA else a.shape
    N = b.shape[0] if tB else b.shape[1]
    c = np.zeros((M, N), dt) if C is None else np.array(C, dtype=dt, copy=True, order="C")
    fn = {"H": lib().orc_gemm_h, "HS": lib().orc_gemm_hs, "S": lib().orc_gemm_s, "D": lib().orc_gemm_d}[kind]
    fn(M, N, K, int(tA), int(tB), alpha, a.ctypes.data, lda, b.ctypes.data, ldb, beta if C is not None else 0.0,
       c.ctypes.data, N)
    return c


def skinny(A, B, alpha=1.0, beta=0.0, C=None, tA=False, tB=False):
    """Skinny product with FP32 accumulation (reference skinny kernels); A, B float16 or float32 as stored."""
    dt = np.float16 if A.dtype == np.float16 else np.float32
    a, lda = _stored(A, dt)
    b, ldb = _stored(B, dt)
    M, K = (a.shape[1], a.shape[0]) if tA else a.shape
    N = b.shape[0] if tB else b.shape[1]
    c = np.zeros((M, N), dt) if C is None else np.array(C, dtype=dt, copy=True, order="C")
    lib().orc_skinny(np.dtype(dt).itemsize, M, N, K, int(tA), int(tB), alpha, a.ctypes.data, lda, b.ctypes.data, ldb,
                     beta if C is not None else 0.0, c.ctypes.data, N)
    return c


def _vec_ptr(x):
    """(base array, pointer to the lowest address, inc) of a 1-D view (negative strides allowed)."""
    inc = x.strides[0] // x.itemsize
    return x.ctypes.data + (min(inc, 0) * (x.shape[0] - 1) * x.itemsize if x.shape[0] else 0), inc


def axpy(a, x, y):
    """In place on y (a 1-D view of float16/float32/float64), as the reference kernel."""
    px, ix = _vec_ptr(x)
    py, iy = _vec_ptr(y)
    lib().orc_axpy(y.itemsize, y.shape[0], a, px, ix, py, iy)
    return y


def reduce(mode, x, y=None):
    px, ix = _vec_ptr(x)
    py, iy = _vec_ptr(y) if y is not None else (None, 0)
    return lib().orc_reduce(x.itemsize, mode, x.shape[0], px, ix, py, iy)


def dot(x, y):
    return reduce(0, x, y)


def gemv(A, x, alpha=1.0, beta=0.0, y=None, trans=False):
    A = np.ascontiguousarray(A)
    M, N = A.shape
    ny = N if trans else M
    out = np.zeros(ny, A.dtype) if y is None else y
    px, ix = _vec_ptr(x)
    py, iy = _vec_ptr(out)
    lib().orc_gemv(A.itemsize, int(trans), M, N, alpha, A.ctypes.data, N, px, ix, beta if y is not None else 0.0, py, iy)
    return out


# ---------------- level 2: symmetric, triangular, band and packed storage (float64 closed forms) ----------------
# The arithmetic of these routines is a plain sum of products (FP32 / FP64 accumulation, reference:
# lib/kernels/level12.cl:424-640), so the oracle is the float64 product of the matrix the storage describes; what a
# kernel can get wrong is the storage mapping, restated here element by element.
def band_dense(P, M, N, KL, KU):
    """M×N float64 matrix of a row-major band array P (rows of lda >= KL+KU+1): A(r, c) = P[r, KL + c − r] for
    −KL <= c − r <= KU, zero elsewhere (reference: lib/kernels/level12.cl:584-590, lib/gen9blas.h:147-150)."""
    P = np.asarray(P, np.float64)
    D = np.zeros((M, N))
    for r in range(M):
        for c in range(max(0, r - KL), min(N, r + KU + 1)):
            D[r, c] = P[r, KL + c - r]
    return D


def packed_dense(Ap, n, uplo):
    """n×n float64 triangle of a packed vector: upper row r (c = r..n−1) starts at r·n − r(r−1)/2, lower row r
    (c = 0..r) at r(r+1)/2 (reference: lib/kernels/level12.cl:588-590, lib/gen9blas.h:150-151)."""
    Ap = np.asarray(Ap, np.float64)
    D = np.zeros((n, n))
    for r in range(n):
        if uplo == "U":
            s0 = r * n - r * (r - 1) // 2
            D[r, r:] = Ap[s0:s0 + n - r]
        else:
            s0 = r * (r + 1) // 2
            D[r, :r + 1] = Ap[s0:s0 + r + 1]
    return D


def triangle(D, uplo, unit=False):
    """The `uplo` triangle of D (float64); unit: ones on the diagonal instead of the stored values."""
    T = np.tril(D) if uplo == "L" else np.triu(D)
    if unit:
        np.fill_diagonal(T, 1.0)
    return T


def symmetric(D, uplo):
    """The symmetric matrix whose `uplo` triangle is that of D."""
    T = triangle(D, uplo)
    return T + T.T - np.diag(np.diag(T))


def mv(Op, x, alpha=1.0, beta=0.0, y=None):
    """(alpha·Op·x + beta·y, its scale |alpha|·|Op|·|x| + |beta·y|) in float64: the product and the error scale of
    the reference's level-2 test (reference: lib/test_level12.py:27-35, 105-113)."""
    X = np.asarray(x, np.float64)
    r, s = alpha * (Op @ X), abs(alpha) * (np.abs(Op) @ np.abs(X))
    if beta:
        Y = np.asarray(y, np.float64)
        r, s = r + beta * Y, s + abs(beta) * np.abs(Y)
    return r, s


def solve(Op, b):
    """op(A)·z = b for a triangular float64 op(A), by substitution in the order of the reference's blocked solve
    (reference: lib/kernels/level12.cl:493-548: forward for a lower op(A), backward for an upper one)."""
    n = Op.shape[0]
    z = np.array(b, np.float64)
    lower = np.allclose(Op, np.tril(Op))
    for k in (range(n) if lower else range(n - 1, -1, -1)):
        z[k] /= Op[k, k]
        rest = slice(k + 1, n) if lower else slice(0, k)
        z[rest] -= Op[rest, k] * z[k]
    return z


# ---------------- the reference's error metric ----------------
def gemm_error(W, opA, opB, alpha=1.0, beta=0.0, C0=None):
    """Element-wise e = |W − ref| / (|alpha|·Σ|a·b| + |beta·c|) against the float64 product of the same (rounded)
    inputs (reference: lib/test_basic.py:4-8, 53-56). opA, opB are op(A), op(B); returns (mean, max)."""
    a64, b64 = np.asarray(opA, np.float64), np.asarray(opB, np.float64)
    ref = alpha * (a64 @ b64)
    scale = abs(alpha) * (np.abs(a64) @ np.abs(b64))
    if beta:
        c64 = np.asarray(C0, np.float64)
        ref = ref + beta * c64
        scale = scale + abs(beta) * np.abs(c64)
    e = np.abs(np.asarray(W, np.float64) - ref) / np.maximum(scale, 1e-300)
    return float(e.mean()), float(e.max())


# ---------------- seeded inputs of the benchmark configurations ----------------
SEED_A, SEED_B, SEED_C, SEED_X, SEED_Y, SEED_W0 = 1, 2, 3, 20, 21, 100


def uniform(shape, dtype, seed):
    return np.random.default_rng(seed).uniform(-1, 1, shape).astype(dtype)


def normal(shape, dtype, seed, scale=1.0):
    g = np.random.default_rng(seed)
    return (g.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(dtype)


# ---------------- the reference's CPU path (OpenBLAS via NumPy / SciPy) ----------------
class cpu_path:
    """What the reference's BLAS layer runs on the CPU: OpenBLAS for FP32/FP64 (cblas_sgemm / sgemv / saxpy / sdot,
    reference: lib/src/cblas.c:186-313), NumPy FP32 math on FP16 inputs for HGEMM and skinny."""

    @staticmethod
    def sgemm(A, B):
        return A @ B                                   # float32 @ float32: OpenBLAS sgemm

    @staticmethod
    def dgemm(A, B):
        return A @ B

    @staticmethod
    def hgemm(A, B):
        return (A.astype(np.float32) @ B.astype(np.float32)).astype(np.float16)

    @staticmethod
    def skinny(A, W):
        return (A.astype(np.float32) @ W.astype(np.float32).T).astype(np.float16)

    @staticmethod
    def saxpy(a, x, y):
        from scipy.linalg import blas
        return blas.saxpy(x, y, a=a)                   # in place on y (float32, contiguous)

    @staticmethod
    def sdot(x, y):
        from scipy.linalg import blas
        return blas.sdot(x, y)

    @staticmethod
    def sgemv(A, x, trans=False):
        return A.T @ x if trans else A @ x             # float32 matrix-vector: OpenBLAS sgemv


def openblas_info():
    """(version string, threads) of the OpenBLAS that NumPy uses, via threadpoolctl when available."""
    try:
        from threadpoolctl import threadpool_info
        for i in threadpool_info():
            if i.get("internal_api") == "openblas":
                return i.get("version"), i.get("num_threads")
    except Exception:
        pass
    return None, None


def gemm_diff(W, R, opA, opB, alpha=1.0, beta=0.0, C0=None):
    """max |W − R| / (|alpha|·Σ|a·b| + |beta·c|): distance between two results in the units of the reference metric."""
    a64, b64 = np.asarray(opA, np.float64), np.asarray(opB, np.float64)
    scale = abs(alpha) * (np.abs(a64) @ np.abs(b64))
    if beta:
        scale = scale + abs(beta) * np.abs(np.asarray(C0, np.float64))
    return float((np.abs(np.asarray(W, np.float64) - np.asarray(R, np.float64)) / np.maximum(scale, 1e-300)).max())
