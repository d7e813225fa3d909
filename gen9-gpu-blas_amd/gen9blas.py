"""gen9blas for MI355X: ctypes + NumPy module over libgen9blas.so (the drop-in for the reference's gen9blas.py).

    import numpy as np, gen9blas
    C = gen9blas.hgemm(A, B)                  # float16 in, float16 out; accurate=True: GEN9BLAS_HS
    C = gen9blas.sgemm(A.T, B, alpha=2.0)     # transposed views pass as transpose flags, no copy
    C = gen9blas.gemm_batched(A3, B3)         # (count, M, K) · (count, K, N)
    y = gen9blas.gemv(A, x); d = gen9blas.dot(x, y); gen9blas.axpy(0.5, x, y)

Same functions, arguments and errors as the reference module (reference: lib/gen9blas.py:96-410): the element type
follows the data, views with a row stride or a transpose are passed without copying, a non-zero status raises
RuntimeError(gen9blas_error()), the library must report version 0.2.x.

MI355X additions: operands may also be torch tensors on the GPU (or any object with __cuda_array_interface__ when
the output is supplied); the kernels then use them in place and results stay on the device. NumPy arrays are host
memory: the library copies them to the GPU and back. gen9blas.empty returns pinned host memory from gen9blas_alloc
(faster DMA than pageable memory).
"""
import ctypes
import os
import weakref

import numpy as np

_HERE = os.path.dirname(os.path.realpath(__file__))


def _find(name):
    p = os.path.join(_HERE, name)
    return p if os.path.exists(p) else name


_lib = ctypes.CDLL(os.environ.get("GEN9BLAS_LIB") or _find("libgen9blas.so"))
_i, _f, _p, _l, _d = ctypes.c_int, ctypes.c_float, ctypes.c_void_p, ctypes.c_long, ctypes.c_double
_lib.gen9blas_init.argtypes = []
_lib.gen9blas_gemm.argtypes = [_i, _i, _i, _i, _i, _i, _d, _p, _i, _p, _i, _d, _p, _i]
_lib.gen9blas_gemm_batched.argtypes = [_i, _i, _i, _i, _i, _i, _d, _p, _i, _l, _p, _i, _l, _d, _p, _i, _l, _i]
_lib.gen9blas_symm.argtypes = [_i, _i, _i, _i, _i, _d, _p, _i, _p, _i, _d, _p, _i]
_lib.gen9blas_syrk.argtypes = [_i, _i, _i, _i, _i, _d, _p, _i, _d, _p, _i]
_lib.gen9blas_syr2k.argtypes = [_i, _i, _i, _i, _i, _d, _p, _i, _p, _i, _d, _p, _i]
_lib.gen9blas_trmm.argtypes = [_i, _i, _i, _i, _i, _i, _i, _d, _p, _i, _p, _i]
_lib.gen9blas_trsm.argtypes = [_i, _i, _i, _i, _i, _i, _i, _d, _p, _i, _p, _i]
_lib.gen9blas_last_time_ms.restype = ctypes.c_double
_lib.gen9blas_alloc.argtypes = [ctypes.c_size_t]
_lib.gen9blas_alloc.restype = ctypes.c_void_p
_lib.gen9blas_free.argtypes = [ctypes.c_void_p]
_lib.gen9blas_error.restype = ctypes.c_char_p
_lib.gen9blas_hip_stream.restype = ctypes.c_void_p
_lib.gen9blas_set_nowait.argtypes = [_i]
_lib.gen9blas_pack_b.argtypes = [_i, _i, _i, _i, _p, _i]
_lib.gen9blas_pack_b.restype = _p
_lib.gen9blas_gemm_pb.argtypes = [_i, _i, _d, _p, _i, _p, _d, _p, _i]
_lib.gen9blas_packed_b_free.argtypes = [_p]
_lib.gen9blas_gemm_pb_skinny.argtypes = [_i, _p, _i, _p, _p, _i, ctypes.POINTER(_i)]   # gen9blas_ml.h
GEN9BLAS_H, GEN9BLAS_S, GEN9BLAS_HS, GEN9BLAS_D = 0, 1, 2, 3
FEAT_FP16, FEAT_FP32, FEAT_FP64 = 0, 1, 2
_lib.gen9blas_version.restype = ctypes.c_int
if _lib.gen9blas_version() // 100 != 2:
    raise ImportError(f"gen9blas.py expects libgen9blas 0.2.x, loaded {_lib.gen9blas_version()}")
_SIDE = {"L": 0, "R": 1}
_TRI = {"L": 0, "U": 1}
_ready = False


def _init():
    global _ready
    if not _ready:
        if _lib.gen9blas_init() != 0:
            raise RuntimeError(_lib.gen9blas_error().decode())
        _ready = True


def _check(w):
    if w != 0:
        raise RuntimeError(_lib.gen9blas_error().decode())


def hip_stream():
    """The library's HIP stream (hipStream_t as an int), e.g. for torch.cuda.ExternalStream."""
    _init()
    return _lib.gen9blas_hip_stream()


def set_nowait(on):
    """No-wait mode: calls on device operands return without waiting; flush() waits."""
    _lib.gen9blas_set_nowait(int(bool(on)))


def flush():
    _check(_lib.gen9blas_flush())


# ---------------- pinned host memory pool (gen9blas.empty) ----------------
_pool = {}
_pool_bytes = 0
POOL_MAX = 1 << 30


def _block_size(n):
    return max(4096, (n + 65535) // 65536 * 65536 if n > 65536 else (n + 4095) // 4096 * 4096)


def _release(p, n):
    global _pool_bytes
    if _pool_bytes + n <= POOL_MAX:
        _pool.setdefault(n, []).append(p)
        _pool_bytes += n
    else:
        _lib.gen9blas_free(p)


def free_pool():
    """Returns the pooled blocks to the runtime (arrays still in use stay)."""
    global _pool_bytes
    for blocks in _pool.values():
        for p in blocks:
            _lib.gen9blas_free(p)
    _pool.clear()
    _pool_bytes = 0


def empty(shape, dtype=np.float16):
    """C-contiguous array in pinned host memory (gen9blas_alloc). When every view is gone the block returns to a pool
    (up to POOL_MAX bytes) for later empty() calls of the same rounded size."""
    global _pool_bytes
    _init()
    dtype = np.dtype(dtype)
    n = int(np.prod(shape)) * dtype.itemsize
    nb = _block_size(n)
    if _pool.get(nb):
        p = _pool[nb].pop()
        _pool_bytes -= nb
    else:
        p = _lib.gen9blas_alloc(nb)
        if not p:
            raise MemoryError(_lib.gen9blas_error().decode())
    raw = (ctypes.c_char * nb).from_address(p)
    f = weakref.finalize(raw, _release, p, nb)
    f.atexit = False
    return np.frombuffer(raw, dtype=np.uint8, count=n).view(dtype).reshape(shape)


def available(dt, accurate=False):
    _init()
    k = _kind(dt, accurate)
    return bool(_lib.gen9blas_has(FEAT_FP32 if k == GEN9BLAS_S else FEAT_FP64 if k == GEN9BLAS_D else FEAT_FP16))


def _kind(dt, accurate):
    dt = _np_dtype(dt)
    if dt == np.float32:
        return GEN9BLAS_S
    if dt == np.float64:
        return GEN9BLAS_D
    if dt == np.float16:
        return GEN9BLAS_HS if accurate else GEN9BLAS_H
    raise TypeError("supported types: float16, float32, float64")


# ---------------- device tensors (torch) ----------------
def _is_dev(X):
    return getattr(X, "is_cuda", False) and hasattr(X, "data_ptr")


def _np_dtype(dt):
    if isinstance(dt, np.dtype) or isinstance(dt, type):
        return np.dtype(dt)
    s = str(dt)   # torch.float16 -> "torch.float16"
    if s.startswith("torch."):
        return np.dtype(s[6:])
    return np.dtype(dt)


def _torch_dtype(dt):
    import torch
    return {np.dtype(np.float16): torch.float16, np.dtype(np.float32): torch.float32,
            np.dtype(np.float64): torch.float64}[np.dtype(dt)]


def _dtype_of_arr(X):
    return _np_dtype(X.dtype)


def _dev_mat(A, dt, write=False):
    """(tensor, pointer, rows, cols, ld, trans) of a 2-D device tensor; strided rows and transposes in place."""
    if A.dim() != 2:
        raise ValueError("expected a 2-D matrix")
    if _np_dtype(A.dtype) != np.dtype(dt):
        if write:
            raise TypeError(f"the result must be a {np.dtype(dt).name} matrix")
        A = A.to(_torch_dtype(dt))
    s0, s1 = A.stride()
    r, c = A.shape
    if s1 == 1 and s0 >= c:
        return A, A.data_ptr(), r, c, s0, 0
    if not write and s0 == 1 and s1 >= r:
        return A, A.data_ptr(), c, r, s1, 1
    if write:
        raise TypeError(f"the result must be a {np.dtype(dt).name} matrix with contiguous rows")
    A = A.contiguous()
    return A, A.data_ptr(), r, c, c, 0


def _dev_vec(x, dt, write=False):
    if x.dim() != 1:
        raise ValueError("expected a 1-D vector")
    if _np_dtype(x.dtype) != np.dtype(dt) or x.stride()[0] == 0:
        if write:
            raise TypeError(f"the result must be a {np.dtype(dt).name} vector with a non-zero stride")
        x = x.to(_torch_dtype(dt)).contiguous()
    n, inc = x.shape[0], x.stride()[0]
    return x, x.data_ptr(), n, inc


# ---------------- level 3 ----------------
def _m3(X, dt, write=False):
    X, p, _, _, ld, tr = _mat(X, dt, write)
    return X, p, ld, tr


def _c(X, dt):
    if _is_dev(X):
        return X.to(_torch_dtype(dt)).contiguous()
    return np.ascontiguousarray(X, dtype=dt)


def _output(C, shape, dt, like):
    """(C, given, ldc): a new C (device tensor for device inputs, else pinned host memory) or the supplied C."""
    if C is None:
        if _is_dev(like):
            import torch
            return torch.empty(tuple(shape), dtype=_torch_dtype(dt), device=like.device), False, shape[-1]
        return empty(shape, dt), False, shape[-1]
    if _is_dev(C):
        if tuple(C.shape) != tuple(shape) or _np_dtype(C.dtype) != np.dtype(dt) or C.stride()[-1] != 1:
            raise ValueError(f"C must have shape {tuple(shape)}, type {np.dtype(dt).name} and contiguous rows")
        if C.dim() == 2:
            return C, True, _dev_mat(C, dt, True)[4]
        if not C.is_contiguous():
            raise ValueError("C (batch) must be C-contiguous")
        return C, True, shape[-1]
    if C.shape != tuple(shape) or C.dtype != dt or C.strides[-1] != C.itemsize:
        raise ValueError(f"C must have shape {tuple(shape)}, type {np.dtype(dt).name} and contiguous rows")
    if C.ndim == 2:
        return C, True, _mat(C, dt, True)[4]
    if not C.flags.c_contiguous:
        raise ValueError("C (batch) must be C-contiguous")
    return C, True, shape[-1]


def _ptr(X):
    return X.data_ptr() if _is_dev(X) else X.ctypes.data


def gemm(A, B, alpha=1.0, beta=0.0, C=None, accurate=False):
    """C = alpha·A·B + beta·C (float16, float32 or float64 according to A)."""
    _init()
    dt = _dtype_of_arr(A)
    if dt not in (np.float16, np.float32, np.float64):
        dt = np.dtype(np.float32)
    (M, K), (K2, N) = tuple(A.shape), tuple(B.shape)
    if K != K2:
        raise ValueError(f"incompatible dimensions: {tuple(A.shape)} · {tuple(B.shape)}")
    a, pa, lda, ta = _m3(A, dt)
    b, pb, ldb, tb = _m3(B, dt)
    C, given, ldc = _output(C, (M, N), dt, A)
    _check(_lib.gen9blas_gemm(_kind(dt, accurate), ta, tb, M, N, K, alpha, pa, lda, pb, ldb, beta if given else 0.0,
                              _ptr(C), ldc))
    return C


def _astype(X, dt):
    if _is_dev(X):
        return X if _np_dtype(X.dtype) == np.dtype(dt) else X.to(_torch_dtype(dt))
    return X if X.dtype == dt else X.astype(dt)


def hgemm(A, B, alpha=1.0, beta=0.0, C=None, accurate=False):
    return gemm(_astype(A, np.float16), _astype(B, np.float16), alpha, beta, C, accurate)


def sgemm(A, B, alpha=1.0, beta=0.0, C=None):
    return gemm(_astype(A, np.float32), _astype(B, np.float32), alpha, beta, C)


def gemm_batched(A, B, alpha=1.0, beta=0.0, C=None, accurate=False):
    """Batch of products: A (count, M, K), B (count, K, N) -> C (count, M, N), one launch."""
    _init()
    dt = _dtype_of_arr(A)
    if dt not in (np.float16, np.float32, np.float64):
        dt = np.dtype(np.float32)
    a, b = _c(A, dt), _c(B, dt)
    (cnt, M, K), (cnt2, K2, N) = tuple(a.shape), tuple(b.shape)
    if K != K2 or cnt != cnt2:
        raise ValueError(f"incompatible dimensions: {tuple(a.shape)} · {tuple(b.shape)}")
    C, given, _ = _output(C, (cnt, M, N), dt, A)
    _check(_lib.gen9blas_gemm_batched(_kind(dt, accurate), 0, 0, M, N, K, alpha, _ptr(a), K, M * K, _ptr(b), N, K * N,
                                      beta if given else 0.0, _ptr(C), N, M * N, cnt))
    return C


def _square(A, dt, uplo):
    A, p, r, c, ld, tr = _mat(A, dt)
    if r != c:
        raise ValueError("expected a square matrix")
    return A, p, r, ld, tr, ({"L": "U", "U": "L"}[uplo] if tr else uplo)


def _copy_of(B, dt):
    b = empty(tuple(B.shape), dt)
    b[...] = B
    return b


def symm(A, B, side="L", uplo="L", alpha=1.0, beta=0.0, C=None, accurate=False):
    _init()
    dt = _dtype_of_arr(B)
    a, pa, n, lda, _, uplo = _square(A, dt, uplo)
    b, pb, ldb, tb = _m3(B, dt)
    if tb:
        b, pb, ldb, tb = _m3(_c(B, dt), dt)
    M, N = B.shape
    C, given, ldc = _output(C, (M, N), dt, B)
    _check(_lib.gen9blas_symm(_kind(dt, accurate), _SIDE[side], _TRI[uplo], M, N, alpha, pa, lda, pb, ldb,
                              beta if given else 0.0, _ptr(C), ldc))
    return C


def syrk(A, uplo="L", trans=False, alpha=1.0, beta=0.0, C=None, accurate=False):
    _init()
    dt = _dtype_of_arr(A)
    N, K = (A.shape[1], A.shape[0]) if trans else A.shape
    a, pa, lda, ta = _m3(A, dt)
    C, given, ldc = _output(C, (N, N), dt, A)
    if not given:
        C[...] = 0
    _check(_lib.gen9blas_syrk(_kind(dt, accurate), _TRI[uplo], int(trans) ^ ta, N, K, alpha, pa, lda,
                              beta if given else 0.0, _ptr(C), ldc))
    return C


def syr2k(A, B, uplo="L", trans=False, alpha=1.0, beta=0.0, C=None, accurate=False):
    _init()
    dt = _dtype_of_arr(A)
    N, K = (A.shape[1], A.shape[0]) if trans else A.shape
    a, pa, lda, ta = _m3(A, dt)
    b, pb, ldb, tb = _m3(B, dt)
    if ta != tb:
        b, pb, ldb, tb = _m3(np.ascontiguousarray(B.T, dtype=dt).T if ta else _c(B, dt), dt)
    C, given, ldc = _output(C, (N, N), dt, A)
    if not given:
        C[...] = 0
    _check(_lib.gen9blas_syr2k(_kind(dt, accurate), _TRI[uplo], int(trans) ^ ta, N, K, alpha, pa, lda, pb, ldb,
                               beta if given else 0.0, _ptr(C), ldc))
    return C


def trmm(A, B, side="L", uplo="L", transA=False, diag=False, alpha=1.0, accurate=False):
    _init()
    dt = _dtype_of_arr(B)
    a, pa, _, lda, ta, uplo = _square(A, dt, uplo)
    b = _copy_of(B, dt)
    M, N = b.shape
    _check(_lib.gen9blas_trmm(_kind(dt, accurate), _SIDE[side], _TRI[uplo], int(transA) ^ ta, int(diag), M, N, alpha, pa,
                              lda, b.ctypes.data, N))
    return b


def trsm(A, B, side="L", uplo="L", transA=False, diag=False, alpha=1.0, accurate=False):
    _init()
    dt = _dtype_of_arr(B)
    if dt not in (np.float16, np.float32, np.float64):
        dt = np.dtype(np.float32)
    a, pa, _, lda, ta, uplo = _square(A, dt, uplo)
    b = _copy_of(B, dt)
    M, N = b.shape
    _check(_lib.gen9blas_trsm(_kind(dt, accurate), _SIDE[side], _TRI[uplo], int(transA) ^ ta, int(diag), M, N, alpha, pa,
                              lda, b.ctypes.data, N))
    return b


def last_time_ms():
    return _lib.gen9blas_last_time_ms()


def last_zero_copy():
    return _lib.gen9blas_last_zero_copy()


# ---------------- levels 1-2 (FP16 computed in FP32, reductions in FP64) ----------------
_lib.gen9blas_axpy.argtypes = [_i, _i, _d, _p, _i, _p, _i]
_lib.gen9blas_scal.argtypes = [_i, _i, _d, _p, _i]
_lib.gen9blas_copy.argtypes = [_i, _i, _p, _i, _p, _i]
_lib.gen9blas_swap.argtypes = [_i, _i, _p, _i, _p, _i]
_lib.gen9blas_rot.argtypes = [_i, _i, _p, _i, _p, _i, _d, _d]
_lib.gen9blas_dot.argtypes = [_i, _i, _p, _i, _p, _i, ctypes.POINTER(_d)]
_lib.gen9blas_asum.argtypes = [_i, _i, _p, _i, ctypes.POINTER(_d)]
_lib.gen9blas_nrm2.argtypes = [_i, _i, _p, _i, ctypes.POINTER(_d)]
_lib.gen9blas_iamax.argtypes = [_i, _i, _p, _i, ctypes.POINTER(_l)]
_lib.gen9blas_gemv.argtypes = [_i, _i, _i, _i, _d, _p, _i, _p, _i, _d, _p, _i]
_lib.gen9blas_ger.argtypes = [_i, _i, _i, _d, _p, _i, _p, _i, _p, _i]


def _dtype_of(*X):
    dt = _dtype_of_arr(X[0])
    return np.dtype(np.float16) if dt == np.float16 else np.dtype(np.float64) if dt == np.float64 else np.dtype(np.float32)


def _vec(x, dt, write=False):
    """(array, pointer to the lowest address, n, inc) of a 1-D vector; inc < 0 as in BLAS."""
    if _is_dev(x):
        x, p, n, inc = _dev_vec(x, dt, write)
        return x, p + (min(inc, 0) * (n - 1) * x.element_size() if n else 0), n, inc
    if x.ndim != 1:
        raise ValueError("expected a 1-D vector")
    if x.dtype != dt or x.strides[0] % x.itemsize or x.strides[0] == 0:
        if write:
            raise TypeError(f"the result must be a {np.dtype(dt).name} vector with a stride that is a multiple of the "
                            "element size")
        x = np.ascontiguousarray(x, dtype=dt)
    n, inc = x.shape[0], x.strides[0] // x.itemsize
    return x, x.ctypes.data + (min(inc, 0) * (n - 1) * x.itemsize if n else 0), n, inc


def _mat(A, dt, write=False):
    """(array, pointer, rows, columns, ld, trans) for a row-major matrix with ld; a transposed view passes as trans."""
    if _is_dev(A):
        return _dev_mat(A, dt, write)
    if A.ndim != 2:
        raise ValueError("expected a 2-D matrix")
    e = A.itemsize
    if A.dtype == dt and A.strides[1] == e and A.strides[0] >= A.shape[1] * e and A.strides[0] % e == 0:
        return A, A.ctypes.data, A.shape[0], A.shape[1], A.strides[0] // e, 0
    if not write and A.dtype == dt and A.strides[0] == e and A.strides[1] >= A.shape[0] * e and A.strides[1] % e == 0:
        return A, A.ctypes.data, A.shape[1], A.shape[0], A.strides[1] // e, 1
    if write:
        raise TypeError(f"the result must be a {np.dtype(dt).name} matrix with contiguous rows")
    A = np.ascontiguousarray(A, dtype=dt)
    return A, A.ctypes.data, A.shape[0], A.shape[1], A.shape[1], 0


def _kind_basic(dt):
    return GEN9BLAS_S if dt == np.float32 else GEN9BLAS_D if dt == np.float64 else GEN9BLAS_H


def _new_vec(n, dt, like):
    if _is_dev(like):
        import torch
        return torch.empty((n,), dtype=_torch_dtype(dt), device=like.device)
    return empty((n,), dt)


def axpy(a, x, y):
    """y = a·x + y (in place); returns y."""
    _init(); t = _dtype_of(y); y, py, n, iy = _vec(y, t, True); x, px, nx, ix = _vec(x, t)
    if nx != n:
        raise ValueError("lengths differ")
    _check(_lib.gen9blas_axpy(_kind_basic(t), n, a, px, ix, py, iy)); return y


def scal(a, x):
    """x = a·x (in place); returns x."""
    _init(); t = _dtype_of(x); x, px, n, ix = _vec(x, t, True)
    _check(_lib.gen9blas_scal(_kind_basic(t), n, a, px, ix)); return x


def copy(x, y=None):
    """y = x; without y: a new array of the type of x."""
    _init(); t = _dtype_of(y if y is not None else x)
    if y is None:
        y = _new_vec(x.shape[0], t, x)
    y, py, n, iy = _vec(y, t, True); x, px, nx, ix = _vec(x, t)
    if nx != n:
        raise ValueError("lengths differ")
    _check(_lib.gen9blas_copy(_kind_basic(t), n, px, ix, py, iy)); return y


def swap(x, y):
    _init(); t = _dtype_of(x); x, px, n, ix = _vec(x, t, True); y, py, ny, iy = _vec(y, t, True)
    if ny != n:
        raise ValueError("lengths differ")
    _check(_lib.gen9blas_swap(_kind_basic(t), n, px, ix, py, iy)); return x, y


def rot(x, y, c, s):
    """x, y = c·x + s·y, c·y − s·x (in place)."""
    _init(); t = _dtype_of(x); x, px, n, ix = _vec(x, t, True); y, py, ny, iy = _vec(y, t, True)
    if ny != n:
        raise ValueError("lengths differ")
    _check(_lib.gen9blas_rot(_kind_basic(t), n, px, ix, py, iy, c, s)); return x, y


def dot(x, y):
    _init(); t = _dtype_of(x); x, px, n, ix = _vec(x, t); y, py, ny, iy = _vec(y, t)
    if ny != n:
        raise ValueError("lengths differ")
    w = _d(); _check(_lib.gen9blas_dot(_kind_basic(t), n, px, ix, py, iy, ctypes.byref(w))); return w.value


def asum(x):
    _init(); t = _dtype_of(x); x, px, n, ix = _vec(x, t)
    w = _d(); _check(_lib.gen9blas_asum(_kind_basic(t), n, px, ix, ctypes.byref(w))); return w.value


def nrm2(x):
    _init(); t = _dtype_of(x); x, px, n, ix = _vec(x, t)
    w = _d(); _check(_lib.gen9blas_nrm2(_kind_basic(t), n, px, ix, ctypes.byref(w))); return w.value


def iamax(x):
    """Index (0-based) of the first largest |x|; -1 for an empty vector."""
    _init(); t = _dtype_of(x); x, px, n, ix = _vec(x, t)
    w = _l(); _check(_lib.gen9blas_iamax(_kind_basic(t), n, px, ix, ctypes.byref(w))); return w.value


def gemv(A, x, alpha=1.0, beta=0.0, y=None, trans=False):
    """y = alpha·op(A)·x + beta·y; without y: a new array. An A.T view is passed as trans."""
    _init(); t = _dtype_of(A); A, pa, M, N, lda, tr = _mat(A, t); tr ^= int(trans)
    x, px, nx, ix = _vec(x, t)
    ny = N if tr else M
    if nx != (M if tr else N):
        raise ValueError("length of x does not match A")
    if y is None:
        y, beta = _new_vec(ny, t, A), 0.0
    y, py, n, iy = _vec(y, t, True)
    if n != ny:
        raise ValueError("length of y does not match A")
    _check(_lib.gen9blas_gemv(_kind_basic(t), tr, M, N, alpha, pa, lda, px, ix, beta, py, iy)); return y


def ger(alpha, x, y, A):
    """A = alpha·x·yᵀ + A (in place); returns A."""
    _init(); t = _dtype_of(A); A, pa, M, N, lda, _ = _mat(A, t, True)
    x, px, nx, ix = _vec(x, t); y, py, ny, iy = _vec(y, t)
    if nx != M or ny != N:
        raise ValueError("lengths of x, y do not match A")
    _check(_lib.gen9blas_ger(_kind_basic(t), M, N, alpha, px, ix, py, iy, pa, lda)); return A


# ---------------- level 2 on symmetric, triangular, banded and packed matrices ----------------
# Full storage: a square matrix of which the `uplo` triangle is used (an A.T view passes as the other triangle, no
# copy). Band: a row-major array (rows, KL+KU+1) with A[i, j] in row i, column KL + j − i (symmetric / triangular:
# lower KL = K, KU = 0; upper KL = 0, KU = K). Packed: a contiguous vector of n(n+1)/2 elements holding the rows of
# the triangle (upper: j = i..n−1, lower: j = 0..i). (reference: lib/gen9blas.py:424-610)
for _name, _types in {
        "gen9blas_symv": [_i, _i, _i, _d, _p, _i, _p, _i, _d, _p, _i], "gen9blas_trmv": [_i] * 5 + [_p, _i, _p, _i],
        "gen9blas_trsv": [_i] * 5 + [_p, _i, _p, _i], "gen9blas_syr": [_i, _i, _i, _d, _p, _i, _p, _i],
        "gen9blas_syr2": [_i, _i, _i, _d, _p, _i, _p, _i, _p, _i],
        "gen9blas_gbmv": [_i] * 6 + [_d, _p, _i, _p, _i, _d, _p, _i], "gen9blas_sbmv": [_i] * 4 + [_d, _p, _i, _p, _i, _d, _p, _i],
        "gen9blas_tbmv": [_i] * 6 + [_p, _i, _p, _i], "gen9blas_tbsv": [_i] * 6 + [_p, _i, _p, _i],
        "gen9blas_spmv": [_i] * 3 + [_d, _p, _p, _i, _d, _p, _i], "gen9blas_tpmv": [_i] * 5 + [_p, _p, _i],
        "gen9blas_tpsv": [_i] * 5 + [_p, _p, _i], "gen9blas_spr": [_i] * 3 + [_d, _p, _i, _p],
        "gen9blas_spr2": [_i] * 3 + [_d, _p, _i, _p, _i, _p],
        "gen9blas_rotm": [_i, _i, _p, _i, _p, _i, ctypes.POINTER(_d)]}.items():
    getattr(_lib, _name).argtypes = _types
_fptr = ctypes.POINTER(_f)
_lib.gen9blas_rotg.argtypes = [_fptr] * 4
_lib.gen9blas_rotmg.argtypes = [_fptr, _fptr, _fptr, _f, _fptr]


def _sq(A, t, uplo):
    """(array, pointer, n, ld, transposed, triangle in memory) of a square matrix; a transposed view swaps uplo."""
    A, pa, r, c, lda, tr = _mat(A, t)
    if r != c:
        raise ValueError("expected a square matrix")
    return A, pa, r, lda, tr, ({"L": "U", "U": "L"}[uplo] if tr else uplo)


def _y_for(y, n, t, like):
    """(y, pointer, inc, beta applies) for an output vector of length n: a new one when y is None."""
    if y is None:
        y = _new_vec(n, t, like)
        y, py, _, iy = _vec(y, t, True)
        return y, py, iy, False
    y, py, ny, iy = _vec(y, t, True)
    if ny != n:
        raise ValueError("length of y does not match A")
    return y, py, iy, True


def symv(A, x, uplo="L", alpha=1.0, beta=0.0, y=None):
    """y = alpha·A·x + beta·y, A symmetric from its `uplo` triangle; without y: a new vector."""
    _init(); t = _dtype_of(A); A, pa, n, lda, _, u = _sq(A, t, uplo)
    x, px, nx, ix = _vec(x, t)
    if nx != n:
        raise ValueError("length of x does not match A")
    y, py, iy, given = _y_for(y, n, t, x)
    _check(_lib.gen9blas_symv(_kind_basic(t), _TRI[u], n, alpha, pa, lda, px, ix, beta if given else 0.0, py, iy))
    return y


def trmv(A, x, uplo="L", trans=False, diag=False):
    """x = op(A)·x in place, A triangular (`uplo`; diag=True: unit diagonal). Returns x."""
    _init(); t = _dtype_of(x); A, pa, n, lda, tr, u = _sq(A, t, uplo)
    x, px, nx, ix = _vec(x, t, True)
    if nx != n:
        raise ValueError("length of x does not match A")
    _check(_lib.gen9blas_trmv(_kind_basic(t), _TRI[u], int(trans) ^ tr, int(diag), n, pa, lda, px, ix)); return x


def trsv(A, x, uplo="L", trans=False, diag=False):
    """Solves op(A)·z = x and stores z in x, A triangular. Returns x."""
    _init(); t = _dtype_of(x); A, pa, n, lda, tr, u = _sq(A, t, uplo)
    x, px, nx, ix = _vec(x, t, True)
    if nx != n:
        raise ValueError("length of x does not match A")
    _check(_lib.gen9blas_trsv(_kind_basic(t), _TRI[u], int(trans) ^ tr, int(diag), n, pa, lda, px, ix)); return x


def syr(alpha, x, A, uplo="L"):
    """A = alpha·x·xᵀ + A on the `uplo` triangle (in place). Returns A."""
    _init(); t = _dtype_of(A); A, pa, M, N, lda, _ = _mat(A, t, True)
    x, px, n, ix = _vec(x, t)
    if not M == N == n:
        raise ValueError("dimensions do not match")
    _check(_lib.gen9blas_syr(_kind_basic(t), _TRI[uplo], n, alpha, px, ix, pa, lda)); return A


def syr2(alpha, x, y, A, uplo="L"):
    """A = alpha·(x·yᵀ + y·xᵀ) + A on the `uplo` triangle (in place). Returns A."""
    _init(); t = _dtype_of(A); A, pa, M, N, lda, _ = _mat(A, t, True)
    x, px, n, ix = _vec(x, t); y, py, ny, iy = _vec(y, t)
    if not M == N == n == ny:
        raise ValueError("dimensions do not match")
    _check(_lib.gen9blas_syr2(_kind_basic(t), _TRI[uplo], n, alpha, px, ix, py, iy, pa, lda)); return A


def _band(A, t, width, write=False):
    A, pa, rows, w, lda, tr = _mat(A, t, write)
    if tr or w != width:
        raise ValueError(f"band: expected a row-major array with {width} columns")
    return A, pa, rows, lda


def _packed(Ap, t, n, write=False):
    Ap, pp, m, inc = _vec(Ap, t, write)
    if inc != 1 or m != n * (n + 1) // 2:
        raise ValueError(f"packed: expected a contiguous vector of length {n * (n + 1) // 2}")
    return Ap, pp


def gbmv(A, x, M, N, KL, KU, alpha=1.0, beta=0.0, y=None, trans=False):
    """y = alpha·op(A)·x + beta·y, A an M×N band matrix stored as an (M, KL+KU+1) array."""
    _init(); t = _dtype_of(A); A, pa, m, lda = _band(A, t, KL + KU + 1)
    if m != M:
        raise ValueError("number of band rows != M")
    x, px, nx, ix = _vec(x, t)
    if nx != (M if trans else N):
        raise ValueError("length of x")
    y, py, iy, given = _y_for(y, N if trans else M, t, x)
    _check(_lib.gen9blas_gbmv(_kind_basic(t), int(trans), M, N, KL, KU, alpha, pa, lda, px, ix, beta if given else 0.0,
                              py, iy))
    return y


def sbmv(A, x, K, uplo="L", alpha=1.0, beta=0.0, y=None):
    """y = alpha·A·x + beta·y, A symmetric band (array (n, K+1), triangle `uplo`)."""
    _init(); t = _dtype_of(A); A, pa, n, lda = _band(A, t, K + 1)
    x, px, nx, ix = _vec(x, t)
    if nx != n:
        raise ValueError("length of x")
    y, py, iy, given = _y_for(y, n, t, x)
    _check(_lib.gen9blas_sbmv(_kind_basic(t), _TRI[uplo], n, K, alpha, pa, lda, px, ix, beta if given else 0.0, py, iy))
    return y


def tbmv(A, x, K, uplo="L", trans=False, diag=False):
    """x = op(A)·x in place, A triangular band (array (n, K+1))."""
    _init(); t = _dtype_of(x); A, pa, n, lda = _band(A, t, K + 1); x, px, nx, ix = _vec(x, t, True)
    if nx != n:
        raise ValueError("length of x")
    _check(_lib.gen9blas_tbmv(_kind_basic(t), _TRI[uplo], int(trans), int(diag), n, K, pa, lda, px, ix)); return x


def tbsv(A, x, K, uplo="L", trans=False, diag=False):
    """Solves op(A)·z = x in place, A triangular band (array (n, K+1))."""
    _init(); t = _dtype_of(x); A, pa, n, lda = _band(A, t, K + 1); x, px, nx, ix = _vec(x, t, True)
    if nx != n:
        raise ValueError("length of x")
    _check(_lib.gen9blas_tbsv(_kind_basic(t), _TRI[uplo], int(trans), int(diag), n, K, pa, lda, px, ix)); return x


def spmv(Ap, x, uplo="L", alpha=1.0, beta=0.0, y=None):
    """y = alpha·A·x + beta·y, A symmetric packed (vector of n(n+1)/2)."""
    _init(); t = _dtype_of(Ap); x, px, n, ix = _vec(x, t); Ap, pp = _packed(Ap, t, n)
    y, py, iy, given = _y_for(y, n, t, x)
    _check(_lib.gen9blas_spmv(_kind_basic(t), _TRI[uplo], n, alpha, pp, px, ix, beta if given else 0.0, py, iy)); return y


def tpmv(Ap, x, uplo="L", trans=False, diag=False):
    """x = op(A)·x in place, A triangular packed."""
    _init(); t = _dtype_of(x); x, px, n, ix = _vec(x, t, True); Ap, pp = _packed(Ap, t, n)
    _check(_lib.gen9blas_tpmv(_kind_basic(t), _TRI[uplo], int(trans), int(diag), n, pp, px, ix)); return x


def tpsv(Ap, x, uplo="L", trans=False, diag=False):
    """Solves op(A)·z = x in place, A triangular packed."""
    _init(); t = _dtype_of(x); x, px, n, ix = _vec(x, t, True); Ap, pp = _packed(Ap, t, n)
    _check(_lib.gen9blas_tpsv(_kind_basic(t), _TRI[uplo], int(trans), int(diag), n, pp, px, ix)); return x


def spr(alpha, x, Ap, uplo="L"):
    """A = alpha·x·xᵀ + A, A packed (in place). Returns Ap."""
    _init(); t = _dtype_of(Ap); x, px, n, ix = _vec(x, t); Ap, pp = _packed(Ap, t, n, True)
    _check(_lib.gen9blas_spr(_kind_basic(t), _TRI[uplo], n, alpha, px, ix, pp)); return Ap


def spr2(alpha, x, y, Ap, uplo="L"):
    """A = alpha·(x·yᵀ + y·xᵀ) + A, A packed (in place). Returns Ap."""
    _init(); t = _dtype_of(Ap); x, px, n, ix = _vec(x, t); y, py, ny, iy = _vec(y, t)
    if ny != n:
        raise ValueError("lengths of x, y")
    Ap, pp = _packed(Ap, t, n, True)
    _check(_lib.gen9blas_spr2(_kind_basic(t), _TRI[uplo], n, alpha, px, ix, py, iy, pp)); return Ap


def rotm(x, y, param):
    """x, y = h11·x + h12·y, h21·x + h22·y in place; param = (flag, h11, h21, h12, h22) as in BLAS."""
    _init(); t = _dtype_of(x); x, px, n, ix = _vec(x, t, True); y, py, ny, iy = _vec(y, t, True)
    if ny != n:
        raise ValueError("lengths differ")
    pr = (_d * 5)(*[float(v) for v in param])
    _check(_lib.gen9blas_rotm(_kind_basic(t), n, px, ix, py, iy, pr)); return x, y


def rotg(a, b):
    """(r, z, c, s) of the Givens rotation that zeroes b (computed on the host)."""
    w = [_f(a), _f(b), _f(), _f()]
    _lib.gen9blas_rotg(*[ctypes.byref(v) for v in w])
    return tuple(v.value for v in w)


def rotmg(d1, d2, x1, y1):
    """(d1, d2, x1, param) of the modified Givens rotation (computed on the host); param has 5 entries."""
    w = [_f(d1), _f(d2), _f(x1)]
    pr = (_f * 5)()
    _lib.gen9blas_rotmg(*[ctypes.byref(v) for v in w], _f(y1), pr)
    return w[0].value, w[1].value, w[2].value, np.array(pr[:], np.float32)
