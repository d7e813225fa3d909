"""gen9blas for MI355X: the Python module over libgen9blas.so (ctypes), for NumPy arrays and torch GPU tensors.

    import numpy as np, gen9blas
    C = gen9blas.hgemm(A, B)                  # float16 in, float16 out; accurate=True selects GEN9BLAS_HS
    C = gen9blas.sgemm(A.T, B, alpha=2.0)     # a transposed view travels as a transpose flag, not as a copy
    C = gen9blas.gemm_batched(A3, B3)         # (count, M, K) · (count, K, N) in one launch
    y = gen9blas.gemv(A, x); d = gen9blas.dot(x, y); gen9blas.axpy(0.5, x, y)

API contract (reference lib/gen9blas.py:96-610): the same public names, positional arguments and defaults.
- The compute type follows the data: float16, float64, and float32 for every other element type.
- Row-strided matrices, transposed views and negative vector strides reach the library without a copy. An input in
  any other layout is copied; an output in such a layout is rejected with TypeError.
- Shape mismatches raise ValueError. A non-zero library status raises RuntimeError with gen9blas_error()'s text.
- The library must report version 0.2.x.

Operands on MI355X. A NumPy array is host memory: the library stages it to the GPU and back. A torch tensor on the
GPU (or an object exposing __cuda_array_interface__) is used in place, and new results for device inputs are
allocated on the same device. empty() hands out pinned host memory (gen9blas_alloc) from a recycling pool.
"""
import atexit
import collections
import ctypes
import importlib.util
import os
import sys
from typing import NamedTuple

import numpy as np

# ------------------------------------------------------------------------------------------------------------------
# The shared library and its C signatures
# ------------------------------------------------------------------------------------------------------------------


def _library_path():
    """$GEN9BLAS_LIB, else the in-tree build next to this file, else whatever the dynamic loader finds."""
    explicit = os.environ.get("GEN9BLAS_LIB")
    if explicit:
        return explicit
    local = os.path.join(os.path.dirname(os.path.realpath(__file__)), "libgen9blas.so")
    return local if os.path.exists(local) else "libgen9blas.so"


def _share_torch_hip_runtime():
    """torch ships its own HIP runtime (torch/lib/libamdhip64.so, soname libamdhip64.so.7, RPATH $ORIGIN) and its
    libraries ask for it by the unversioned name. libgen9blas.so asks for libamdhip64.so.7, so when it is loaded
    before torch the process ends up with two HIP (and HSA) runtimes, and the second to initialize finds no device.
    Loading torch's runtime first makes libgen9blas.so bind to it by soname, and torch later reuses the same file:
    one runtime in either import order. Without torch installed, the system runtime is used."""
    if "torch" in sys.modules:
        return                                   # torch's runtime is loaded already; the soname binds to it
    spec = importlib.util.find_spec("torch")
    if spec is None or not spec.submodule_search_locations:
        return
    runtime = os.path.join(list(spec.submodule_search_locations)[0], "lib", "libamdhip64.so")
    if os.path.exists(runtime):
        ctypes.CDLL(runtime, mode=ctypes.RTLD_GLOBAL)


_share_torch_hip_runtime()
_lib = ctypes.CDLL(_library_path())

# One letter per C type. Upper case letters are pointers to the lower case scalar.
_CTYPE = {"i": ctypes.c_int, "l": ctypes.c_int64, "d": ctypes.c_double, "f": ctypes.c_float,
          "p": ctypes.c_void_p, "z": ctypes.c_size_t, "s": ctypes.c_char_p, "v": None,
          "I": ctypes.POINTER(ctypes.c_int), "L": ctypes.POINTER(ctypes.c_int64),
          "D": ctypes.POINTER(ctypes.c_double), "F": ctypes.POINTER(ctypes.c_float)}

# gen9blas_<name> = <result>:<arguments>, as declared in include/gen9blas.h, gen9blas_ml.h and gen9blas_hip.h.
_SIGNATURES = """
    version=i:  init=i:  device_gen=i:  has=i:i  error=s:  last_status=i:  last_time_ms=d:  last_zero_copy=i:
    alloc=p:z  free=v:p  is_usm=i:pz
    gemm=i:iiiiiidpipidpi  gemm_batched=i:iiiiiidpilpildpili  hgemm=i:iiidpipidpi  sgemm=i:iiidpipidpi
    pack_b=p:iiiipi  gemm_pb=i:iidpipdpi  packed_b_free=v:p  gemm_pb_skinny=i:ipippiI
    symm=i:iiiiidpipidpi  syrk=i:iiiiidpidpi  syr2k=i:iiiiidpipidpi  trmm=i:iiiiiiidpipi  trsm=i:iiiiiiidpipi
    axpy=i:iidpipi  scal=i:iidpi  copy=i:iipipi  swap=i:iipipi  rot=i:iipipidd  rotm=i:iipipiD
    rotg=v:FFFF  rotmg=v:FFFfF  dot=i:iipipiD  asum=i:iipiD  nrm2=i:iipiD  iamax=i:iipiL
    gemv=i:iiiidpipidpi  ger=i:iiidpipipi  symv=i:iiidpipidpi  trmv=i:iiiiipipi  trsv=i:iiiiipipi
    syr=i:iiidpipi  syr2=i:iiidpipipi  gbmv=i:iiiiiidpipidpi  sbmv=i:iiiidpipidpi  tbmv=i:iiiiiipipi
    tbsv=i:iiiiiipipi  spmv=i:iiidppidpi  tpmv=i:iiiiippi  tpsv=i:iiiiippi  spr=i:iiidpip  spr2=i:iiidpipip
    device_arch=i:  hip_stream=p:  device_alloc=p:z  device_free=v:p  is_device=i:pz  memcpy=i:ppz
    set_nowait=v:i  flush=i:
"""


def _declare(spec):
    for item in spec.split():
        name, sig = item.split("=")
        result, args = sig.split(":")
        fn = getattr(_lib, "gen9blas_" + name)
        fn.restype = _CTYPE[result]
        fn.argtypes = [_CTYPE[c] for c in args]


_declare(_SIGNATURES)

# Type codes of the C API (gen9blas.h) and gen9blas_has features.
GEN9BLAS_H, GEN9BLAS_S, GEN9BLAS_HS, GEN9BLAS_D = 0, 1, 2, 3
FEAT_FP16, FEAT_FP32, FEAT_FP64 = 0, 1, 2

_found = _lib.gen9blas_version()
if _found // 100 != 2:
    raise ImportError(f"this gen9blas module is written for libgen9blas 0.2.x; the library reports {_found}")

_F16, _F32, _F64 = np.dtype(np.float16), np.dtype(np.float32), np.dtype(np.float64)
_TYPE_CODE = {_F16: GEN9BLAS_H, _F32: GEN9BLAS_S, _F64: GEN9BLAS_D}
_FEATURE = {GEN9BLAS_H: FEAT_FP16, GEN9BLAS_HS: FEAT_FP16, GEN9BLAS_S: FEAT_FP32, GEN9BLAS_D: FEAT_FP64}
_SIDE_CODE = {"L": 0, "R": 1}
_UPLO_CODE = {"L": 0, "U": 1}
_OTHER_UPLO = {"L": "U", "U": "L"}
_initialized = False


def _init():
    """Initializes the library once per process; raises RuntimeError with the library's message if it cannot."""
    global _initialized
    if _initialized:
        return
    if _lib.gen9blas_init() != 0:
        raise RuntimeError(_lib.gen9blas_error().decode())
    _initialized = True


def _call(name, *args):
    """gen9blas_<name>(*args) after initialization; a non-zero status becomes RuntimeError(gen9blas_error())."""
    _init()
    if getattr(_lib, "gen9blas_" + name)(*args) != 0:
        raise RuntimeError(_lib.gen9blas_error().decode())


def hip_stream():
    """The library's HIP stream (hipStream_t as an int), e.g. for torch.cuda.ExternalStream."""
    _init()
    return _lib.gen9blas_hip_stream()


def set_nowait(on):
    """No-wait mode: calls whose operands are all in device memory return once queued; flush() waits for them."""
    _lib.gen9blas_set_nowait(1 if on else 0)


def flush():
    _call("flush")


def last_time_ms():
    """Duration of the last call in ms: the device time of its kernels with GEN9BLAS_PROFILE=1, else the whole call."""
    return _lib.gen9blas_last_time_ms()


def last_zero_copy():
    """Operands of the last level-3 call used in place in device memory, as bits: 1 = A, 2 = B, 4 = C."""
    return _lib.gen9blas_last_zero_copy()


# ------------------------------------------------------------------------------------------------------------------
# Pinned host memory: empty() and its pool
# ------------------------------------------------------------------------------------------------------------------
POOL_MAX = 1 << 30     # bytes of released pinned blocks kept for reuse; blocks beyond that are freed at release
_exiting = False


@atexit.register
def _mark_exit():
    # Arrays collected during interpreter shutdown must not call into a library that may already be torn down; the
    # process exit returns pinned memory to the driver anyway.
    global _exiting
    _exiting = True


class _PinnedPool:
    """Pinned (page-locked) host blocks from gen9blas_alloc, which the DMA engines read at full speed but which are
    slow to allocate. A released block waits, keyed by its size class, for a later request of the same class."""

    def __init__(self):
        self.spare = collections.defaultdict(list)
        self.spare_bytes = 0

    @staticmethod
    def size_class(nbytes):
        """Powers of two up to 1 MiB (at least one 4 KiB page), whole MiB above: a small block wastes at most half of
        itself, a large one less than 1 MiB."""
        if nbytes <= 1 << 20:
            return max(4096, 1 << max(nbytes - 1, 0).bit_length())
        return -(-nbytes >> 20) << 20

    def take(self, nbytes):
        size = self.size_class(nbytes)
        if self.spare[size]:
            self.spare_bytes -= size
            return self.spare[size].pop(), size
        _init()
        ptr = _lib.gen9blas_alloc(size)
        if not ptr:
            raise MemoryError(_lib.gen9blas_error().decode())
        return ptr, size

    def give(self, ptr, size):
        if self.spare_bytes + size > POOL_MAX:
            _lib.gen9blas_free(ptr)
            return
        self.spare[size].append(ptr)
        self.spare_bytes += size

    def drain(self):
        for blocks in self.spare.values():
            while blocks:
                _lib.gen9blas_free(blocks.pop())
        self.spare_bytes = 0


_pool = _PinnedPool()


class _PinnedBlock:
    """Owns one pooled block. NumPy arrays built on it hold it through their .base chain, so it is collected, and the
    block handed back to the pool, only when no view of it is left."""

    def __init__(self, ptr, size, nbytes):
        self.ptr, self.size = ptr, size
        self.__array_interface__ = {"version": 3, "shape": (nbytes,), "typestr": "|u1", "data": (ptr, False)}

    def __del__(self):
        if not _exiting:
            _pool.give(self.ptr, self.size)


def empty(shape, dtype=np.float16):
    """Uninitialized C-contiguous array in pinned host memory (faster transfers than pageable NumPy memory). When
    every view of it is gone, its block returns to a pool (up to POOL_MAX bytes) for later empty() calls."""
    dt = np.dtype(dtype)
    shape = (int(shape),) if np.ndim(shape) == 0 else tuple(int(s) for s in shape)
    nbytes = int(np.prod(shape, dtype=np.int64)) * dt.itemsize
    ptr, size = _pool.take(nbytes)
    return np.asarray(_PinnedBlock(ptr, size, nbytes)).view(dt).reshape(shape)


def free_pool():
    """Frees the released blocks waiting in the pool (arrays still in use keep theirs)."""
    _pool.drain()


# ------------------------------------------------------------------------------------------------------------------
# Operands: one description for NumPy arrays and torch tensors
# ------------------------------------------------------------------------------------------------------------------
_torch = None


def _torch_module():
    global _torch
    if _torch is None:
        import torch
        _torch = torch
    return _torch


def _is_tensor(X):
    return type(X).__module__.startswith("torch") and hasattr(X, "data_ptr")


def _torch_dtype(t):
    torch = _torch_module()
    return {_F16: torch.float16, _F32: torch.float32, _F64: torch.float64}[t]


def _numpy_dtype(X):
    """Element type of X as a NumPy dtype, or None for a torch type NumPy does not know (bfloat16, ...)."""
    if _is_tensor(X):
        name = str(X.dtype).rpartition(".")[2]
        return np.dtype(name) if name in ("float16", "float32", "float64") else None
    return np.asarray(X).dtype if not hasattr(X, "dtype") else np.dtype(X.dtype)


class _Operand(NamedTuple):
    obj: object        # the array or tensor the address belongs to
    ptr: int
    shape: tuple
    steps: tuple       # strides in elements; None if one of them is not a whole number of elements
    dtype: object      # NumPy dtype, or None (an element type the library has no kernel for)
    on_gpu: bool


def _operand(X):
    if _is_tensor(X):
        if X.is_cuda:
            return _Operand(X, X.data_ptr(), tuple(X.shape), tuple(X.stride()), _numpy_dtype(X), True)
        X = X.numpy()                                   # a CPU tensor: its NumPy view shares the memory
    elif hasattr(X, "__cuda_array_interface__") and not isinstance(X, np.ndarray):
        return _operand(_torch_module().as_tensor(X, device="cuda"))
    X = X if isinstance(X, np.ndarray) else np.asarray(X)
    e = X.itemsize
    steps = tuple(s // e for s in X.strides) if all(s % e == 0 for s in X.strides) else None
    return _Operand(X, X.ctypes.data, X.shape, steps, X.dtype, False)


def _compute_type(X):
    """float16 and float64 compute in their own type, everything else in float32."""
    dt = _numpy_dtype(X)
    return dt if dt in (_F16, _F64) else _F32


def _strict_type(X):
    dt = _numpy_dtype(X)
    if dt not in _TYPE_CODE:
        raise TypeError("supported types: float16, float32, float64")
    return dt


def _kind(t, accurate=False):
    return GEN9BLAS_HS if (accurate and t == _F16) else _TYPE_CODE[t]


def available(dt, accurate=False):
    """Whether the device runs this element type (float16 with accurate=True: the GEN9BLAS_HS mode)."""
    _init()
    dt = np.dtype(str(dt).rpartition(".")[2]) if not isinstance(dt, (np.dtype, type)) else np.dtype(dt)
    if dt not in _TYPE_CODE:
        raise TypeError("supported types: float16, float32, float64")
    return bool(_lib.gen9blas_has(_FEATURE[_kind(dt, accurate)]))


def _dense(X, t):
    """X as a C-contiguous array of type t on the same side (host or device); no copy if it already is one."""
    if _is_tensor(X) and X.is_cuda:
        return X.to(dtype=_torch_dtype(t)).contiguous()
    return np.ascontiguousarray(X, dtype=t)


def _as_type(X, t):
    """X itself if its elements are already of type t (any layout), else a converted copy."""
    if _numpy_dtype(X) == t:
        return X
    if _is_tensor(X) and X.is_cuda:
        return X.to(dtype=_torch_dtype(t))
    return np.asarray(X).astype(t)


def _transposed(X):
    return X.t() if _is_tensor(X) else X.T


def _writable_check(X, what):
    if not (isinstance(X, np.ndarray) or _is_tensor(X) or hasattr(X, "__cuda_array_interface__")):
        raise TypeError(f"the result ({what}) must be a NumPy array or a GPU tensor")


class _Mat(NamedTuple):
    keep: object       # what the address belongs to (the argument, or its copy)
    ptr: int
    shape: tuple       # the shape the caller sees
    ld: int            # row stride of the matrix as it lies in memory
    trans: int         # 1: the caller's matrix is the transpose of the row-major matrix in memory

    @property
    def stored(self):
        return self.shape[::-1] if self.trans else self.shape


def _matrix(X, t, out=False):
    """A 2-D operand of type t as the library takes it: row-major with a row stride, or (inputs only) the transpose
    of one. Inputs in another layout or type are copied; outputs must already be row-major of type t."""
    if out:
        _writable_check(X, "matrix")
    d = _operand(X)
    if len(d.shape) != 2:
        raise ValueError("expected a 2-D matrix")
    rows, cols = d.shape
    if d.dtype == t and d.steps is not None:
        row_step, col_step = d.steps
        if col_step == 1 and row_step >= max(cols, 1):
            return _Mat(d.obj, d.ptr, (rows, cols), row_step, 0)
        if not out and row_step == 1 and col_step >= max(rows, 1):
            return _Mat(d.obj, d.ptr, (rows, cols), col_step, 1)
        if rows <= 1 and col_step == 1:                 # one row: any row stride will do
            return _Mat(d.obj, d.ptr, (rows, cols), max(cols, 1), 0)
    if out:
        raise TypeError(f"the result must be a {t.name} matrix with contiguous rows")
    return _matrix(_dense(d.obj, t), t)


class _Vec(NamedTuple):
    keep: object
    ptr: int           # lowest address touched (for inc < 0 the last element), as BLAS expects
    n: int
    inc: int


def _vector(x, t, out=False):
    """A 1-D operand of type t with a non-zero element stride (negative strides allowed). Inputs of another type or
    with a stride that is not a whole number of elements are copied; outputs raise TypeError instead."""
    if out:
        _writable_check(x, "vector")
    d = _operand(x)
    if len(d.shape) != 1:
        raise ValueError("expected a 1-D vector")
    n = d.shape[0]
    if d.dtype == t and d.steps is not None and d.steps[0] != 0:
        inc = d.steps[0]
        low = d.ptr + (inc * (n - 1) * t.itemsize if inc < 0 and n > 0 else 0)
        return _Vec(d.obj, low, n, inc)
    if out:
        raise TypeError(f"the result must be a {t.name} vector whose stride is a non-zero multiple of the element size")
    return _vector(_dense(d.obj, t), t)


def _equal_lengths(*vs):
    if len({v.n for v in vs}) > 1:
        raise ValueError("vector lengths differ")
    return vs


SMALL_RESULT = 128 << 10   # bytes: host results up to this size are plain NumPy arrays


def _new(shape, t, like):
    """A new result: on the device of `like` if that is a GPU tensor; else in host memory, pinned (copied back by
    one DMA) above SMALL_RESULT bytes, and a plain NumPy array below, which the library copies back through its own
    pinned bounce area (a pinned block costs more Python time than such a copy saves)."""
    d = _operand(like)
    if d.on_gpu:
        return _torch_module().empty(tuple(shape), dtype=_torch_dtype(t), device=d.obj.device)
    if int(np.prod(shape, dtype=np.int64)) * np.dtype(t).itemsize <= SMALL_RESULT:
        return np.empty(shape, t)
    return empty(shape, t)


class _Out(NamedTuple):
    obj: object
    ptr: int
    ld: int            # row stride (matrices) or element stride (vectors)
    given: bool        # the caller supplied it, so beta applies

    def beta(self, beta):
        return beta if self.given else 0.0


def _out_matrix(C, shape, t, like):
    if C is None:
        C = _new(shape, t, like)
        return _Out(C, _operand(C).ptr, shape[-1], False)
    _writable_check(C, "C")
    d = _operand(C)
    if tuple(d.shape) != tuple(shape) or d.dtype != t or d.steps is None or d.steps[-1] != 1:
        raise ValueError(f"C must have shape {tuple(shape)}, type {t.name} and contiguous rows")
    if len(shape) == 2:
        return _Out(C, d.ptr, _matrix(C, t, out=True).ld, True)
    dense_steps = tuple(int(np.prod(shape[i + 1:], dtype=np.int64)) for i in range(len(shape)))
    if any(s != w for s, w, n in zip(d.steps, dense_steps, shape) if n > 1):
        raise ValueError("C (batch) must be C-contiguous")
    return _Out(C, d.ptr, shape[-1], True)


def _out_vector(y, n, t, like):
    if y is None:
        y = _new((n,), t, like)
        v = _vector(y, t, out=True)
        return _Out(y, v.ptr, v.inc, False)
    v = _vector(y, t, out=True)
    if v.n != n:
        raise ValueError(f"y has length {v.n}, the product has {n}")
    return _Out(y, v.ptr, v.inc, True)


def _square(A, t, uplo):
    """A square matrix whose `uplo` triangle is meant, and the triangle as it lies in memory (a transposed view holds
    the caller's lower triangle in the stored matrix's upper one)."""
    a = _matrix(A, t)
    if a.shape[0] != a.shape[1]:
        raise ValueError("expected a square matrix")
    return a, (_OTHER_UPLO[uplo] if a.trans else uplo)


def _private_copy(B, t):
    """A new C-contiguous copy of B that a routine may overwrite: on B's device, or in pinned host memory."""
    if _is_tensor(B) and B.is_cuda:
        return B.to(dtype=_torch_dtype(t), copy=True).contiguous()
    b = empty(np.shape(B), t)
    b[...] = B
    return b


# ------------------------------------------------------------------------------------------------------------------
# Level 3
# ------------------------------------------------------------------------------------------------------------------


def gemm(A, B, alpha=1.0, beta=0.0, C=None, accurate=False):
    """C = alpha·A·B + beta·C in the type of A (float16, float32, float64; other types compute in float32). beta
    applies only to a supplied C. float16 with accurate=True is GEN9BLAS_HS."""
    t = _compute_type(A)
    a, b = _matrix(A, t), _matrix(B, t)
    (M, K), (K_b, N) = a.shape, b.shape
    if K != K_b:
        raise ValueError(f"incompatible dimensions: {a.shape} · {b.shape}")
    c = _out_matrix(C, (M, N), t, A)
    _call("gemm", _kind(t, accurate), a.trans, b.trans, M, N, K, alpha, a.ptr, a.ld, b.ptr, b.ld, c.beta(beta),
          c.ptr, c.ld)
    return c.obj


def hgemm(A, B, alpha=1.0, beta=0.0, C=None, accurate=False):
    """gemm in float16 (inputs of another type are converted first)."""
    return gemm(_as_type(A, _F16), _as_type(B, _F16), alpha, beta, C, accurate)


def sgemm(A, B, alpha=1.0, beta=0.0, C=None):
    """gemm in float32 (inputs of another type are converted first)."""
    return gemm(_as_type(A, _F32), _as_type(B, _F32), alpha, beta, C)


def gemm_batched(A, B, alpha=1.0, beta=0.0, C=None, accurate=False):
    """C[i] = alpha·A[i]·B[i] + beta·C[i] for stacks A (count, M, K) and B (count, K, N), in one launch."""
    t = _compute_type(A)
    a, b = _dense(A, t), _dense(B, t)
    if len(a.shape) != 3 or len(b.shape) != 3:
        raise ValueError("expected stacks of matrices (count, rows, columns)")
    (count, M, K), (count_b, K_b, N) = tuple(a.shape), tuple(b.shape)
    if (count, K) != (count_b, K_b):
        raise ValueError(f"incompatible dimensions: {tuple(a.shape)} · {tuple(b.shape)}")
    c = _out_matrix(C, (count, M, N), t, A)
    _call("gemm_batched", _kind(t, accurate), 0, 0, M, N, K, alpha, _operand(a).ptr, K, M * K, _operand(b).ptr, N,
          K * N, c.beta(beta), c.ptr, N, M * N, count)
    return c.obj


def symm(A, B, side="L", uplo="L", alpha=1.0, beta=0.0, C=None, accurate=False):
    """C = alpha·A·B + beta·C (side "L") or alpha·B·A + beta·C (side "R"), A symmetric from its `uplo` triangle."""
    t = _strict_type(B)
    a, stored_uplo = _square(A, t, uplo)
    b = _matrix(B, t)
    if b.trans:
        b = _matrix(_dense(B, t), t)
    M, N = b.shape
    c = _out_matrix(C, (M, N), t, B)
    _call("symm", _kind(t, accurate), _SIDE_CODE[side], _UPLO_CODE[stored_uplo], M, N, alpha, a.ptr, a.ld, b.ptr,
          b.ld, c.beta(beta), c.ptr, c.ld)
    return c.obj


def syrk(A, uplo="L", trans=False, alpha=1.0, beta=0.0, C=None, accurate=False):
    """The `uplo` triangle of alpha·A·Aᵀ + beta·C (trans: alpha·Aᵀ·A + beta·C); a new C is zero off the triangle."""
    t = _strict_type(A)
    a = _matrix(A, t)
    N, K = a.shape[::-1] if trans else a.shape
    c = _out_matrix(C, (N, N), t, A)
    if not c.given:
        c.obj[...] = 0
    _call("syrk", _kind(t, accurate), _UPLO_CODE[uplo], int(bool(trans)) ^ a.trans, N, K, alpha, a.ptr, a.ld,
          c.beta(beta), c.ptr, c.ld)
    return c.obj


def syr2k(A, B, uplo="L", trans=False, alpha=1.0, beta=0.0, C=None, accurate=False):
    """The `uplo` triangle of alpha·(A·Bᵀ + B·Aᵀ) + beta·C (trans: alpha·(Aᵀ·B + Bᵀ·A) + beta·C)."""
    t = _strict_type(A)
    a, b = _matrix(A, t), _matrix(B, t)
    if b.trans != a.trans:
        # One transpose flag covers both operands: lay B out in memory the way A lies.
        b = _matrix(_transposed(_dense(_transposed(B), t)) if a.trans else _dense(B, t), t)
    N, K = a.shape[::-1] if trans else a.shape
    c = _out_matrix(C, (N, N), t, A)
    if not c.given:
        c.obj[...] = 0
    _call("syr2k", _kind(t, accurate), _UPLO_CODE[uplo], int(bool(trans)) ^ a.trans, N, K, alpha, a.ptr, a.ld, b.ptr,
          b.ld, c.beta(beta), c.ptr, c.ld)
    return c.obj


def _triangular_solve_or_product(name, A, B, side, uplo, transA, diag, alpha, accurate, t):
    a, stored_uplo = _square(A, t, uplo)
    X = _private_copy(B, t)
    M, N = X.shape
    _call(name, _kind(t, accurate), _SIDE_CODE[side], _UPLO_CODE[stored_uplo], int(bool(transA)) ^ a.trans,
          int(bool(diag)), M, N, alpha, a.ptr, a.ld, _operand(X).ptr, max(N, 1))
    return X


def trmm(A, B, side="L", uplo="L", transA=False, diag=False, alpha=1.0, accurate=False):
    """alpha·op(A)·B (side "L") or alpha·B·op(A) (side "R"), A triangular (diag: unit diagonal). B is unchanged."""
    return _triangular_solve_or_product("trmm", A, B, side, uplo, transA, diag, alpha, accurate, _strict_type(B))


def trsm(A, B, side="L", uplo="L", transA=False, diag=False, alpha=1.0, accurate=False):
    """X with op(A)·X = alpha·B (side "L") or X·op(A) = alpha·B (side "R"), A triangular. B is unchanged."""
    return _triangular_solve_or_product("trsm", A, B, side, uplo, transA, diag, alpha, accurate, _compute_type(B))


# ------------------------------------------------------------------------------------------------------------------
# Level 1 (float16 computes in float32; dot, asum and nrm2 accumulate in float64)
# ------------------------------------------------------------------------------------------------------------------


def _two_in_place(name, x, y, *extra):
    t = _compute_type(x)
    vx, vy = _equal_lengths(_vector(x, t, out=True), _vector(y, t, out=True))
    _call(name, _TYPE_CODE[t], vx.n, vx.ptr, vx.inc, vy.ptr, vy.inc, *extra)
    return x, y


def _reduction(name, box, *xs):
    t = _compute_type(xs[0])
    vs = _equal_lengths(*(_vector(x, t) for x in xs))
    args = [a for v in vs for a in (v.ptr, v.inc)]
    result = box()
    _call(name, _TYPE_CODE[t], vs[0].n, *args, ctypes.byref(result))
    return result.value


def axpy(a, x, y):
    """y = a·x + y in place; returns y."""
    t = _compute_type(y)
    vy, vx = _equal_lengths(_vector(y, t, out=True), _vector(x, t))
    _call("axpy", _TYPE_CODE[t], vy.n, a, vx.ptr, vx.inc, vy.ptr, vy.inc)
    return y


def scal(a, x):
    """x = a·x in place; returns x."""
    t = _compute_type(x)
    vx = _vector(x, t, out=True)
    _call("scal", _TYPE_CODE[t], vx.n, a, vx.ptr, vx.inc)
    return x


def copy(x, y=None):
    """y = x; without y, a new vector of x's type (on x's device for a GPU tensor)."""
    t = _compute_type(x if y is None else y)
    if y is None:
        y = _new((len(x),), t, x)
    vy, vx = _equal_lengths(_vector(y, t, out=True), _vector(x, t))
    _call("copy", _TYPE_CODE[t], vy.n, vx.ptr, vx.inc, vy.ptr, vy.inc)
    return y


def swap(x, y):
    """Exchanges x and y in place; returns (x, y)."""
    return _two_in_place("swap", x, y)


def rot(x, y, c, s):
    """x, y = c·x + s·y, c·y − s·x in place; returns (x, y)."""
    return _two_in_place("rot", x, y, c, s)


def rotm(x, y, param):
    """x, y = h11·x + h12·y, h21·x + h22·y in place; param = (flag, h11, h21, h12, h22) as in BLAS."""
    return _two_in_place("rotm", x, y, (ctypes.c_double * 5)(*map(float, param)))


def dot(x, y):
    """Σ x·y as a Python float (float64 accumulation)."""
    return _reduction("dot", ctypes.c_double, x, y)


def asum(x):
    """Σ |x|."""
    return _reduction("asum", ctypes.c_double, x)


def nrm2(x):
    """Euclidean norm of x."""
    return _reduction("nrm2", ctypes.c_double, x)


def iamax(x):
    """0-based index of the first element of largest |x|; -1 for an empty vector."""
    return _reduction("iamax", ctypes.c_int64, x)


def rotg(a, b):
    """(r, z, c, s) of the Givens rotation that zeroes b (computed on the host, in float32)."""
    cells = [ctypes.c_float(v) for v in (a, b, 0.0, 0.0)]
    _lib.gen9blas_rotg(*map(ctypes.byref, cells))
    return tuple(c.value for c in cells)


def rotmg(d1, d2, x1, y1):
    """(d1, d2, x1, param) of the modified Givens rotation (host, float32); param holds 5 numbers as in BLAS."""
    cells = [ctypes.c_float(v) for v in (d1, d2, x1)]
    param = (ctypes.c_float * 5)()
    _lib.gen9blas_rotmg(*map(ctypes.byref, cells), ctypes.c_float(y1), param)
    return cells[0].value, cells[1].value, cells[2].value, np.frombuffer(param, np.float32).copy()


# ------------------------------------------------------------------------------------------------------------------
# Level 2 on general and full-storage matrices
# ------------------------------------------------------------------------------------------------------------------


def _vector_of_length(x, n, t, out=False, what="x"):
    v = _vector(x, t, out)
    if v.n != n:
        raise ValueError(f"{what} has length {v.n}, the matrix needs {n}")
    return v


def gemv(A, x, alpha=1.0, beta=0.0, y=None, trans=False):
    """y = alpha·op(A)·x + beta·y (op = transpose when trans); without y, a new vector. A.T passes as a flag."""
    t = _compute_type(A)
    a = _matrix(A, t)
    M, N = a.stored
    tr = a.trans ^ int(bool(trans))
    vx = _vector_of_length(x, M if tr else N, t)
    o = _out_vector(y, N if tr else M, t, A)
    _call("gemv", _TYPE_CODE[t], tr, M, N, alpha, a.ptr, a.ld, vx.ptr, vx.inc, o.beta(beta), o.ptr, o.ld)
    return o.obj


def ger(alpha, x, y, A):
    """A = alpha·x·yᵀ + A in place; returns A."""
    t = _compute_type(A)
    a = _matrix(A, t, out=True)
    M, N = a.shape
    vx, vy = _vector_of_length(x, M, t), _vector_of_length(y, N, t, what="y")
    _call("ger", _TYPE_CODE[t], M, N, alpha, vx.ptr, vx.inc, vy.ptr, vy.inc, a.ptr, a.ld)
    return A


def symv(A, x, uplo="L", alpha=1.0, beta=0.0, y=None):
    """y = alpha·A·x + beta·y with A symmetric from its `uplo` triangle; without y, a new vector."""
    t = _compute_type(A)
    a, u = _square(A, t, uplo)
    n = a.shape[0]
    vx = _vector_of_length(x, n, t)
    o = _out_vector(y, n, t, x)
    _call("symv", _TYPE_CODE[t], _UPLO_CODE[u], n, alpha, a.ptr, a.ld, vx.ptr, vx.inc, o.beta(beta), o.ptr, o.ld)
    return o.obj


def _triangular_vector(name, A, x, uplo, trans, diag):
    t = _compute_type(x)
    a, u = _square(A, t, uplo)
    vx = _vector_of_length(x, a.shape[0], t, out=True)
    _call(name, _TYPE_CODE[t], _UPLO_CODE[u], int(bool(trans)) ^ a.trans, int(bool(diag)), vx.n, a.ptr, a.ld, vx.ptr,
          vx.inc)
    return x


def trmv(A, x, uplo="L", trans=False, diag=False):
    """x = op(A)·x in place, A triangular (`uplo`; diag: unit diagonal); returns x."""
    return _triangular_vector("trmv", A, x, uplo, trans, diag)


def trsv(A, x, uplo="L", trans=False, diag=False):
    """Overwrites x with the solution z of op(A)·z = x, A triangular; returns x."""
    return _triangular_vector("trsv", A, x, uplo, trans, diag)


def syr(alpha, x, A, uplo="L"):
    """A = alpha·x·xᵀ + A on the `uplo` triangle, in place; returns A."""
    t = _compute_type(A)
    a = _matrix(A, t, out=True)
    if a.shape[0] != a.shape[1]:
        raise ValueError("expected a square matrix")
    vx = _vector_of_length(x, a.shape[0], t)
    _call("syr", _TYPE_CODE[t], _UPLO_CODE[uplo], vx.n, alpha, vx.ptr, vx.inc, a.ptr, a.ld)
    return A


def syr2(alpha, x, y, A, uplo="L"):
    """A = alpha·(x·yᵀ + y·xᵀ) + A on the `uplo` triangle, in place; returns A."""
    t = _compute_type(A)
    a = _matrix(A, t, out=True)
    if a.shape[0] != a.shape[1]:
        raise ValueError("expected a square matrix")
    vx, vy = _vector_of_length(x, a.shape[0], t), _vector_of_length(y, a.shape[0], t, what="y")
    _call("syr2", _TYPE_CODE[t], _UPLO_CODE[uplo], vx.n, alpha, vx.ptr, vx.inc, vy.ptr, vy.inc, a.ptr, a.ld)
    return A


# ------------------------------------------------------------------------------------------------------------------
# Level 2 on band and packed storage (row layout of CBLAS RowMajor).
# Band: an array (rows, KL+KU+1) with A[i, j] at row i, column KL + j − i; symmetric and triangular band matrices use
# KL = K, KU = 0 (lower) or KL = 0, KU = K (upper). Packed: a contiguous vector of n(n+1)/2 elements holding the rows
# of the triangle one after another (upper: j = i..n−1, lower: j = 0..i). (reference lib/gen9blas.py:517-610)
# ------------------------------------------------------------------------------------------------------------------


def _band(A, t, width):
    a = _matrix(A, t)
    if a.trans or a.shape[1] != width:
        raise ValueError(f"band storage: expected a row-major array with {width} columns")
    return a


def _packed(Ap, t, n, out=False):
    v = _vector(Ap, t, out)
    if v.inc != 1 or v.n != n * (n + 1) // 2:
        raise ValueError(f"packed storage: expected a contiguous vector of {n * (n + 1) // 2} elements")
    return v


def gbmv(A, x, M, N, KL, KU, alpha=1.0, beta=0.0, y=None, trans=False):
    """y = alpha·op(A)·x + beta·y, A an M×N band matrix with KL sub- and KU super-diagonals."""
    t = _compute_type(A)
    a = _band(A, t, KL + KU + 1)
    if a.shape[0] != M:
        raise ValueError(f"band storage has {a.shape[0]} rows, M is {M}")
    vx = _vector_of_length(x, M if trans else N, t)
    o = _out_vector(y, N if trans else M, t, x)
    _call("gbmv", _TYPE_CODE[t], int(bool(trans)), M, N, KL, KU, alpha, a.ptr, a.ld, vx.ptr, vx.inc, o.beta(beta),
          o.ptr, o.ld)
    return o.obj


def sbmv(A, x, K, uplo="L", alpha=1.0, beta=0.0, y=None):
    """y = alpha·A·x + beta·y, A symmetric band (array (n, K+1) of its `uplo` triangle)."""
    t = _compute_type(A)
    a = _band(A, t, K + 1)
    n = a.shape[0]
    vx = _vector_of_length(x, n, t)
    o = _out_vector(y, n, t, x)
    _call("sbmv", _TYPE_CODE[t], _UPLO_CODE[uplo], n, K, alpha, a.ptr, a.ld, vx.ptr, vx.inc, o.beta(beta), o.ptr, o.ld)
    return o.obj


def _band_triangular(name, A, x, K, uplo, trans, diag):
    t = _compute_type(x)
    a = _band(A, t, K + 1)
    vx = _vector_of_length(x, a.shape[0], t, out=True)
    _call(name, _TYPE_CODE[t], _UPLO_CODE[uplo], int(bool(trans)), int(bool(diag)), vx.n, K, a.ptr, a.ld, vx.ptr,
          vx.inc)
    return x


def tbmv(A, x, K, uplo="L", trans=False, diag=False):
    """x = op(A)·x in place, A triangular band (array (n, K+1))."""
    return _band_triangular("tbmv", A, x, K, uplo, trans, diag)


def tbsv(A, x, K, uplo="L", trans=False, diag=False):
    """Overwrites x with the solution of op(A)·z = x, A triangular band (array (n, K+1))."""
    return _band_triangular("tbsv", A, x, K, uplo, trans, diag)


def spmv(Ap, x, uplo="L", alpha=1.0, beta=0.0, y=None):
    """y = alpha·A·x + beta·y, A symmetric in packed storage."""
    t = _compute_type(Ap)
    vx = _vector(x, t)
    ap = _packed(Ap, t, vx.n)
    o = _out_vector(y, vx.n, t, x)
    _call("spmv", _TYPE_CODE[t], _UPLO_CODE[uplo], vx.n, alpha, ap.ptr, vx.ptr, vx.inc, o.beta(beta), o.ptr, o.ld)
    return o.obj


def _packed_triangular(name, Ap, x, uplo, trans, diag):
    t = _compute_type(x)
    vx = _vector(x, t, out=True)
    ap = _packed(Ap, t, vx.n)
    _call(name, _TYPE_CODE[t], _UPLO_CODE[uplo], int(bool(trans)), int(bool(diag)), vx.n, ap.ptr, vx.ptr, vx.inc)
    return x


def tpmv(Ap, x, uplo="L", trans=False, diag=False):
    """x = op(A)·x in place, A triangular in packed storage."""
    return _packed_triangular("tpmv", Ap, x, uplo, trans, diag)


def tpsv(Ap, x, uplo="L", trans=False, diag=False):
    """Overwrites x with the solution of op(A)·z = x, A triangular in packed storage."""
    return _packed_triangular("tpsv", Ap, x, uplo, trans, diag)


def spr(alpha, x, Ap, uplo="L"):
    """A = alpha·x·xᵀ + A in packed storage, in place; returns Ap."""
    t = _compute_type(Ap)
    vx = _vector(x, t)
    ap = _packed(Ap, t, vx.n, out=True)
    _call("spr", _TYPE_CODE[t], _UPLO_CODE[uplo], vx.n, alpha, vx.ptr, vx.inc, ap.ptr)
    return Ap


def spr2(alpha, x, y, Ap, uplo="L"):
    """A = alpha·(x·yᵀ + y·xᵀ) + A in packed storage, in place; returns Ap."""
    t = _compute_type(Ap)
    vx, vy = _equal_lengths(_vector(x, t), _vector(y, t))
    ap = _packed(Ap, t, vx.n, out=True)
    _call("spr2", _TYPE_CODE[t], _UPLO_CODE[uplo], vx.n, alpha, vx.ptr, vx.inc, vy.ptr, vy.inc, ap.ptr)
    return Ap
