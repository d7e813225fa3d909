"""Status codes and error reporting on a GPU, following the reference's error test (reference: lib/test_errors.py:33-61).

init succeeds once per process; has(unknown) = 0; device_gen is 9; a wrong type gives UNSUPPORTED; a bad leading
dimension or a zero increment gives INVALID_ARG; gemm_pb(NULL) gives INVALID_ARG; pack_b with a bad type or K = 0
returns NULL and sets last_status; an impossible pinned allocation returns NULL with OUT_OF_MEMORY. Also: a
non-positive dimension is a no-op returning 0 (reference: lib/src/gemm.c:10), and gen9blas_error() holds a message
after every failure.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

OK, DECLINED, ERR, UNSUPPORTED, INVALID, OOM, NO_DEVICE = 0, 1, -1, -2, -3, -4, -5


@pytest.fixture(scope="module")
def L(g9):
    L = g9._lib
    i, d, p = ctypes.c_int, ctypes.c_double, ctypes.c_void_p
    L.gen9blas_gemv.argtypes = [i, i, i, i, d, p, i, p, i, d, p, i]
    L.gen9blas_axpy.argtypes = [i, i, d, p, i, p, i]
    L.gen9blas_gemm_pb.argtypes = [i, i, d, p, i, p, d, p, i]
    L.gen9blas_pack_b.argtypes = [i, i, i, i, p, i]
    L.gen9blas_pack_b.restype = p
    return L


def test_library_state(L):
    assert L.gen9blas_version() // 100 == 2
    assert L.gen9blas_init() == OK
    assert L.gen9blas_init() == OK
    assert L.gen9blas_has(999) == 0
    assert L.gen9blas_has(0) == 1 and L.gen9blas_has(1) == 1 and L.gen9blas_has(2) == 1
    assert L.gen9blas_device_gen() in (8, 9)
    assert L.gen9blas_device_arch() == 950


def test_status_codes(L):
    a = np.ones((8, 8), np.float32)
    b = np.ones((8, 8), np.float32)
    c = np.zeros((8, 8), np.float32)
    pa, pb, pc = a.ctypes.data, b.ctypes.data, c.ctypes.data
    assert L.gen9blas_gemm(1, 0, 0, 8, 8, 8, 1.0, pa, 8, pb, 8, 0.0, pc, 8) == OK
    assert L.gen9blas_last_status() == OK
    assert np.all(c == 8.0)
    assert L.gen9blas_gemm(7, 0, 0, 8, 8, 8, 1.0, pa, 8, pb, 8, 0.0, pc, 8) == UNSUPPORTED
    assert L.gen9blas_last_status() == UNSUPPORTED and L.gen9blas_error()
    c[:] = -1
    for M, N, K in ((0, 8, 8), (8, -1, 8), (8, 8, 0)):
        assert L.gen9blas_gemm(1, 0, 0, M, N, K, 1.0, pa, 8, pb, 8, 0.0, pc, 8) == OK
    assert np.all(c == -1), "a call with a non-positive dimension wrote C"
    assert L.gen9blas_gemm(1, 0, 0, 8, 8, 8, 1.0, pa, 4, pb, 8, 0.0, pc, 8) == INVALID   # lda < K
    x = np.ones(8, np.float32)
    y = np.zeros(8, np.float32)
    assert L.gen9blas_gemv(1, 0, 8, 8, 1.0, pa, 4, x.ctypes.data, 1, 0.0, y.ctypes.data, 1) == INVALID
    assert L.gen9blas_axpy(1, 8, 1.0, x.ctypes.data, 0, y.ctypes.data, 1) == INVALID
    assert b"increment" in L.gen9blas_error()
    assert L.gen9blas_gemm_pb(0, 8, 1.0, pa, 8, None, 0.0, pc, 8) == INVALID
    assert L.gen9blas_pack_b(7, 0, 8, 8, pb, 8) is None
    assert L.gen9blas_last_status() == UNSUPPORTED
    assert L.gen9blas_pack_b(1, 0, 0, 8, pb, 8) is None
    assert L.gen9blas_last_status() == INVALID
    assert L.gen9blas_alloc(1 << 44) is None
    assert L.gen9blas_last_status() == OOM
    assert L.gen9blas_gemm(1, 0, 0, 8, 8, 8, 1.0, pa, 8, pb, 8, 0.0, pc, 8) == OK   # errors are not sticky


def test_level23_type_check_and_host_operands(L):
    """Level 2 / level 3 entry points check the type first, as the reference does (UNSUPPORTED, with the type in the
    message), and compute on host memory like every other entry point (reference: lib/src/level12.c, level3.c)."""
    a = np.eye(8, dtype=np.float32) * 2
    x = np.arange(8, dtype=np.float32)
    y = np.zeros(8, np.float32)
    d = ctypes.c_double
    assert L.gen9blas_symv(1, 0, 8, d(1.0), a.ctypes.data, 8, x.ctypes.data, 1, d(0.0), y.ctypes.data, 1) == OK
    assert np.array_equal(y, 2 * x)
    assert L.gen9blas_symv(9, 0, 8, d(1.0), a.ctypes.data, 8, x.ctypes.data, 1, d(0.0), y.ctypes.data, 1) == UNSUPPORTED
    assert b"type 9" in L.gen9blas_error()
    assert L.gen9blas_symm(9, 0, 0, 8, 8, d(1.0), a.ctypes.data, 8, a.ctypes.data, 8, d(0.0), a.ctypes.data, 8) == UNSUPPORTED
    assert b"type 9" in L.gen9blas_error()


def test_device_operand_past_its_allocation(L):
    """A device operand whose span (rows × ld) runs past the end of its allocation gives INVALID_ARG: it is neither
    used in place (a kernel would read past the buffer) nor taken for host memory (host threads would copy from a
    device address). The gemm call is made only after gen9blas_is_device has classified the span: device memory
    (in range for the buffer's own size) whose requested span lies outside the allocation."""
    n = 64
    nbytes = n * n * 4
    bufs = [L.gen9blas_device_alloc(nbytes) for _ in range(3)]
    try:
        assert all(bufs)
        zeros = np.zeros(n * n, np.float32)
        for p in bufs:
            assert L.gen9blas_memcpy(p, zeros.ctypes.data, nbytes) == OK
        A, B, C = bufs
        big_ld = 1 << 20
        span = ((n - 1) * big_ld + n) * 4
        assert L.gen9blas_is_device(A, nbytes) == 1
        assert L.gen9blas_is_device(A, span) == 0
        assert L.gen9blas_gemm(1, 0, 0, n, n, n, 1.0, A, big_ld, B, n, 0.0, C, n) == INVALID
        assert L.gen9blas_last_status() == INVALID and b"allocation" in L.gen9blas_error()
        assert L.gen9blas_gemm(1, 0, 0, n, n, n, 1.0, A, n, B, n, 0.0, C, n) == OK
    finally:
        for p in bufs:
            if p:
                L.gen9blas_device_free(p)
