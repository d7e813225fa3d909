"""Host-side logic of gen9blas.py, without a GPU: how operands are described to the C ABI (pointer, ld, transpose
flag, increment), which layouts are passed in place and which are copied or rejected, and the pinned pool's size
classes and block lifetime. The rules follow the reference module's contract (lib/gen9blas.py:304-328 for matrices
and vectors, :96-115 for gen9blas.empty); the GPU tests check that the library computes the right thing with them."""
import ctypes

import numpy as np
import pytest

import gen9blas as g

F32, F16 = np.dtype(np.float32), np.dtype(np.float16)


def test_matrix_layouts_in_place():
    A = np.zeros((6, 8), np.float32)
    m = g._matrix(A, F32)
    assert (m.ptr, m.shape, m.ld, m.trans) == (A.ctypes.data, (6, 8), 8, 0)
    m = g._matrix(A.T, F32)                       # stored row-major 6×8, the caller sees 8×6
    assert (m.ptr, m.shape, m.stored, m.ld, m.trans) == (A.ctypes.data, (8, 6), (6, 8), 8, 1)
    m = g._matrix(A[1:, 2:5], F32)                # column slice keeps the row stride
    assert (m.ptr, m.shape, m.ld, m.trans) == (A[1:, 2:].ctypes.data, (5, 3), 8, 0)
    m = g._matrix(A[::2], F32)                    # every other row: ld doubles
    assert (m.shape, m.ld, m.ptr, m.trans) == ((3, 8), 16, A.ctypes.data, 0)


def test_matrix_copies_inputs_and_rejects_outputs():
    A = np.arange(48, dtype=np.float32).reshape(6, 8)
    m = g._matrix(A[:, ::2], F32)                 # column stride 2: not expressible, copied
    assert m.keep is not A and m.ld == 4 and m.trans == 0
    assert np.array_equal(np.asarray(m.keep), A[:, ::2])
    m = g._matrix(A.astype(np.float64), F32)      # another type: converted
    assert np.asarray(m.keep).dtype == F32
    with pytest.raises(TypeError):
        g._matrix(A.T, F32, out=True)             # results must have contiguous rows
    with pytest.raises(TypeError):
        g._matrix(A, F16, out=True)               # ... and the compute type
    with pytest.raises(ValueError):
        g._matrix(np.zeros(4, np.float32), F32)


def test_vector_strides():
    x = np.arange(10, dtype=np.float32)
    v = g._vector(x[::-2], F32)                   # 9, 7, 5, 3, 1: BLAS wants the lowest address, x[1]
    assert (v.n, v.inc, v.ptr) == (5, -2, x.ctypes.data + 4)
    v = g._vector(x[2::3], F32)
    assert (v.n, v.inc, v.ptr) == (3, 3, x.ctypes.data + 8)
    b = np.broadcast_to(np.float32(1), (4,))      # stride 0: copied for an input, rejected as an output
    assert g._vector(b, F32).inc == 1
    with pytest.raises(TypeError):
        g._vector(b, F32, out=True)
    raw = np.zeros(20, np.uint8)
    odd = raw[1:17].view(np.float32)              # 4 floats at an odd byte offset, stride fine
    assert g._vector(odd, F32).inc == 1
    with pytest.raises(ValueError):
        g._equal_lengths(g._vector(x, F32), g._vector(x[:3], F32))


def test_compute_type_rules():
    assert g._compute_type(np.zeros(2, np.float16)) == F16
    assert g._compute_type(np.zeros(2, np.float64)) == np.float64
    assert g._compute_type(np.zeros(2, np.int32)) == F32      # anything else computes in float32
    with pytest.raises(TypeError):
        g._strict_type(np.zeros(2, np.int32))
    assert g._kind(F16, accurate=True) == g.GEN9BLAS_HS and g._kind(F32, accurate=True) == g.GEN9BLAS_S


def test_output_checks():
    C = np.zeros((2, 3, 4), np.float32)
    out = g._out_matrix(C, (2, 3, 4), F32, C)
    assert out.given and out.ld == 4 and out.beta(0.5) == 0.5
    with pytest.raises(ValueError):
        g._out_matrix(C[:, :, :2], (2, 3, 2), F32, C)          # a batch must be C-contiguous
    with pytest.raises(ValueError):
        g._out_matrix(C[0], (3, 5), F32, C)                    # wrong shape
    big = np.zeros((5, 9), np.float32)
    out = g._out_matrix(big[1:4, 2:6], (3, 4), F32, big)       # a strided C keeps its row stride
    assert out.ld == 9 and out.ptr == big[1:, 2:].ctypes.data
    with pytest.raises(TypeError):
        g._out_vector([0.0, 1.0], 2, F32, None)                # a list cannot receive a result


def test_pool_size_classes():
    sc = g._PinnedPool.size_class
    assert [sc(n) for n in (0, 1, 4096, 4097, 1 << 20)] == [4096, 4096, 4096, 8192, 1 << 20]
    assert sc((1 << 20) + 1) == 2 << 20 and sc(5 << 20) == 5 << 20
    for n in range(0, 1 << 22, 12345):
        assert sc(n) >= n


def test_pinned_block_returns_when_last_view_dies(monkeypatch):
    buf = (ctypes.c_char * 64)()
    given = []
    monkeypatch.setattr(g._pool, "give", lambda p, s: given.append((p, s)))
    arr = np.asarray(g._PinnedBlock(ctypes.addressof(buf), 64, 32)).view(np.float32).reshape(2, 4)
    assert arr.ctypes.data == ctypes.addressof(buf)
    row = arr[1]
    del arr
    assert given == []                            # a view is still alive
    del row
    assert given == [(ctypes.addressof(buf), 64)]


def test_every_declared_function_is_exported():
    for item in g._SIGNATURES.split():
        assert hasattr(g._lib, "gen9blas_" + item.split("=")[0]), item
