"""CPU checks of the level-1/2 test helpers (tests/l12_util.py) against the oracle's storage maps, so the GPU tests
that build operands with them test the library, not the helpers."""
import numpy as np
import pytest

import oracle
from l12_util import assert_close, band_store, dominant_triangle, in_band, packed_store, strided


@pytest.mark.parametrize("M,N,KL,KU", [(1, 1, 0, 0), (50, 40, 3, 5), (300, 310, 0, 7), (257, 200, 30, 0),
                                       (100, 100, 99, 99), (7, 12, 2, 9)])
def test_band_store_round_trip(M, N, KL, KU):
    rng = np.random.default_rng(M + N)
    D = rng.uniform(-1, 1, (M, N)) * in_band(M, N, KL, KU)
    P = band_store(D, KL, KU)
    assert P.shape == (M, KL + KU + 1)
    assert np.array_equal(oracle.band_dense(P, M, N, KL, KU), D)
    # the mask against its definition, element by element
    for r in range(min(M, 20)):
        for c in range(min(N, 20)):
            assert in_band(M, N, KL, KU)[r, c] == (-KL <= c - r <= KU)


@pytest.mark.parametrize("n", [1, 2, 5, 64, 131])
@pytest.mark.parametrize("uplo", "LU")
def test_packed_store_round_trip(n, uplo):
    T = oracle.triangle(np.random.default_rng(n).uniform(-1, 1, (n, n)), uplo)
    Ap = packed_store(T, uplo)
    assert Ap.size == n * (n + 1) // 2
    assert np.array_equal(oracle.packed_dense(Ap, n, uplo), T)


@pytest.mark.parametrize("inc,lead", [(1, 0), (1, 1), (3, 5), (-2, 0), (-1, 2)])
def test_strided_positions(inc, lead):
    """Element i of the view lies at byte lead·es + i·inc·es of its array (inc > 0), or at (n − 1 − i)·|inc|·es past
    the lead (inc < 0); writes go through to the array."""
    n = 17
    v = strided(np.random.default_rng(1), n, np.float32, inc, lead)
    base = v.base
    while base.base is not None:
        base = base.base
    start = base.__array_interface__["data"][0]
    for i in range(n):
        k = i if inc > 0 else n - 1 - i
        addr = v[i:].__array_interface__["data"][0]
        assert addr - start == (lead + k * abs(inc)) * 4
    v[3] = 7.0
    assert 7.0 in np.frombuffer(base, np.float32)


@pytest.mark.parametrize("unit", [False, True])
def test_dominant_triangle(unit):
    A = np.random.default_rng(2).uniform(-1, 1, (300, 300)).astype(np.float32)
    W = dominant_triangle(A, unit).astype(np.float64)
    off = np.abs(W).sum(axis=1) - np.abs(np.diag(W))
    assert (off < 1).all()
    if not unit:
        assert (np.abs(np.diag(W)) >= 1).all() and (np.sign(np.diag(W)) == np.sign(np.diag(A))).all()


def test_assert_close_floor_and_failure():
    # FP16 results: scales below the smallest normal FP16 count as that value
    assert_close("tiny", np.array([2.0 ** -25], np.float16), [0.0], [0.0], 2e-3 * 1.1)
    with pytest.raises(AssertionError):
        assert_close("wrong", np.array([1.0, 2.0]), [1.0, 2.1], [1.0, 2.0], 1e-6)
    assert_close("exact", np.array([1.0, 2.0]), [1.0, 2.0], 1.0, 0.0)
