"""Operand builders and the error check shared by the level-1 and level-2 GPU tests.

The error measure is the reference's for level 1-2 (reference: lib/test_level12.py:3-8, 27-31): the largest
element-wise |got − ref| / scale, where scale is the formula's magnitude (|a·x| + |y| for axpy, |alpha|·|op(A)|·|x| +
|beta·y| for a product). Results stored in FP16 take the smallest normal FP16 number as the least scale, since
rounding a tiny value to FP16 has an absolute, not a relative, error.
"""
import numpy as np
from numpy.lib.stride_tricks import as_strided

FP16_TINY = float(np.finfo(np.float16).tiny)   # 2**-14


def assert_close(name, got, ref, scale, tol):
    """Fails with the measured error when max |got − ref| / scale exceeds tol (tol = 0: exact)."""
    got = np.asarray(got)
    floor = FP16_TINY if got.dtype == np.float16 else 1e-300
    diff = np.abs(got.astype(np.float64) - np.asarray(ref, np.float64))
    err = float(np.max(diff / np.maximum(np.asarray(scale, np.float64), floor), initial=0.0))
    assert err <= tol, f"{name}: error {err:.2e} above {tol:.0e}"


def strided(rng, n, dt, inc=1, lead=0):
    """A vector of n uniform[-1, 1) values seen through BLAS storage: element i sits at lead + i·inc (inc > 0) of a
    larger host array, or at lead + (n − 1 − i)·|inc| (inc < 0, a view running backwards), the other elements of the
    array being filled too. Returned as a writable NumPy view, so calls that take it see the stride and offset."""
    step = abs(inc)
    store = rng.uniform(-1, 1, lead + step * max(n - 1, 0) + 1 + 2).astype(dt)
    view = as_strided(store[lead:], shape=(n,), strides=(step * store.itemsize,))
    return view[::-1] if inc < 0 else view


def band_store(D, KL, KU):
    """Row-major band array of D (M×N): row r holds the diagonals −KL..KU of D's row r, diagonal d = c − r at column
    KL + d; positions outside D stay zero (the storage of reference lib/gen9blas.h:147-150). Vectorized over the
    diagonals."""
    M, N = D.shape
    P = np.zeros((M, KL + KU + 1), D.dtype)
    rows = np.arange(M)
    for d in range(-KL, KU + 1):
        cols = rows + d
        ok = (cols >= 0) & (cols < N)
        P[rows[ok], KL + d] = D[rows[ok], cols[ok]]
    return P


def in_band(M, N, KL, KU):
    """Boolean M×N mask of the elements with −KL ≤ c − r ≤ KU."""
    offset = np.arange(N)[None, :] - np.arange(M)[:, None]
    return (offset >= -KL) & (offset <= KU)


def packed_store(T, uplo):
    """Packed vector of T's `uplo` triangle, row by row (the layout oracle.packed_dense reads back)."""
    n = T.shape[0]
    return T[np.triu_indices(n)] if uplo == "U" else T[np.tril_indices(n)]


def dominant_triangle(A, unit):
    """A copy of square A whose triangular solves are well conditioned in either triangle: off-diagonal entries
    scaled by 1/n, so each row's off-diagonal sum stays below 1, and a stored diagonal of magnitude 1 + |a_ii|
    (sign kept). With unit = True the stored diagonal is never read; it is scaled like the rest."""
    n = A.shape[0]
    W = np.asarray(A, np.float64) / max(n, 1)
    if not unit:
        d = np.diag(np.asarray(A, np.float64))
        np.fill_diagonal(W, np.where(d < 0, -1.0, 1.0) * (1 + np.abs(d)))
    return W.astype(A.dtype)
