"""Pins the oracle (oracle/oracle.c) before it is trusted as the parity checker. CPU only.

Every check below is independent of the code it checks, and chosen so that a plausible mistake in the restatement
(a dropped rounding, a wrong chunk length, a transposed operand, a wrong sign or index) fails at least one of them:
- binary16 rounding against NumPy's correctly rounded float64 → float16 conversion, and all 65536 bit patterns;
- the FP16 chains (GEN9BLAS_H / _HS) against an independent pure-Python restatement on tiny shapes, bit for bit;
- the error profile of the FP16/FP32 chains at n = 4096 against the numbers the reference publishes for its own
  kernels (reference: README.md:73-74; lib/test_basic.py:7): a missing FP32 chunking or an FP32-accumulating H mode
  moves the mean error by an order of magnitude;
- closed forms: exact small-integer products, float64 products under the reference's error metric, transpose flags
  against explicitly transposed operands, beta = 0 ignoring NaN in C;
- reductions to textbook routines: skinny with M = 1 equals GEMV bit for bit, GEN9BLAS_HS equals GEN9BLAS_H when
  K ≤ 32 (one chunk), the FP64 dot against math.fsum of the exact products;
- the golden fixtures committed under tests/golden/ (float64 closed forms of seeded inputs).
"""
import json
import math
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.realpath(__file__)), "golden")


# ---------------- binary16 ----------------
def test_f16_round_matches_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000) * 10.0 ** rng.integers(-9, 6, 200000),
        rng.uniform(-70000, 70000, 20000),
        np.array([65504, 65519.99, 65520, 65536, 1e9, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * (1 + 2 ** -40),
                  3 * 2.0 ** -26, 2.0 ** -14, 2.0 ** -14 * (1 - 2 ** -12), 0.0, -0.0, 1e-30, -1e-300]),
    ])
    # ties: midpoints between consecutive binary16 values round to the even neighbour
    h = np.arange(0x0001, 0x7bff, 7, dtype=np.uint16)
    lo, hi = h.view(np.float16).astype(np.float64), (h + 1).view(np.float16).astype(np.float64)
    x = np.concatenate([x, (lo + hi) / 2, -(lo + hi) / 2])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f16_round(x), ref)
    assert O.f16_round(np.array([np.inf, -np.inf]))[0] == 0x7C00
    assert (O.f16_round(np.array([np.nan])) & 0x7C00) == 0x7C00


def test_f16_all_bit_patterns_round_trip():
    h = np.arange(65536, dtype=np.uint16)
    v = O.f16_value(h)
    finite = ~np.isnan(v)
    assert np.array_equal(v[finite], h.view(np.float16).astype(np.float64)[finite])
    assert np.array_equal(O.f16_round(v[finite]), h[finite])


# ---------------- FP16 chains against an independent restatement ----------------
def _py_chain(a, b, chunk):
    """Independent restatement: acc = fp16(a·b + acc) with one rounding (Python float = double, exact here, then
    NumPy's correctly rounded conversion); chunk: FP32 sum every `chunk` products (GEN9BLAS_HS), None for H."""
    M, K = a.shape
    N = b.shape[1]
    out = np.empty((M, N), np.float16)
    for i in range(M):
        for j in range(N):
            h, f = 0.0, np.float32(0)
            for k in range(K):
                h = float(np.float16(float(a[i, k]) * float(b[k, j]) + h))
                if chunk and (k + 1) % chunk == 0:
                    f = np.float32(f + np.float32(h))
                    h = 0.0
            out[i, j] = np.float16(np.float32(f + np.float32(h))) if chunk else np.float16(h)
    return out


@pytest.mark.parametrize("kind,chunk", [("H", None), ("HS", 32)])
def test_fp16_chains_bit_exact(kind, chunk):
    rng = np.random.default_rng(1)
    for (M, N, K) in [(3, 4, 40), (2, 3, 97), (1, 1, 130)]:
        a = rng.uniform(-1, 1, (M, K)).astype(np.float16)
        b = rng.uniform(-1, 1, (K, N)).astype(np.float16)
        assert np.array_equal(O.gemm(kind, a, b).view(np.uint16), _py_chain(a, b, chunk).view(np.uint16)), (M, N, K)


def test_hs_equals_h_for_one_chunk():
    rng = np.random.default_rng(2)
    for K in (1, 5, 31, 32):
        a = rng.uniform(-1, 1, (7, K)).astype(np.float16)
        b = rng.uniform(-1, 1, (K, 9)).astype(np.float16)
        assert np.array_equal(O.gemm("H", a, b).view(np.uint16), O.gemm("HS", a, b).view(np.uint16)), K
    a = rng.uniform(-1, 1, (7, 33)).astype(np.float16)
    b = rng.uniform(-1, 1, (33, 9)).astype(np.float16)
    assert not np.array_equal(O.gemm("H", a, b), O.gemm("HS", a, b)), "chunking must change the K = 33 result"


def test_error_profile_matches_reference_publication():
    """At n = 4096 with U[-1, 1] inputs the reference publishes mean / max relative errors (normalized by Σ|a·b|):
    H 1.4e-4 / 8.5e-4, HS 1.5e-5 / 5.6e-5, S 1.6e-8 / 7.8e-8 (reference: README.md:73-74; its test describes H max as
    1.7-2.4e-3, lib/test_basic.py:7). The oracle's chains reproduce the means to within a factor of 1.5 on sampled
    rows; an FP32-accumulating H (mean ~1e-5), an unchunked HS (~1.4e-4) or an FP16 S would be far outside."""
    ref = json.load(open(os.path.join(GOLDEN, "reference_error_profile.json")))
    rng = np.random.default_rng(3)
    n, rows = 4096, 3
    for kind, dt in (("H", np.float16), ("HS", np.float16), ("S", np.float32)):
        a = rng.uniform(-1, 1, (rows, n)).astype(dt)
        b = rng.uniform(-1, 1, (n, n)).astype(dt)
        mean, mx = O.gemm_error(O.gemm(kind, a, b), a, b)
        pub = ref[kind]
        assert pub["mean"] / 1.5 <= mean <= pub["mean"] * 1.5, f"{kind}: mean {mean:.2e} vs published {pub['mean']:.1e}"
        assert mx <= pub["max_test"], f"{kind}: max {mx:.2e}"


# ---------------- closed forms ----------------
@pytest.mark.parametrize("kind", ["H", "HS", "S", "D"])
def test_exact_small_integer_products(kind):
    dt = {"H": np.float16, "HS": np.float16, "S": np.float32, "D": np.float64}[kind]
    rng = np.random.default_rng(4)
    a = rng.integers(-4, 5, (13, 21)).astype(dt)
    b = rng.integers(-4, 5, (21, 17)).astype(dt)
    ref = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.int64)
    assert np.array_equal(O.gemm(kind, a, b).astype(np.int64), ref)


@pytest.mark.parametrize("kind", ["H", "HS", "S", "D"])
def test_transpose_flags_and_epilogue(kind):
    dt = {"H": np.float16, "HS": np.float16, "S": np.float32, "D": np.float64}[kind]
    rng = np.random.default_rng(5)
    a = rng.uniform(-1, 1, (9, 40)).astype(dt)
    b = rng.uniform(-1, 1, (40, 11)).astype(dt)
    c0 = rng.uniform(-1, 1, (9, 11)).astype(dt)
    base = O.gemm(kind, a, b, 0.5, -1.25, c0)
    for tA in (False, True):
        for tB in (False, True):
            A = np.ascontiguousarray(a.T) if tA else a
            B = np.ascontiguousarray(b.T) if tB else b
            assert np.array_equal(O.gemm(kind, A, B, 0.5, -1.25, c0, tA=tA, tB=tB), base), (tA, tB)
    bound = {"H": 5e-3, "HS": 5e-3, "S": 1e-6, "D": 1e-13}[kind]
    assert O.gemm_error(base, a, b, 0.5, -1.25, c0)[1] <= bound
    nan_c = np.full((9, 11), np.nan, dt)
    assert np.isfinite(O.gemm(kind, a, b, 1.0, 0.0, nan_c)).all(), "beta = 0 must not read C"


def test_reference_test_shapes_within_bounds():
    """The reference's GEMM test shapes (lib/test_basic.py:65-66) that fit a brute-force CPU run, under its bounds."""
    rng = np.random.default_rng(6)
    for (M, N, K, al, be) in [(1, 1, 1, 1, 0), (17, 33, 15, 1, 0), (100, 70, 300, 2.0, 0), (64, 96, 48, 0.5, 1.0)]:
        for kind, dt, (mb, xb) in (("H", np.float16, (4.9e-4, 5e-3)), ("HS", np.float16, (4.9e-4, 5e-3)),
                                   ("S", np.float32, (1e-6, 1e-5)), ("D", np.float64, (1e-14, 1e-13))):
            a = rng.uniform(-1, 1, (M, K)).astype(dt)
            b = rng.uniform(-1, 1, (K, N)).astype(dt)
            c0 = rng.uniform(-1, 1, (M, N)).astype(dt)
            mean, mx = O.gemm_error(O.gemm(kind, a, b, al, be, c0 if be else None), a, b, al, be, c0)
            assert mean <= mb and mx <= xb, (kind, M, N, K, mean, mx)


# ---------------- skinny, level 1/2 ----------------
def test_skinny_m1_is_gemv_bit_exact():
    rng = np.random.default_rng(7)
    for dt in (np.float16, np.float32):
        a = rng.uniform(-1, 1, (1, 301)).astype(dt)
        w = rng.uniform(-1, 1, (77, 301)).astype(dt)
        s = O.skinny(a, w, 1.5, 0.0, tB=True)[0]
        g = O.gemv(w, a[0], alpha=1.5)
        assert np.array_equal(s, g)
        ref = 1.5 * (a.astype(np.float64) @ w.astype(np.float64).T)[0]
        assert np.max(np.abs(s - ref)) / np.max(np.abs(ref)) <= (4e-3 if dt == np.float16 else 2e-6)


def test_skinny_layouts_and_beta():
    rng = np.random.default_rng(8)
    a = rng.uniform(-1, 1, (5, 64)).astype(np.float32)
    w = rng.uniform(-1, 1, (33, 64)).astype(np.float32)
    c0 = rng.uniform(-1, 1, (5, 33)).astype(np.float32)
    r1 = O.skinny(a, w, 0.75, -1.5, c0, tB=True)
    r2 = O.skinny(np.ascontiguousarray(a.T), np.ascontiguousarray(w.T), 0.75, -1.5, c0, tA=True, tB=False)
    assert np.array_equal(r1, r2)
    ref = 0.75 * a.astype(np.float64) @ w.astype(np.float64).T - 1.5 * c0
    assert np.max(np.abs(r1 - ref)) / np.max(np.abs(ref)) <= 2e-6


def test_axpy_single_rounding():
    rng = np.random.default_rng(9)
    x = rng.uniform(-1, 1, 5000).astype(np.float32)
    y = rng.uniform(-1, 1, 5000).astype(np.float32)
    exact = 0.75 * x.astype(np.float64) + y.astype(np.float64)
    got = O.axpy(0.75, x, y.copy()).astype(np.float64)
    # one rounding of the exact value: within half an ulp
    ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - exact) <= 0.5 * ulp)
    yh = rng.uniform(-1, 1, 300).astype(np.float16)
    xh = rng.uniform(-1, 1, 300).astype(np.float16)
    got = O.axpy(-2.0, xh, yh.copy()).astype(np.float64)
    ref = -2.0 * xh.astype(np.float64) + yh.astype(np.float64)
    assert np.max(np.abs(got - ref) / (2 * np.abs(xh) + np.abs(yh) + 6.2e-5)) <= 2e-3


def test_strided_vectors():
    rng = np.random.default_rng(10)
    base = rng.uniform(-1, 1, 40).astype(np.float64)
    x = base[1:31:3]          # stride 3
    y = base.copy()[::-1][:10]  # stride -1
    yy = y.copy()
    O.axpy(0.5, x, y)
    assert np.allclose(y, yy + 0.5 * x, rtol=0, atol=1e-15)


def test_dot_against_fsum():
    rng = np.random.default_rng(11)
    for n in (1, 5, 1000, 100003):
        x = rng.uniform(-1, 1, n).astype(np.float32)
        y = rng.uniform(-1, 1, n).astype(np.float32)
        exact = math.fsum((x.astype(np.float64) * y.astype(np.float64)).tolist())   # products exact in float64
        scale = float(np.abs(x).astype(np.float64) @ np.abs(y).astype(np.float64))
        assert abs(O.dot(x, y) - exact) <= n * 2.0 ** -52 * scale
        assert abs(O.reduce(1, x) - math.fsum(np.abs(x).astype(np.float64).tolist())) <= n * 2.0 ** -52 * scale + 1e-300
        assert abs(O.reduce(2, x) - math.sqrt(math.fsum((x.astype(np.float64) ** 2).tolist()))) <= 1e-12 * max(1, math.sqrt(n))


def test_gemv_against_float64():
    rng = np.random.default_rng(12)
    for dt, tol in ((np.float32, 1e-6), (np.float16, 2e-3), (np.float64, 1e-13)):
        A = rng.uniform(-1, 1, (37, 53)).astype(dt)
        x = rng.uniform(-1, 1, 53).astype(dt)
        xt = rng.uniform(-1, 1, 37).astype(dt)
        y0 = rng.uniform(-1, 1, 53).astype(dt)
        Ad = A.astype(np.float64)
        yn = O.gemv(A, x, alpha=1.5)
        ref = 1.5 * Ad @ x.astype(np.float64)
        assert np.max(np.abs(yn - ref) / np.maximum(1.5 * np.abs(Ad) @ np.abs(x.astype(np.float64)), 6.2e-5)) <= tol
        yt = O.gemv(A, xt, alpha=0.5, beta=-2.0, y=y0.copy(), trans=True)
        ref = 0.5 * Ad.T @ xt.astype(np.float64) - 2.0 * y0.astype(np.float64)
        scale = 0.5 * np.abs(Ad.T) @ np.abs(xt.astype(np.float64)) + 2 * np.abs(y0.astype(np.float64))
        assert np.max(np.abs(yt - ref) / np.maximum(scale, 6.2e-5)) <= tol


# ---------------- golden fixtures ----------------
def test_golden_fixtures():
    """Seeded inputs and their float64 closed-form products (tests/golden/make_golden.py): the oracle's restatement of
    each type meets the reference bound against them, and the fixture inputs regenerate from their seeds."""
    d = np.load(os.path.join(GOLDEN, "gemm_small.npz"))
    for kind, dt, bound in (("H", np.float16, 5e-3), ("HS", np.float16, 5e-3), ("S", np.float32, 1e-6),
                            ("D", np.float64, 1e-13)):
        a, b, c0 = d[f"{kind}_A"], d[f"{kind}_B"], d[f"{kind}_C0"]
        ref, scale = d[f"{kind}_ref"], d[f"{kind}_scale"]
        al, be = float(d["alpha"]), float(d["beta"])
        got = O.gemm(kind, a, b, al, be, c0).astype(np.float64)
        assert np.max(np.abs(got - ref) / scale) <= bound, kind
        assert np.array_equal(a, np.random.default_rng(int(d["seed"])).uniform(-1, 1, a.shape).astype(dt))
    v = np.load(os.path.join(GOLDEN, "level12_small.npz"))
    assert abs(O.dot(v["x"], v["y"]) - float(v["dot"])) <= 1e-12 * float(v["dot_scale"])
    assert np.max(np.abs(O.gemv(v["A"], v["x"][:v["A"].shape[1]]) - v["gemv"]) / v["gemv_scale"]) <= 1e-6


# ---------------- level 2 storage (band, packed, triangles) ----------------
def _band_from(D, KL, KU, width=None):
    """Row-major band array of D built diagonal by diagonal (independent of oracle.band_dense's row loop)."""
    M, N = D.shape
    P = np.zeros((M, width or KL + KU + 1))
    for d in range(-KL, KU + 1):            # diagonal c − r = d sits in column KL + d
        r = np.arange(max(0, -d), min(M, N - d))
        P[r, KL + d] = D[r, r + d]
    return P


@pytest.mark.parametrize("M,N,KL,KU", [(1, 1, 0, 0), (50, 40, 3, 5), (300, 310, 0, 7), (257, 200, 30, 0),
                                       (100, 100, 99, 99), (7, 30, 2, 40)])
def test_band_storage_against_openblas(M, N, KL, KU):
    """oracle.band_dense against an independent diagonal-wise packer (round trip, exact) and against OpenBLAS dgbmv
    (the reference's CPU path) reading the same row-major array as the column-major band of Aᵀ (kl = KU, ku = KL),
    which is how a CBLAS row-major call maps onto Fortran storage."""
    from scipy.linalg import blas
    rng = np.random.default_rng(M * 1000 + N)
    i, j = np.indices((M, N))
    D = rng.uniform(-1, 1, (M, N)) * ((j - i >= -KL) & (j - i <= KU))
    P = _band_from(D, KL, KU, width=KL + KU + 3)          # lda > KL+KU+1: padding columns never read
    P[:, KL + KU + 1:] = np.nan
    assert np.array_equal(O.band_dense(P, M, N, KL, KU), D)
    if N < KL + KU + 1:
        return   # SciPy's dgbmv wrapper requires m >= kl + ku + 1 (its own check; BLAS needs only lda >= kl + ku + 1)
    x, xt = rng.uniform(-1, 1, N), rng.uniform(-1, 1, M)
    Pf = np.asfortranarray(P.T)
    assert np.allclose(blas.dgbmv(N, M, KU, KL, 1.0, Pf, x, trans=1), D @ x, rtol=0, atol=1e-13)
    assert np.allclose(blas.dgbmv(N, M, KU, KL, 1.0, Pf, xt, trans=0), D.T @ xt, rtol=0, atol=1e-13)


@pytest.mark.parametrize("n", [1, 2, 60, 130])
@pytest.mark.parametrize("uplo", ["U", "L"])
def test_packed_and_symmetric_band_against_openblas(n, uplo):
    """oracle.packed_dense against NumPy's row-major triangle indices (round trip, exact); symmetric products of the
    packed and band storages against OpenBLAS dspmv / dsbmv, and triangular ones against dtpmv / dtbmv, on the same
    arrays (row-major upper = column-major lower of the transpose); oracle.solve against dtpsv and the residual."""
    from scipy.linalg import blas
    rng = np.random.default_rng(n + (uplo == "U"))
    D = rng.uniform(-1, 1, (n, n))
    T = O.triangle(D, uplo)
    idx = np.triu_indices(n) if uplo == "U" else np.tril_indices(n)
    Ap = D[idx]
    assert np.array_equal(O.packed_dense(Ap, n, uplo), T)
    x = rng.uniform(-1, 1, n)
    fl = int(uplo == "U")                         # Fortran triangle of the transpose
    assert np.allclose(blas.dspmv(n, 1.0, Ap, x, lower=fl), O.symmetric(D, uplo) @ x, rtol=0, atol=1e-13)
    for trans in (0, 1):
        for unit in (0, 1):
            Op = O.triangle(D, uplo, unit)
            Op = Op.T if trans else Op
            assert np.allclose(blas.dtpmv(n, Ap, x, lower=fl, trans=1 - trans, diag=unit), Op @ x, rtol=0, atol=1e-13)
            S = Op / n                               # well conditioned: small off-diagonal entries
            np.fill_diagonal(S, 2 + np.abs(np.diag(Op)) if not unit else 1.0)
            b = S @ x
            z = O.solve(S, b)
            assert np.allclose(S @ z, b, rtol=0, atol=1e-12) and np.allclose(z, x, rtol=0, atol=1e-12)
    K = max(0, min(n - 1, 5))
    i, j = np.indices((n, n))
    Tb = T * (np.abs(j - i) <= K)
    P = _band_from(Tb, 0 if uplo == "U" else K, K if uplo == "U" else 0)
    assert np.array_equal(O.band_dense(P, n, n, 0 if uplo == "U" else K, K if uplo == "U" else 0), Tb)
    S = Tb + Tb.T - np.diag(np.diag(Tb))
    assert np.allclose(blas.dsbmv(K, 1.0, np.asfortranarray(P.T), x, lower=fl), S @ x, rtol=0, atol=1e-13)
    assert np.allclose(blas.dtbmv(K, np.asfortranarray(P.T), x, lower=fl, trans=1), Tb @ x, rtol=0, atol=1e-13)


def test_solve_order_and_planted_mistakes():
    """oracle.solve handles both substitution orders, and a planted transpose or dropped diagonal fails the
    residual check that the GPU tests rely on."""
    rng = np.random.default_rng(5)
    n = 40
    L = np.tril(rng.uniform(-1, 1, (n, n))) / n
    np.fill_diagonal(L, 1 + rng.uniform(0, 1, n))
    b = rng.uniform(-1, 1, n)
    for Op in (L, L.T):
        z = O.solve(Op, b)
        assert np.allclose(Op @ z, b, rtol=0, atol=1e-13)
        wrong = O.solve(Op.T, b)
        assert not np.allclose(Op @ wrong, b, rtol=0, atol=1e-6)
    U = np.triu(L.T)
    np.fill_diagonal(U, 1.0)
    assert not np.allclose(U @ O.solve(L.T, b), b, rtol=0, atol=1e-6)   # unit diagonal is not the stored one
