"""Level-2 parity on the GPU: SYMV, TRMV, TRSV, SYR, SYR2 on full storage and GBMV, SBMV, TBMV, TBSV, SPMV, TPMV,
TPSV, SPR, SPR2 on band and packed storage, through the C ABI (gen9blas.py) against the oracle's float64 restatement
of each storage format (oracle.band_dense / packed_dense / triangle / symmetric / solve).

Cases follow the reference's level-2 test (reference: lib/test_level12.py:98-146, 180-259): orders 1, 5, 63, 64, 65,
200, 1000; both triangles, both transposes, unit and stored diagonals, an A.T view (the other triangle in memory),
strided and negative-stride vectors; band shapes (M, N, KL, KU) and (n, K) as there. Bounds as there: error relative
to |alpha|·|op(A)|·|x| + |beta·y|, FP32 1e-6, FP16 2e-3, FP64 1e-13; solutions relative to max|z|: FP32 1e-5,
FP16 3e-3, FP64 1e-12. Device-resident cases at n = 4096 exercise the multi-block solves and both load paths of the
product kernel (16-byte rows and an odd row stride); orders below 1280 take the substituting solve, from 1280 up the
solve on inverted diagonal blocks.
"""
import itertools

import numpy as np
import pytest

from l12_util import assert_close, band_store, dominant_triangle, in_band, packed_store, strided

pytestmark = pytest.mark.gpu

TOL = {np.float32: 1e-6, np.float16: 2e-3, np.float64: 1e-13}
SOLVE_TOL = {np.float32: 1e-5, np.float16: 3e-3, np.float64: 1e-12}
DTYPES = [np.float32, np.float16, np.float64]
rng = np.random.default_rng(12)


def f64(a):
    return np.asarray(a, np.float64)


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("n", [1, 5, 63, 64, 65, 200, 1000])
def test_full_storage(g9, orc, dt, n):
    tol = TOL[dt]
    A = rng.uniform(-1, 1, (n, n)).astype(dt)
    Ad = f64(A)
    for uplo in "LU":
        S = orc.symmetric(Ad, uplo)
        x, y0 = strided(rng, n, dt, -2, 1), strided(rng, n, dt, 3)
        ref, scale = orc.mv(S, x, 0.5, 2.0, y0)
        g9.symv(A, x, uplo=uplo, alpha=0.5, beta=2.0, y=y0)
        assert_close(f"symv {uplo} n={n}", y0, ref, scale, tol)
        ref, scale = orc.mv(orc.symmetric(Ad.T, uplo), x)
        assert_close(f"symv A.T {uplo} n={n}", g9.symv(A.T, x, uplo=uplo), ref, scale, tol)
        for trans in (False, True):
            for diag in (False, True):
                label = f"{uplo} trans={int(trans)} diag={int(diag)} n={n}"
                Op = orc.triangle(Ad, uplo, diag)
                Op = Op.T if trans else Op
                xx = strided(rng, n, dt, 2)
                ref, scale = orc.mv(Op, xx)
                g9.trmv(A, xx, uplo=uplo, trans=trans, diag=diag)
                assert_close("trmv " + label, xx, ref, scale, tol)
                # solve: a diagonally dominant triangle (well conditioned in every type)
                Ab = dominant_triangle(A, diag)
                Ob = orc.triangle(f64(Ab), uplo, diag)
                Ob = Ob.T if trans else Ob
                b = strided(rng, n, dt, -1)
                ref = orc.solve(Ob, f64(b))
                g9.trsv(Ab, b, uplo=uplo, trans=trans, diag=diag)
                assert_close("trsv " + label, b, ref, np.max(np.abs(ref)), SOLVE_TOL[dt])
        xs, ys = strided(rng, n, dt, 1, 2), strided(rng, n, dt, -3, 0)
        X, Y = f64(xs), f64(ys)
        mask = np.tril(np.ones((n, n), bool)) if uplo == "L" else np.triu(np.ones((n, n), bool))
        A1 = A.copy()
        g9.syr(-0.5, xs, A1, uplo=uplo)
        assert_close(f"syr {uplo} n={n}", A1, np.where(mask, Ad - 0.5 * np.outer(X, X), Ad),
              np.abs(Ad) + 0.5 * np.outer(np.abs(X), np.abs(X)), tol)
        A2 = A.copy()
        g9.syr2(0.25, xs, ys, A2, uplo=uplo)
        assert_close(f"syr2 {uplo} n={n}", A2, np.where(mask, Ad + 0.25 * (np.outer(X, Y) + np.outer(Y, X)), Ad),
              np.abs(Ad) + 0.25 * (np.outer(np.abs(X), np.abs(Y)) + np.outer(np.abs(Y), np.abs(X))), tol)


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("n", [1000, 1100])
def test_full_storage_unreferenced_nan(g9, orc, dt, n):
    """SYMV, TRMV, SYR and SYR2 on full storage with NaN in the triangle they must not reference. Rows that meet a
    column group's diagonal block read whole 16-byte chunks, the unreferenced part included, and mask those elements
    when used (masking by selection keeps the NaN out, a multiplication by zero would not); the rank updates write
    back only the referenced elements. n = 1000 and 1100 take whole column
    groups and a partial last one (16-byte rows in FP32 and FP64; FP16 at n = 1100 takes single elements)."""
    tol = TOL[dt]
    A = rng.uniform(-1, 1, (n, n)).astype(dt)
    Ad = f64(A)
    for uplo in "LU":
        other = np.triu(np.ones((n, n), bool), 1) if uplo == "L" else np.tril(np.ones((n, n), bool), -1)
        An = A.copy()
        An[other] = np.nan
        x = strided(rng, n, dt, 1)
        ref, scale = orc.mv(orc.symmetric(Ad, uplo), x)
        assert_close(f"symv NaN {uplo} n={n}", g9.symv(An, x, uplo=uplo), ref, scale, tol)
        for trans in (False, True):
            xx = strided(rng, n, dt, 2)
            Op = orc.triangle(Ad, uplo, False)
            ref, scale = orc.mv(Op.T if trans else Op, xx)
            g9.trmv(An, xx, uplo=uplo, trans=trans)
            assert_close(f"trmv NaN {uplo} trans={int(trans)} n={n}", xx, ref, scale, tol)
        # rank updates read whole chunks too, but write only the referenced triangle: the NaN stay where they were
        xs, ys = strided(rng, n, dt, 1, 2), strided(rng, n, dt, -3, 0)
        X, Y = f64(xs), f64(ys)
        ref_mask = ~other
        for name, upd, ref, scale in (
                ("syr", lambda M: g9.syr(-0.5, xs, M, uplo=uplo), Ad - 0.5 * np.outer(X, X),
                 np.abs(Ad) + 0.5 * np.outer(np.abs(X), np.abs(X))),
                ("syr2", lambda M: g9.syr2(0.25, xs, ys, M, uplo=uplo), Ad + 0.25 * (np.outer(X, Y) + np.outer(Y, X)),
                 np.abs(Ad) + 0.25 * (np.outer(np.abs(X), np.abs(Y)) + np.outer(np.abs(Y), np.abs(X))))):
            A1 = An.copy()
            upd(A1)
            assert_close(f"{name} NaN {uplo} n={n}", A1[ref_mask], ref[ref_mask], scale[ref_mask], tol)
            assert np.isnan(A1[other]).all(), f"{name} {uplo} n={n}: the unreferenced triangle was written"


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("n", [1280, 1300, 4095, 4096, 4100])
def test_trsv_blocked_inverse(g9, orc, dt, n):
    """TRSV from order 1280 up runs on inverted diagonal blocks (x_q = inv(D_q)·r_q − E_q·x_(q-1), inverses in FP64),
    of 256 rows below order 4096 and of 512 rows from there: n = 1280 is the smallest such order (5 whole blocks),
    n = 1300 ends on a partial block of 20 rows (the last in solve order, at the start of A for a backward solve),
    n = 4095 is the largest order on 256-row blocks (16, the last one row short), n = 4096 the smallest on 512-row
    blocks (8 whole ones), n = 4100 ends on one of 4 rows after them. Both triangles, both transposes, unit and stored
    diagonals, a negative-stride x, and the unreferenced triangle (and a unit diagonal) filled with huge values, which
    must not be read into the result."""
    A = rng.uniform(-1, 1, (n, n)).astype(dt)
    Ad = f64(A)
    big = {np.float16: 6e4, np.float32: 1e30, np.float64: 1e300}[dt]
    for uplo in "LU":
        other = np.triu(np.ones((n, n), bool), 1) if uplo == "L" else np.tril(np.ones((n, n), bool), -1)
        for trans in (False, True):
            for diag in (False, True):
                Ab = dominant_triangle(A, diag)
                Ob = orc.triangle(f64(Ab), uplo, diag)
                Ob = Ob.T if trans else Ob
                Ag = Ab.copy()
                Ag[other] = big
                if diag:
                    np.fill_diagonal(Ag, big)
                b = strided(rng, n, dt, -1)
                ref = orc.solve(Ob, f64(b))
                g9.trsv(Ag, b, uplo=uplo, trans=trans, diag=diag)
                assert_close(f"trsv {uplo} trans={int(trans)} diag={int(diag)} n={n}", b, ref, np.max(np.abs(ref)),
                      SOLVE_TOL[dt])


# Normwise backward error ||b − op(T)·x||∞ / (||op(T)||∞·||x||∞) a solve must stay within, per type: γ_n = n·u of
# the work precision (FP32 for FP16 and FP32, FP64 for FP64), plus, for FP16, the rounding of x to FP16.
def _backward_bound(dt, n):
    if dt == np.float64:
        return n * 2.0 ** -53
    return n * 2.0 ** -24 + (2.0 ** -11 if dt == np.float16 else 0.0)


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("n", [1000, 1280, 1300, 4500])
def test_trsv_not_dominant(g9, orc, dt, n):
    """Triangles that are not diagonally dominant: off-diagonal entries uniform(−1, 1)/√n (row sums of |T| near
    √n/2, far above the diagonal), unit or stored diagonal of magnitude 1..2. The solution stays bounded (its
    variance grows by at most (1 + 1/n)^n ≈ e), but the solve is no longer well conditioned entry by entry, so the
    check is the normwise backward error. n = 1000 takes the substitution, 1280 and 1300 the inverted 256-row blocks,
    4500 the 512-row blocks (8 whole ones and one of 404 rows), whose off-diagonal couplings are work-precision
    products: all meet the same bound."""
    r = np.random.default_rng(n + 3 * DTYPES.index(dt))
    A = (r.uniform(-1, 1, (n, n)) / np.sqrt(n))
    d = r.uniform(-1, 1, n)
    np.fill_diagonal(A, np.where(d < 0, -1.0, 1.0) * (1 + np.abs(d)))
    A = A.astype(dt)
    worst = 0.0
    for uplo in "LU":
        for trans in (False, True):
            for diag in (False, True):
                Op = orc.triangle(f64(A), uplo, diag)
                Op = Op.T if trans else Op
                b = r.uniform(-1, 1, n).astype(dt)
                B = np.array(b, np.float64)   # a copy: the solve overwrites b
                g9.trsv(A, b, uplo=uplo, trans=trans, diag=diag)
                x = f64(b)
                assert np.isfinite(x).all()
                res = np.max(np.abs(B - Op @ x))
                err = res / (np.max(np.abs(Op).sum(axis=1)) * np.max(np.abs(x)))
                worst = max(worst, err)
                assert err <= _backward_bound(dt, n), (
                    f"trsv {uplo} trans={int(trans)} diag={int(diag)} n={n}: backward error {err:.2e}")
    print(f"trsv not dominant {np.dtype(dt).name} n={n}: worst normwise backward error {worst:.2e}")


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("M,N,KL,KU", [(1, 1, 0, 0), (50, 40, 3, 5), (300, 310, 0, 7), (257, 200, 30, 0),
                                       (100, 100, 99, 99), (1200, 1100, 2, 300)])
def test_gbmv(g9, orc, dt, M, N, KL, KU):
    tol = TOL[dt]
    D = f64(rng.uniform(-1, 1, (M, N)).astype(dt)) * in_band(M, N, KL, KU)
    P = band_store(D, KL, KU).astype(dt)
    assert np.array_equal(orc.band_dense(P, M, N, KL, KU), D)
    for tr in (False, True):
        x, y0 = strided(rng, M if tr else N, dt, -2), strided(rng, N if tr else M, dt, 3)
        ref, scale = orc.mv(D.T if tr else D, x, 0.5, 2.0, y0)
        g9.gbmv(P, x, M, N, KL, KU, alpha=0.5, beta=2.0, y=y0, trans=tr)
        assert_close(f"gbmv {M}x{N} KL={KL} KU={KU} tr={tr}", y0, ref, scale, tol)


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("n,K", [(1, 0), (60, 4), (300, 17), (130, 129), (700, 70)])
def test_band_packed(g9, orc, dt, n, K):
    tol = TOL[dt]
    Dp = f64(rng.uniform(-1, 1, (n, n)).astype(dt))
    for uplo in "UL":
        g = uplo == "U"
        KL, KU = (0, K) if g else (K, 0)
        T = Dp * in_band(n, n, KL, KU)
        P = band_store(T, KL, KU).astype(dt)
        x = strided(rng, n, dt, 2)
        ref, scale = orc.mv(orc.symmetric(T, uplo), x, 1.5)
        assert_close(f"sbmv n={n} K={K} {uplo}", g9.sbmv(P, x, K, uplo=uplo, alpha=1.5), ref, scale, tol)
        Tp = orc.triangle(Dp, uplo)
        Ap = packed_store(Tp, uplo).astype(dt)
        assert np.array_equal(orc.packed_dense(Ap, n, uplo), Tp)
        y0 = strided(rng, n, dt, -1)
        ref, scale = orc.mv(orc.symmetric(Tp, uplo), x, 0.5, -1.0, y0)
        g9.spmv(Ap, x, uplo=uplo, alpha=0.5, beta=-1.0, y=y0)
        assert_close(f"spmv n={n} {uplo}", y0, ref, scale, tol)
        for tr, dg in itertools.product((False, True), repeat=2):
            label = f"{uplo} n={n} K={K} trans={tr} unit={dg}"
            Ob, Op = orc.triangle(T, uplo, dg), orc.triangle(Tp, uplo, dg)
            Ob, Op = (Ob.T, Op.T) if tr else (Ob, Op)
            x = strided(rng, n, dt, -3)
            ref, scale = orc.mv(Ob, x)
            g9.tbmv(P, x, K, uplo=uplo, trans=tr, diag=dg)
            assert_close("tbmv " + label, x, ref, scale, tol)
            x = strided(rng, n, dt, 1)
            ref, scale = orc.mv(Op, x)
            g9.tpmv(Ap, x, uplo=uplo, trans=tr, diag=dg)
            assert_close("tpmv " + label, x, ref, scale, tol)
            # solves: well conditioned (small off-diagonal entries, diagonal 1..2)
            Ts = T / max(K, 1) / 4
            np.fill_diagonal(Ts, 1 + np.abs(np.diag(T)))
            Ps = band_store(Ts, KL, KU).astype(dt)
            Os = orc.triangle(orc.band_dense(Ps, n, n, KL, KU), uplo, dg)
            b = strided(rng, n, dt, 2)
            ref = orc.solve(Os.T if tr else Os, f64(b))
            g9.tbsv(Ps, b, K, uplo=uplo, trans=tr, diag=dg)
            assert_close("tbsv " + label, b, ref, np.max(np.abs(ref)), SOLVE_TOL[dt])
            Tq = Tp / n
            np.fill_diagonal(Tq, 1 + np.abs(np.diag(Tp)))
            Aq = packed_store(Tq, uplo).astype(dt)
            Oq = orc.triangle(orc.packed_dense(Aq, n, uplo), uplo, dg)
            b = strided(rng, n, dt, -1)
            ref = orc.solve(Oq.T if tr else Oq, f64(b))
            g9.tpsv(Aq, b, uplo=uplo, trans=tr, diag=dg)
            assert_close("tpsv " + label, b, ref, np.max(np.abs(ref)), SOLVE_TOL[dt])
        xs, ys = strided(rng, n, dt, 1), strided(rng, n, dt, -2)
        X, Y = f64(xs), f64(ys)
        Ap1 = Ap.copy()
        g9.spr(-0.5, xs, Ap1, uplo=uplo)
        assert_close(f"spr n={n} {uplo}", Ap1, packed_store(orc.triangle(Tp - 0.5 * np.outer(X, X), uplo), uplo),
              packed_store(np.abs(Tp) + 0.5 * np.outer(np.abs(X), np.abs(X)), uplo), tol)
        Ap2 = Ap.copy()
        g9.spr2(0.25, xs, ys, Ap2, uplo=uplo)
        assert_close(f"spr2 n={n} {uplo}", Ap2, packed_store(orc.triangle(Tp + 0.25 * (np.outer(X, Y) + np.outer(Y, X)), uplo), uplo),
              packed_store(np.abs(Tp) + 0.25 * (np.outer(np.abs(X), np.abs(Y)) + np.outer(np.abs(Y), np.abs(X))), uplo), tol)


def test_trsv_blocks_read_in_place(g9, orc, torch_dev):
    """The forward solve on A itself (uplo L, not transposed, FP32 / FP64, whole blocks of 256 or 512 rows) reads the
    diagonal blocks, their lower-left quadrants and the couplings where they lie in A: 16 seeded cases on device
    views with a row stride of n + 0..8, unit and stored diagonals, and huge values in the unreferenced triangle (and
    on a unit diagonal) that must not reach the result; every fourth case another triangle or transpose (gathered)."""
    torch = torch_dev
    r = np.random.default_rng(2024)
    big = {np.float32: 1e30, np.float64: 1e300}
    for c in range(16):
        dt = (np.float32, np.float64)[c % 2]
        n = int(r.choice([1280, 1536, 2048, 4096, 4608]))
        pad = int(r.integers(0, 9))
        other_case = c % 4 == 3
        uplo = "LU"[int(r.integers(0, 2))] if other_case else "L"
        trans = bool(r.integers(0, 2)) if other_case else False
        diag = bool(r.integers(0, 2))
        A = dominant_triangle(r.uniform(-1, 1, (n, n)), diag).astype(dt)
        Ab = A.copy()
        Ab[np.triu_indices(n, 1) if uplo == "L" else np.tril_indices(n, -1)] = big[dt]
        if diag:
            np.fill_diagonal(Ab, big[dt])
        base = r.uniform(-1, 1, (n, n + pad)).astype(dt)
        base[:, :n] = Ab
        Ob = orc.triangle(f64(A), uplo, diag)
        Ob = Ob.T if trans else Ob
        b = r.uniform(-1, 1, n).astype(dt)
        ref = orc.solve(Ob, f64(b))
        Ad = torch.from_numpy(base).cuda()[:, :n]
        bd = torch.from_numpy(b).cuda()
        g9.trsv(Ad, bd, uplo=uplo, trans=trans, diag=diag)
        assert_close(f"trsv case {c} {np.dtype(dt).name} n={n} ld={n + pad} {uplo} trans={int(trans)} diag={int(diag)}",
                     bd.cpu().numpy(), ref, np.max(np.abs(ref)), SOLVE_TOL[dt])


@pytest.mark.parametrize("dt", [np.float32, np.float64])
@pytest.mark.parametrize("odd_ld", [False, True])
def test_level2_device_n4096(g9, orc, torch_dev, dt, odd_ld):
    """n = 4096 on device tensors: 32 diagonal blocks per solve; odd_ld passes a view with row stride 4097, which takes
    the element-wise load path of the product kernel instead of the 16-byte one."""
    torch = torch_dev
    n = 4096
    base = rng.uniform(-1, 1, (n, n + 1 if odd_ld else n)).astype(dt)
    A = base[:, :n]
    Ad = f64(A)
    Adev = torch.from_numpy(base).cuda()[:, :n]
    assert Adev.stride()[0] == (n + 1 if odd_ld else n)
    x = rng.uniform(-1, 1, n).astype(dt)
    xd = torch.from_numpy(x).cuda()
    for uplo in "LU":
        ref, scale = orc.mv(orc.symmetric(Ad, uplo), x, 1.25)
        assert_close(f"symv {uplo}", g9.symv(Adev, xd, uplo=uplo, alpha=1.25).cpu().numpy(), ref, scale, TOL[dt])
        for trans in (False, True):
            Op = orc.triangle(Ad, uplo)
            Op = Op.T if trans else Op
            v = xd.clone()
            g9.trmv(Adev, v, uplo=uplo, trans=trans)
            ref, scale = orc.mv(Op, x)
            assert_close(f"trmv {uplo} trans={trans}", v.cpu().numpy(), ref, scale, TOL[dt])
        Ab = base.copy()
        Ab[:, :n] = dominant_triangle(A, False)
        Abd = torch.from_numpy(Ab).cuda()[:, :n]
        for trans in (False, True):
            Ob = orc.triangle(f64(Ab[:, :n]), uplo)
            Ob = Ob.T if trans else Ob
            v = xd.clone()
            g9.trsv(Abd, v, uplo=uplo, trans=trans)
            ref = orc.solve(Ob, f64(x))
            assert_close(f"trsv {uplo} trans={trans}", v.cpu().numpy(), ref, np.max(np.abs(ref)), SOLVE_TOL[dt])
        Ap = packed_store(orc.triangle(Ad, uplo), uplo).astype(dt)
        ref, scale = orc.mv(orc.symmetric(Ad, uplo), x)
        assert_close(f"spmv {uplo}", g9.spmv(torch.from_numpy(Ap).cuda(), xd, uplo=uplo).cpu().numpy(), ref, scale, TOL[dt])


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_packed_products_unaligned_device(g9, orc, torch_dev, dt):
    """Packed-storage products read 16 bytes per lane from rows that are only element-aligned: here the packed matrix
    starts one element into its device buffer (4 or 8 bytes off a 16-byte boundary), n = 1500 so that whole column
    groups take the unchecked path; SPMV and TPMV in both triangles against the oracle."""
    torch = torch_dev
    n = 1500
    Dp = f64(rng.uniform(-1, 1, (n, n)).astype(dt))
    x = strided(rng, n, dt, 1)
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    for uplo in "LU":
        Tp = orc.triangle(Dp, uplo)
        Ap = packed_store(Tp, uplo).astype(dt)
        buf = torch.zeros(Ap.size + 1, dtype=torch.float32 if dt == np.float32 else torch.float64, device="cuda")
        buf[1:] = torch.from_numpy(Ap).cuda()
        Apd = buf[1:]
        assert Apd.data_ptr() % 16 != 0
        ref, scale = orc.mv(orc.symmetric(Tp, uplo), x)
        assert_close(f"spmv unaligned {uplo}", g9.spmv(Apd, xd, uplo=uplo).cpu().numpy(), ref, scale, TOL[dt])
        for tr in (False, True):
            Op = Tp.T if tr else Tp
            v = xd.clone()
            g9.tpmv(Apd, v, uplo=uplo, trans=tr)
            ref, scale = orc.mv(Op, x)
            assert_close(f"tpmv unaligned {uplo} trans={tr}", v.cpu().numpy(), ref, scale, TOL[dt])


def test_level2_errors(g9):
    """Status codes as in the reference (reference: lib/src/level12.c:267-519): lda < n and band widths are
    INVALID_ARG, a zero increment is INVALID_ARG, an unknown type UNSUPPORTED, an empty problem 0 with nothing
    read."""
    L = g9._lib
    a = np.zeros((4, 4), np.float32)
    x = np.zeros(4, np.float32)
    p = a.ctypes.data
    px = x.ctypes.data
    assert L.gen9blas_symv(1, 0, 4, 1.0, p, 3, px, 1, 0.0, px, 1) == -3
    assert L.gen9blas_trsv(1, 0, 0, 0, 4, p, 4, px, 0) == -3
    assert L.gen9blas_gbmv(1, 0, 4, 4, -1, 0, 1.0, p, 4, px, 1, 0.0, px, 1) == -3
    assert L.gen9blas_gbmv(1, 0, 4, 4, 2, 2, 1.0, p, 4, px, 1, 0.0, px, 1) == -3
    assert L.gen9blas_tbsv(1, 0, 0, 0, 4, 4, p, 4, px, 1) == -3
    assert L.gen9blas_spmv(7, 0, 4, 1.0, p, px, 1, 0.0, px, 1) == -2
    assert L.gen9blas_tpsv(1, 0, 0, 0, 0, None, None, 1) == 0
    assert L.gen9blas_syr2(1, 0, -1, 1.0, None, 1, None, 1, None, 1) == 0


def _l2_cases(seed, count):
    """Seeded random level-2 calls on full, band and packed storage: operation, type, order (small, near a multiple
    of 64, mid-sized, or 1280-1399 for the solves on inverted blocks), band width, triangle, transpose, unit diagonal
    and x's stride."""
    r = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        op = str(r.choice(["symv", "trmv", "trsv", "sbmv", "tbmv", "tbsv", "spmv", "tpmv", "tpsv"]))
        c = int(r.integers(0, 4))
        n = (int(r.integers(1, 80)) if c == 0 else max(1, 64 * int(r.integers(1, 16)) + int(r.integers(-3, 4)))
             if c == 1 else int(r.integers(80, 1000)) if c == 2 else int(r.integers(1280, 1400)))
        out.append((op, int(r.integers(0, 3)), n, int(r.integers(0, 40)), str(r.choice(["L", "U"])),
                    bool(r.integers(0, 2)), bool(r.integers(0, 2)), int(r.choice([1, 2, -1, -3]))))
    return out


@pytest.mark.parametrize("case", _l2_cases(2030, 120), ids=lambda c: "-".join(str(v) for v in c))
def test_level2_random(g9, orc, case):
    """120 seeded random products and solves on full, band and packed storage in every type, against the oracle's
    float64 restatement of each storage format, with the bounds above (solves on well-conditioned triangles)."""
    op, ti, n, K, uplo, tr, dg, sx = case
    dt = DTYPES[ti]
    tol = TOL[dt]
    r = np.random.default_rng(n * 31 + K * 7 + ti)

    def vec(step):
        base = r.uniform(-1, 1, n * abs(step) + 2).astype(dt)
        v = base[1:1 + n * abs(step):abs(step)]
        return v[::-1] if step < 0 else v
    tag = f"{op} {np.dtype(dt).name} n={n} K={K} {uplo} tr={tr} diag={dg} incx={sx}"
    D = f64(r.uniform(-1, 1, (n, n)).astype(dt))
    K = min(K, max(n - 1, 0))
    KL, KU = (0, K) if uplo == "U" else (K, 0)
    solve = op.endswith("sv")
    if solve:   # well conditioned: small off-diagonal entries, diagonal 1..2
        D = D / max(n if op != "tbsv" else K, 1) / 4
        np.fill_diagonal(D, 1 + np.abs(np.diag(D)) * 4)
        D = f64(D.astype(dt))
    x = vec(sx)
    X = f64(x)
    if op in ("symv", "trmv", "trsv"):
        A = D.astype(dt)
        T = orc.triangle(D, uplo, dg)
        if op == "symv":
            ref, scale = orc.mv(orc.symmetric(D, uplo), x, 1.5)
            assert_close(tag, g9.symv(A, x, uplo=uplo, alpha=1.5), ref, scale, tol)
        elif op == "trmv":
            ref, scale = orc.mv(T.T if tr else T, x)
            g9.trmv(A, x, uplo=uplo, trans=tr, diag=dg)
            assert_close(tag, x, ref, scale, tol)
        else:
            ref = orc.solve(T.T if tr else T, X)
            g9.trsv(A, x, uplo=uplo, trans=tr, diag=dg)
            assert_close(tag, x, ref, np.max(np.abs(ref)), SOLVE_TOL[dt])
    elif op in ("sbmv", "tbmv", "tbsv"):
        Tb = D * in_band(n, n, KL, KU)
        P = band_store(Tb, KL, KU).astype(dt)
        T = orc.triangle(orc.band_dense(P, n, n, KL, KU), uplo, dg)
        if op == "sbmv":
            ref, scale = orc.mv(orc.symmetric(Tb, uplo), x, -0.5)
            assert_close(tag, g9.sbmv(P, x, K, uplo=uplo, alpha=-0.5), ref, scale, tol)
        elif op == "tbmv":
            ref, scale = orc.mv(T.T if tr else T, x)
            g9.tbmv(P, x, K, uplo=uplo, trans=tr, diag=dg)
            assert_close(tag, x, ref, scale, tol)
        else:
            ref = orc.solve(T.T if tr else T, X)
            g9.tbsv(P, x, K, uplo=uplo, trans=tr, diag=dg)
            assert_close(tag, x, ref, np.max(np.abs(ref)), SOLVE_TOL[dt])
    else:
        Tp = orc.triangle(D, uplo)
        Ap = packed_store(Tp, uplo).astype(dt)
        T = orc.triangle(orc.packed_dense(Ap, n, uplo), uplo, dg)
        if op == "spmv":
            ref, scale = orc.mv(orc.symmetric(Tp, uplo), x, 0.25)
            assert_close(tag, g9.spmv(Ap, x, uplo=uplo, alpha=0.25), ref, scale, tol)
        elif op == "tpmv":
            ref, scale = orc.mv(T.T if tr else T, x)
            g9.tpmv(Ap, x, uplo=uplo, trans=tr, diag=dg)
            assert_close(tag, x, ref, scale, tol)
        else:
            ref = orc.solve(T.T if tr else T, X)
            g9.tpsv(Ap, x, uplo=uplo, trans=tr, diag=dg)
            assert_close(tag, x, ref, np.max(np.abs(ref)), SOLVE_TOL[dt])
