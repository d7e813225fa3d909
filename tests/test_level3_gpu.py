"""Level 3 beyond GEMM on the GPU: SYMM, SYRK, SYR2K, TRMM, TRSM against the float64 closed forms.

Follows the reference's level-3 test (reference: lib/test_level3.py:38-137): the same sides, triangles, transposes and
unit diagonals, error e = |result − ref| / (|alpha|·(|A|·|B|) + |beta·C|) with the reference's mean / max bounds
(FP16 both modes 4.9e-4 / 5e-3, FP32 1e-6 / 1e-5, FP64 1e-14 / 1e-13), the other triangle of C unchanged by SYRK and
SYR2K, and TRSM's solution error max|X − X_ref| / max|X_ref| on well-conditioned triangles (FP64 1e-12, FP32 1e-4, FP16
5e-3). Added: sizes from 512 (the banded products and several TRSM blocks) and device-resident operands.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TYPES = [("H", np.float16, False, (4.9e-4, 5e-3)), ("HS", np.float16, True, (4.9e-4, 5e-3)),
         ("S", np.float32, False, (1e-6, 1e-5)), ("D", np.float64, False, (1e-14, 1e-13))]
IDS = [t[0] for t in TYPES]


def _check(W, ref, scale, tol, mask=None, tag=""):
    e = np.abs(np.asarray(W, np.float64) - ref) / np.maximum(scale, 1e-30)
    if mask is not None:
        e = e[mask]
    assert e.mean() <= tol[0] and e.max() <= tol[1], f"{tag}: mean {e.mean():.2e} max {e.max():.2e}"


def f64(x):
    return np.asarray(x, np.float64)


@pytest.mark.parametrize("kind,dt,acc,tol", TYPES, ids=IDS)
@pytest.mark.parametrize("M,N", [(70, 45), (520, 300)])
def test_symm(g9, kind, dt, acc, tol, M, N):
    rng = np.random.default_rng(1)
    for side in "LR":
        for uplo in "LU":
            n = M if side == "L" else N
            S = rng.uniform(-1, 1, (n, n)).astype(dt)
            Ss = np.tril(f64(S)) + np.tril(f64(S), -1).T if uplo == "L" else np.triu(f64(S)) + np.triu(f64(S), 1).T
            B, C0 = rng.uniform(-1, 1, (M, N)).astype(dt), rng.uniform(-1, 1, (M, N)).astype(dt)
            W = g9.symm(S, B, side, uplo, 2.0, -1.0, C0.copy(), accurate=acc)
            P = Ss @ f64(B) if side == "L" else f64(B) @ Ss
            Pa = np.abs(Ss) @ np.abs(f64(B)) if side == "L" else np.abs(f64(B)) @ np.abs(Ss)
            _check(W, 2.0 * P - f64(C0), 2.0 * Pa + np.abs(f64(C0)), tol, tag=f"symm {side}{uplo} {M}x{N}")


@pytest.mark.parametrize("kind,dt,acc,tol", TYPES, ids=IDS)
@pytest.mark.parametrize("N,K", [(60, 90), (600, 200)])
def test_syrk_syr2k(g9, kind, dt, acc, tol, N, K):
    rng = np.random.default_rng(2)
    for uplo in "LU":
        mask = np.tril(np.ones((N, N), bool)) if uplo == "L" else np.triu(np.ones((N, N), bool))
        for tr in (False, True):
            A = rng.uniform(-1, 1, (K, N) if tr else (N, K)).astype(dt)
            B = rng.uniform(-1, 1, (K, N) if tr else (N, K)).astype(dt)
            C0 = rng.uniform(-1, 1, (N, N)).astype(dt)
            oA, oB = (f64(A).T, f64(B).T) if tr else (f64(A), f64(B))
            W = g9.syrk(A, uplo, tr, 0.7, 0.3, C0.copy(), accurate=acc)
            _check(W, 0.7 * oA @ oA.T + 0.3 * f64(C0), 0.7 * np.abs(oA) @ np.abs(oA).T + 0.3 * np.abs(f64(C0)), tol,
                   mask, f"syrk {uplo} t={tr}")
            assert np.array_equal(W[~mask], C0[~mask]), "syrk changed the other triangle"
            W = g9.syr2k(A, B, uplo, tr, 0.7, 0.3, C0.copy(), accurate=acc)
            _check(W, 0.7 * (oA @ oB.T + oB @ oA.T) + 0.3 * f64(C0),
                   0.7 * (np.abs(oA) @ np.abs(oB).T + np.abs(oB) @ np.abs(oA).T) + 0.3 * np.abs(f64(C0)), tol, mask,
                   f"syr2k {uplo} t={tr}")
            assert np.array_equal(W[~mask], C0[~mask]), "syr2k changed the other triangle"
            # beta = 0: C is not read (NaN in the triangle does not propagate), the other triangle stays
            Cn = C0.copy()
            Cn[mask] = np.nan
            W = g9.syrk(A, uplo, tr, 1.0, 0.0, Cn, accurate=acc)
            assert np.isfinite(W[mask]).all() and np.array_equal(W[~mask], C0[~mask])


@pytest.mark.parametrize("kind,dt,acc,tol", TYPES, ids=IDS)
@pytest.mark.parametrize("M,N", [(50, 70), (530, 260)])
def test_trmm(g9, kind, dt, acc, tol, M, N):
    rng = np.random.default_rng(3)
    for side in "LR":
        for uplo in "LU":
            for ta in (False, True):
                for dg in (False, True):
                    n = M if side == "L" else N
                    A, B = rng.uniform(-1, 1, (n, n)).astype(dt), rng.uniform(-1, 1, (M, N)).astype(dt)
                    T = np.tril(f64(A)) if uplo == "L" else np.triu(f64(A))
                    if dg:
                        np.fill_diagonal(T, 1.0)
                    T = T.T if ta else T
                    W = g9.trmm(A, B, side, uplo, ta, dg, 1.5, accurate=acc)
                    P = T @ f64(B) if side == "L" else f64(B) @ T
                    Pa = np.abs(T) @ np.abs(f64(B)) if side == "L" else np.abs(f64(B)) @ np.abs(T)
                    _check(W, 1.5 * P, 1.5 * Pa, tol, tag=f"trmm {side}{uplo} tA={ta} diag={dg}")


TRSM_TYPES = [("D", np.float64, False, 1e-12), ("S", np.float32, False, 1e-4), ("H", np.float16, False, 5e-3),
              ("HS", np.float16, True, 5e-3)]


@pytest.mark.parametrize("kind,dt,acc,tol", TRSM_TYPES, ids=[t[0] for t in TRSM_TYPES])
def test_trsm(g9, kind, dt, acc, tol):
    rng = np.random.default_rng(4)
    for side in "LR":
        for uplo in "LU":
            for ta in (False, True):
                for dg in (False, True):
                    for (M, N) in [(40, 30), (300, 200), (70, 600), (400, 400)]:   # n = 400: one partial leaf, its
                        # 256-row inverse composed with a last 16 rows, then with a last 144
                        n = M if side == "L" else N
                        A = rng.uniform(-1, 1, (n, n)).astype(np.float32)
                        A[np.diag_indices(n)] = n if not dg else 0.5
                        if dg:   # the diagonal is not read; conditioning from a scaled off-diagonal part
                            A *= 1.0 / n
                            A[np.diag_indices(n)] = 123.0
                        B = rng.uniform(-1, 1, (M, N)).astype(np.float32)
                        A, B = A.astype(dt), B.astype(dt)
                        T = np.tril(f64(A)) if uplo == "L" else np.triu(f64(A))
                        if dg:
                            np.fill_diagonal(T, 1.0)
                        T = T.T if ta else T
                        Xr = (np.linalg.solve(T, 2.0 * f64(B)) if side == "L" else np.linalg.solve(T.T, 2.0 * f64(B).T).T)
                        X = f64(g9.trsm(A, B, side, uplo, ta, dg, 2.0, accurate=acc))
                        e = np.abs(X - Xr).max() / np.abs(Xr).max()
                        assert e <= tol, f"trsm {kind} {side}{uplo} tA={ta} diag={dg} {M}x{N}: {e:.1e}"


@pytest.mark.parametrize("kind,dt,acc,tol", TRSM_TYPES, ids=[t[0] for t in TRSM_TYPES])
@pytest.mark.parametrize("n", [1300, 1450, 2048])
def test_trsm_left_lower_in_place(g9, torch_dev, kind, dt, acc, tol, n):
    """The left, lower, non-transposed solve reads A and B where they lie: B is updated in place as the right-hand
    side, alpha is applied by the first product touching each block of rows, the FP64 block inversion masks A's other
    triangle and (unit) diagonal itself. A's upper triangle (and a unit diagonal) hold huge values that must not be
    read; B is a column slice of a wider array (row stride above N) whose other columns must survive; alpha 0.5 and
    0 (X = 0), on host and device operands. FP32 / FP64 leaves of 512 rows: n = 1300 ends in a partial leaf of 276 rows
    (its inverse composed from 256 and 20 rows), n = 1450 in one of 426 (a 128 + 42-row block composed first), n = 2048
    has 4 whole leaves; FP16 leaves have 128 rows."""
    torch = torch_dev
    rng = np.random.default_rng(n)
    big = {np.float16: 6e4, np.float32: 1e30, np.float64: 1e300}[dt]
    m = 96
    for dg in (False, True):
        A = (rng.uniform(-1, 1, (n, n)) / n).astype(np.float32)
        A[np.diag_indices(n)] = 1.0 + rng.uniform(0, 1, n)
        T = np.tril(f64(A.astype(dt)))
        if dg:
            np.fill_diagonal(T, 1.0)
        Ag = A.astype(dt)
        Ag[np.triu_indices(n, 1)] = big
        if dg:
            Ag[np.diag_indices(n)] = big
        for off, pad in ((3, 7), (4, 8)):
            # B = columns off .. off + m of a wider array (row stride m + pad): off 3 misaligns B's rows, off 4 with
            # pad 8 keeps FP32 / FP64 rows 16-byte aligned (the solution is then stored 16 bytes per lane)
            wide = rng.uniform(-1, 1, (n, m + pad)).astype(dt)
            code = {"H": 0, "S": 1, "HS": 2, "D": 3}[kind]
            es = np.dtype(dt).itemsize
            d, p = ctypes.c_double, ctypes.c_void_p
            for alpha in (0.5, 0.0):
                for where in ("host", "device"):
                    if where == "host":
                        W = wide.copy()
                        rc = g9._lib.gen9blas_trsm(code, 0, 0, 0, int(dg), n, m, d(alpha), p(Ag.ctypes.data), n,
                                                   p(W.ctypes.data + off * es), m + pad)
                    else:
                        Wd = torch.from_numpy(wide.copy()).cuda()
                        Ad = torch.from_numpy(Ag).cuda()
                        rc = g9._lib.gen9blas_trsm(code, 0, 0, 0, int(dg), n, m, d(alpha), p(Ad.data_ptr()), n,
                                                   p(Wd.data_ptr() + off * es), m + pad)
                        torch.cuda.synchronize()
                        W = Wd.cpu().numpy()
                    assert rc == 0, g9._lib.gen9blas_error()
                    tag = f"trsm LLN {kind} n={n} diag={dg} alpha={alpha} {where} B at column {off}"
                    assert np.array_equal(W[:, :off], wide[:, :off]) and \
                        np.array_equal(W[:, off + m:], wide[:, off + m:]), tag + ": columns outside B changed"
                    X = f64(W[:, off:off + m])
                    if alpha == 0.0:
                        assert np.array_equal(X, np.zeros_like(X)), tag
                    else:
                        Xr = np.linalg.solve(T, alpha * f64(wide[:, off:off + m]))
                        e = np.abs(X - Xr).max() / np.abs(Xr).max()
                        assert e <= tol, f"{tag}: {e:.1e}"


def test_level3_device_operands(g9, torch_dev):
    """SYMM, SYRK, TRMM and TRSM on device tensors through the C ABI: results in place, zero-copy bits set."""
    torch = torch_dev
    rng = np.random.default_rng(5)
    L = g9._lib
    d, p = ctypes.c_double, ctypes.c_void_p
    n, m = 256, 192
    A = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    A[np.diag_indices(n)] = n
    B = rng.uniform(-1, 1, (n, m)).astype(np.float32)
    Ad, Bd = torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda()
    Cd = torch.zeros((n, m), dtype=torch.float32, device="cuda")
    assert L.gen9blas_symm(1, 0, 0, n, m, d(1.0), p(Ad.data_ptr()), n, p(Bd.data_ptr()), m, d(0.0), p(Cd.data_ptr()), m) == 0
    torch.cuda.synchronize()
    Ss = np.tril(f64(A)) + np.tril(f64(A), -1).T
    _check(Cd.cpu().numpy(), Ss @ f64(B), np.abs(Ss) @ np.abs(f64(B)), (1e-6, 1e-5), tag="symm device")
    Sd = torch.zeros((n, n), dtype=torch.float32, device="cuda")
    assert L.gen9blas_syrk(1, 0, 0, n, m, d(1.0), p(Bd.data_ptr()), m, d(0.0), p(Sd.data_ptr()), n) == 0
    torch.cuda.synchronize()
    mask = np.tril(np.ones((n, n), bool))
    _check(Sd.cpu().numpy(), f64(B) @ f64(B).T, np.abs(f64(B)) @ np.abs(f64(B)).T, (1e-6, 1e-5), mask, "syrk device")
    assert g9.last_zero_copy() == 5
    Td = Bd.clone()
    assert L.gen9blas_trmm(1, 0, 1, 0, 0, n, m, d(1.0), p(Ad.data_ptr()), n, p(Td.data_ptr()), m) == 0
    torch.cuda.synchronize()
    U = np.triu(f64(A))
    _check(Td.cpu().numpy(), U @ f64(B), np.abs(U) @ np.abs(f64(B)), (1e-6, 1e-5), tag="trmm device")
    Xd = Bd.clone()
    assert L.gen9blas_trsm(1, 0, 1, 0, 0, n, m, d(1.0), p(Ad.data_ptr()), n, p(Xd.data_ptr()), m) == 0
    torch.cuda.synchronize()
    Xr = np.linalg.solve(U, f64(B))
    assert np.abs(Xd.cpu().numpy() - Xr).max() / np.abs(Xr).max() <= 1e-4


@pytest.mark.parametrize("N,K", [(1536, 96), (3968, 64)])
def test_syrk_syr2k_fp32_whole_tiles(g9, N, K):
    """FP32 SYRK / SYR2K large enough for the whole-tile kernel's triangle mode (N = 1536: 300 tiles of 64×64; N = 3968:
    496 tiles of 128×128, which fill their last round better than 1953 of 64×64), both triangles and transposes, on small integers (every result exact, so a misplaced tile,
    a diagonal-tile element written outside the triangle or a lost k-step shows up bit-exactly), alpha 1.5, beta 0.5 on
    an integer C; the other triangle unchanged."""
    rng = np.random.default_rng(6)
    for uplo in "LU":
        mask = np.tril(np.ones((N, N), bool)) if uplo == "L" else np.triu(np.ones((N, N), bool))
        for tr in (False, True):
            A = rng.integers(-2, 3, (K, N) if tr else (N, K)).astype(np.float32)
            B = rng.integers(-2, 3, (K, N) if tr else (N, K)).astype(np.float32)
            C0 = rng.integers(-4, 5, (N, N)).astype(np.float32)
            oA, oB = (f64(A).T, f64(B).T) if tr else (f64(A), f64(B))
            W = g9.syrk(A, uplo, tr, 1.5, 0.5, C0.copy())
            assert np.array_equal(f64(W)[mask], (1.5 * oA @ oA.T + 0.5 * f64(C0))[mask]), f"syrk {uplo} t={tr}"
            assert np.array_equal(W[~mask], C0[~mask]), "syrk changed the other triangle"
            W = g9.syr2k(A, B, uplo, tr, 1.5, 0.5, C0.copy())
            assert np.array_equal(f64(W)[mask], (1.5 * (oA @ oB.T + oB @ oA.T) + 0.5 * f64(C0))[mask]), f"syr2k {uplo} t={tr}"
            assert np.array_equal(W[~mask], C0[~mask]), "syr2k changed the other triangle"


@pytest.mark.parametrize("M,N,full", [(1024, 1024, True), (2048, 4096, False)])
def test_trmm_fp32_whole_tiles(g9, M, N, full):
    """FP32 TRMM large enough for the whole-tile kernel's k-limited mode (1024²: 64×64 tiles, every side, triangle,
    transpose and diagonal; 2048×4096: 128×256 tiles, left side), on small integers: every result exact."""
    rng = np.random.default_rng(7)
    for side in ("LR" if full else "L"):
        for uplo in "LU":
            for ta in ((False, True) if full else (False,)):
                for dg in ((False, True) if full else (False,)):
                    n = M if side == "L" else N
                    A = rng.integers(-2, 3, (n, n)).astype(np.float32)
                    B = rng.integers(-2, 3, (M, N)).astype(np.float32)
                    T = np.tril(f64(A)) if uplo == "L" else np.triu(f64(A))
                    if dg:
                        np.fill_diagonal(T, 1.0)
                    T = T.T if ta else T
                    W = g9.trmm(A, B, side, uplo, ta, dg, 1.5)
                    P = T @ f64(B) if side == "L" else f64(B) @ T
                    assert np.array_equal(f64(W), 1.5 * P), f"trmm {side}{uplo} tA={ta} diag={dg}"


@pytest.mark.parametrize("kind,M,N", [("S", 512, 4096), ("S", 500, 4000), ("D", 512, 4096)])
def test_trmm_paired_k_limited_tiles(g9, kind, M, N):
    """k-limited products with more tiles than CUs but at most two per CU, all resident at once, take the paired
    dispatch order (the second half of the longest-first order reversed): FP32 512×4096 on the whole-tile kernel's
    64×64 tiles (512), 500×4000 on the general kernel's (504), FP64 512×4096 on its 64×64 tiles (512); both sides
    and triangles (the four k-limit modes), small integers, so every result is exact and a tile computed twice or
    not at all shows up."""
    dt = np.float32 if kind == "S" else np.float64
    rng = np.random.default_rng(8)
    for side in "LR":
        for uplo in "LU":
            m, n_ = (M, N) if side == "L" else (N, M)
            n = m if side == "L" else n_
            A = rng.integers(-2, 3, (n, n)).astype(dt)
            B = rng.integers(-2, 3, (m, n_)).astype(dt)
            T = np.tril(f64(A)) if uplo == "L" else np.triu(f64(A))
            W = g9.trmm(A, B, side, uplo, False, False, 1.5)
            P = T @ f64(B) if side == "L" else f64(B) @ T
            assert np.array_equal(f64(W), 1.5 * P), f"trmm {kind} {side}{uplo} {m}x{n_}"


@pytest.mark.parametrize("kind,dt,tol", [("S", np.float32, 1e-4), ("D", np.float64, 1e-12)])
def test_trsm_paired_leaf_products(g9, kind, dt, tol):
    """TRSM of order 1024 with 4096 right-hand sides: its two 512-row leaves are applied by k-limited products of
    512×4096 (512 tiles of 64×64, the paired dispatch order), for every side and triangle against float64."""
    rng = np.random.default_rng(9)
    n, m = 1024, 4096
    for uplo in "LU":
        A = (rng.uniform(-1, 1, (n, n)) / n).astype(dt)
        A[np.diag_indices(n)] = 1.0 + rng.uniform(0, 1, n)
        B = rng.uniform(-1, 1, (n, m)).astype(dt)
        T = np.tril(f64(A)) if uplo == "L" else np.triu(f64(A))
        X = f64(g9.trsm(A, B, "L", uplo, False, False, 0.5))
        Xr = np.linalg.solve(T, 0.5 * f64(B))
        e = np.abs(X - Xr).max() / np.abs(Xr).max()
        assert e <= tol, f"trsm {kind} L{uplo} {n}x{m}: {e:.1e}"


def _l3_cases(seed, count):
    """Seeded random level-3 calls: operation, type, side / triangle / transpose / unit diagonal, and dimensions that
    are small (1-79), multiples of 64 (the whole-tile classes of the GEMMs underneath), within 3 of one, or 80-599."""
    r = np.random.default_rng(seed)

    def dim():
        c = int(r.integers(0, 4))
        if c == 0:
            return int(r.integers(1, 80))
        if c == 1:
            return 64 * int(r.integers(1, 10))
        if c == 2:
            return max(1, 64 * int(r.integers(1, 10)) + int(r.integers(-3, 4)))
        return int(r.integers(80, 600))
    out = []
    for _ in range(count):
        out.append((str(r.choice(["symm", "syrk", "syr2k", "trmm", "trsm"])), int(r.integers(0, 4)), dim(), dim(),
                    str(r.choice(["L", "R"])), str(r.choice(["L", "U"])), bool(r.integers(0, 2)), bool(r.integers(0, 2))))
    return out


@pytest.mark.parametrize("case", _l3_cases(2027, 120), ids=lambda c: "-".join(str(v) for v in c))
def test_level3_random(g9, case):
    """120 seeded random SYMM / SYRK / SYR2K / TRMM / TRSM calls in every type, against the float64 closed forms with
    the bounds of the tests above (TRSM: solution error on a well-conditioned triangle)."""
    op, ti, M, N, side, uplo, ta, dg = case
    kind, dt, acc, tol = TYPES[ti]
    rng = np.random.default_rng(M * 1009 + N * 17 + ti)
    tag = f"{op} {kind} {M}x{N} side={side} uplo={uplo} t={ta} diag={dg}"
    n = M if side == "L" else N
    if op == "symm":
        S = rng.uniform(-1, 1, (n, n)).astype(dt)
        Ss = np.tril(f64(S)) + np.tril(f64(S), -1).T if uplo == "L" else np.triu(f64(S)) + np.triu(f64(S), 1).T
        B, C0 = rng.uniform(-1, 1, (M, N)).astype(dt), rng.uniform(-1, 1, (M, N)).astype(dt)
        W = g9.symm(S, B, side, uplo, -0.5, 1.5, C0.copy(), accurate=acc)
        P = Ss @ f64(B) if side == "L" else f64(B) @ Ss
        Pa = np.abs(Ss) @ np.abs(f64(B)) if side == "L" else np.abs(f64(B)) @ np.abs(Ss)
        _check(W, -0.5 * P + 1.5 * f64(C0), 0.5 * Pa + 1.5 * np.abs(f64(C0)), tol, tag=tag)
    elif op in ("syrk", "syr2k"):
        Nn, K = M, N
        mask = np.tril(np.ones((Nn, Nn), bool)) if uplo == "L" else np.triu(np.ones((Nn, Nn), bool))
        A = rng.uniform(-1, 1, (K, Nn) if ta else (Nn, K)).astype(dt)
        B = rng.uniform(-1, 1, (K, Nn) if ta else (Nn, K)).astype(dt)
        C0 = rng.uniform(-1, 1, (Nn, Nn)).astype(dt)
        oA, oB = (f64(A).T, f64(B).T) if ta else (f64(A), f64(B))
        if op == "syrk":
            W = g9.syrk(A, uplo, ta, 0.7, -0.3, C0.copy(), accurate=acc)
            ref, scale = 0.7 * oA @ oA.T - 0.3 * f64(C0), 0.7 * np.abs(oA) @ np.abs(oA).T + 0.3 * np.abs(f64(C0))
        else:
            W = g9.syr2k(A, B, uplo, ta, 0.7, -0.3, C0.copy(), accurate=acc)
            ref = 0.7 * (oA @ oB.T + oB @ oA.T) - 0.3 * f64(C0)
            scale = 0.7 * (np.abs(oA) @ np.abs(oB).T + np.abs(oB) @ np.abs(oA).T) + 0.3 * np.abs(f64(C0))
        _check(W, ref, scale, tol, mask, tag)
        assert np.array_equal(W[~mask], C0[~mask]), f"{tag}: the other triangle changed"
    elif op == "trmm":
        A, B = rng.uniform(-1, 1, (n, n)).astype(dt), rng.uniform(-1, 1, (M, N)).astype(dt)
        T = np.tril(f64(A)) if uplo == "L" else np.triu(f64(A))
        if dg:
            np.fill_diagonal(T, 1.0)
        T = T.T if ta else T
        W = g9.trmm(A, B, side, uplo, ta, dg, -2.0, accurate=acc)
        P = T @ f64(B) if side == "L" else f64(B) @ T
        Pa = np.abs(T) @ np.abs(f64(B)) if side == "L" else np.abs(f64(B)) @ np.abs(T)
        _check(W, -2.0 * P, 2.0 * Pa, tol, tag=tag)
    else:
        stol = {"D": 1e-12, "S": 1e-4, "H": 5e-3, "HS": 5e-3}[kind]
        A = rng.uniform(-1, 1, (n, n)).astype(np.float32)
        A[np.diag_indices(n)] = n if not dg else 0.5
        if dg:
            A *= 1.0 / n
            A[np.diag_indices(n)] = 123.0
        B = rng.uniform(-1, 1, (M, N)).astype(np.float32)
        A, B = A.astype(dt), B.astype(dt)
        T = np.tril(f64(A)) if uplo == "L" else np.triu(f64(A))
        if dg:
            np.fill_diagonal(T, 1.0)
        T = T.T if ta else T
        Xr = np.linalg.solve(T, 2.0 * f64(B)) if side == "L" else np.linalg.solve(T.T, 2.0 * f64(B).T).T
        X = f64(g9.trsm(A, B, side, uplo, ta, dg, 2.0, accurate=acc))
        e = np.abs(X - Xr).max() / max(np.abs(Xr).max(), 1e-300)
        assert e <= stol, f"{tag}: {e:.1e}"
