"""GEMM parity on the GPU: libgen9blas (through its C ABI) against the oracle and the float64 closed form.

Follows the reference's GEMM test (reference: lib/test_basic.py:44-79): the same sizes, alpha/beta values, all four
transpose combinations, plain and "zero-copy" memory (here: host NumPy arrays, staged by the library, and device
tensors, used in place), and the reference's error metric e = |C − ref| / (|alpha|·Σ|a·b| + |beta·c|).

Bounds on the reference-test shapes are the reference test's mean / max (lib/test_basic.py:4-8, 70-73; FP64 from
lib/test_level3.py:4-6), tightened to north_star's maxima where those hold at every K: SGEMM max 1e-6, DGEMM 1e-13,
HGEMM (H) 2e-3. For HS the reference's K-dependent bound applies (K < 256: 4.9e-4 / 5e-3, else 1e-4 / 1e-3): at
small K the final FP16 rounding of C alone exceeds north_star's 1e-4, which is written for the n ≥ 1024 configs,
where test_gemm_config_sizes applies it. Where the oracle is cheap (M·N·K ≤ 2e7) the
GPU result is also compared with the oracle's restatement of the reference kernel: both must meet the same bound
against float64, and they must agree with each other to twice that bound.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

KIND_DT = {"H": np.float16, "HS": np.float16, "S": np.float32, "D": np.float64}
MAX_E = {"H": 2e-3, "HS": 1e-4, "S": 1e-6, "D": 1e-13}       # north_star, for the config sizes
MEAN_E = {"H": 4.9e-4, "HS": 1e-4, "S": 1e-6, "D": 1e-14}


def case_bounds(kind, K):
    """(mean, max) bound of the reference test for one shape (lib/test_basic.py:4-8, 70-73)."""
    if kind == "HS":
        return (4.9e-4, 5e-3) if K < 256 else (1e-4, 1e-3)
    return MEAN_E[kind], MAX_E[kind]
SIZES = [(1, 1, 1, 1.0, 0.0), (17, 33, 15, 1.0, 0.0), (100, 70, 300, 2.0, 0.0), (64, 96, 48, 0.5, 1.0),
         (333, 129, 1000, 1.0, -1.0), (1000, 1024, 777, 1.0, 0.5),
         # FP32/FP64 two-k-group tiles: the second group's only block tile lies past K (K = 20), and one whole block
         # tile per group (K = 64)
         (1024, 960, 20, 1.0, 0.0), (960, 1024, 64, -1.0, 0.25)]


def _to_dev(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _run_case(g9, torch, kind, M, N, K, al, be, ta, tb, dev, seed=0):
    dt = KIND_DT[kind]
    rng = np.random.default_rng(seed)
    a = rng.uniform(-1, 1, (K, M) if ta else (M, K)).astype(dt)
    b = rng.uniform(-1, 1, (N, K) if tb else (K, N)).astype(dt)
    C0 = rng.uniform(-1, 1, (M, N)).astype(dt)
    if dev:
        A_, B_ = _to_dev(torch, a), _to_dev(torch, b)
        C_ = _to_dev(torch, C0 if be else np.zeros_like(C0))
        A = A_.t() if ta else A_
        B = B_.t() if tb else B_
    else:
        A, B = (a.T if ta else a), (b.T if tb else b)
        C_ = (C0 if be else np.zeros_like(C0)).copy()
    W = g9.gemm(A, B, al, be, C_, accurate=(kind == "HS"))
    zc = g9.last_zero_copy()
    if dev:
        torch.cuda.synchronize()
        W = W.cpu().numpy()
    opA, opB = (a.T if ta else a), (b.T if tb else b)
    return W, opA, opB, C0, zc


@pytest.mark.parametrize("kind", ["H", "HS", "S", "D"])
@pytest.mark.parametrize("M,N,K,al,be", SIZES)
def test_gemm_reference_cases(g9, orc, torch_dev, kind, M, N, K, al, be):
    for ta, tb in [(0, 0), (1, 0), (0, 1), (1, 1)]:
        for dev in (False, True):
            W, opA, opB, C0, zc = _run_case(g9, torch_dev, kind, M, N, K, al, be, ta, tb, dev)
            mean, mx = orc.gemm_error(W, opA, opB, al, be, C0)
            tag = f"{kind} M={M} N={N} K={K} a={al} b={be} tA={ta} tB={tb} dev={dev}"
            bmean, bmax = case_bounds(kind, K)
            assert mx <= bmax, f"{tag}: max e {mx:.2e}"
            assert mean <= bmean, f"{tag}: mean e {mean:.2e}"
            assert zc == (7 if dev else 0), f"{tag}: zero-copy bits {zc:03b}"
            if dev or M * N * K > 2e7:
                continue
            # the oracle's restatement of the reference kernel meets the same bound, and the two agree
            R = orc.gemm(kind, opA, opB, al, be, C0)
            bound = 2.5e-3 if kind == "H" else bmax
            omean, omx = orc.gemm_error(R, opA, opB, al, be, C0)
            assert omx <= bound, f"oracle {tag}: max e {omx:.2e}"
            assert orc.gemm_diff(W, R, opA, opB, al, be, C0) <= 2 * bound, f"GPU vs oracle {tag}"


def _random_cases(seed, count):
    """Seeded random shapes: each of M, N, K is small (1-79), a multiple of 64 (the tile classes), within 3 of one
    (edge strips, short k-steps), or in 80-699; with a type, layout, alpha, beta and operand residency."""
    r = np.random.default_rng(seed)

    def dim():
        c = int(r.integers(0, 4))
        if c == 0:
            return int(r.integers(1, 80))
        if c == 1:
            return 64 * int(r.integers(1, 12))
        if c == 2:
            return max(1, 64 * int(r.integers(1, 12)) + int(r.integers(-3, 4)))
        return int(r.integers(80, 700))
    cases = []
    for _ in range(count):
        M, N, K = dim(), dim(), dim()
        cases.append((str(r.choice(["H", "HS", "S", "D"])), M, N, K, float(r.choice([1.0, -0.5, 2.0])),
                      float(r.choice([0.0, 0.0, 1.0, -1.5])), int(r.integers(0, 2)), int(r.integers(0, 2)),
                      bool(r.integers(0, 2))))
    return cases


@pytest.mark.parametrize("case", _random_cases(2026, 256), ids=lambda c: "-".join(str(v) for v in c))
def test_gemm_random_shapes(g9, orc, torch_dev, case):
    """256 seeded random products across the dispatch's size classes (the skinny kernels, 64×64 / 128×128 / 256×256
    whole tiles and their edge strips, split-K, the general kernel), every type and layout, host and device
    operands, against float64 with the reference test's bounds."""
    kind, M, N, K, al, be, ta, tb, dev = case
    W, opA, opB, C0, zc = _run_case(g9, torch_dev, kind, M, N, K, al, be, ta, tb, dev, seed=M * 7919 + N * 31 + K)
    mean, mx = orc.gemm_error(W, opA, opB, al, be, C0)
    bmean, bmax = case_bounds(kind, K)
    tag = f"{kind} M={M} N={N} K={K} a={al} b={be} tA={ta} tB={tb} dev={dev}"
    assert mx <= bmax, f"{tag}: max e {mx:.2e}"
    assert mean <= bmean, f"{tag}: mean e {mean:.2e}"
    assert zc == (7 if dev else 0), f"{tag}: zero-copy bits {zc:03b}"


def _skinny_cases(seed, count):
    """Seeded skinny products C = A·Wᵀ (A not transposed, B stored N×K): M from 1 to 16 (or N, when swapped), the
    other side and K small, a multiple of 64 or 256 (the matrix-core skinny kernel takes K in 256-k groups), or in
    80-1999."""
    r = np.random.default_rng(seed)

    def dim(big):
        c = int(r.integers(0, 4))
        if c == 0:
            return int(r.integers(1, 80))
        if c == 1:
            return 64 * int(r.integers(1, 32))
        if c == 2:
            return 256 * int(r.integers(1, 9))
        return int(r.integers(80, 2000 if big else 700))
    out = []
    for _ in range(count):
        m, other, K = int(r.integers(1, 17)), dim(True), dim(False)
        M, N = (m, other) if r.integers(0, 4) else (other, m)
        out.append((str(r.choice(["H", "HS", "S", "D"])), M, N, K, float(r.choice([1.0, -0.75])),
                    float(r.choice([0.0, 0.0, 1.0, 0.5])), bool(r.integers(0, 2))))
    return out


@pytest.mark.parametrize("case", _skinny_cases(2028, 128), ids=lambda c: "-".join(str(v) for v in c))
def test_skinny_random_shapes(g9, orc, torch_dev, case):
    """128 seeded random skinny products (one side at most 16, A not transposed, B stored N×K: the skinny kernels, or
    the roles swapped when N is the small side), every type, host and device, against float64 with the reference
    test's bounds."""
    kind, M, N, K, al, be, dev = case
    W, opA, opB, C0, zc = _run_case(g9, torch_dev, kind, M, N, K, al, be, 0, 1, dev, seed=M * 131 + N * 7 + K)
    mean, mx = orc.gemm_error(W, opA, opB, al, be, C0)
    bmean, bmax = case_bounds(kind, K)
    tag = f"{kind} M={M} N={N} K={K} a={al} b={be} dev={dev}"
    assert mx <= bmax, f"{tag}: max e {mx:.2e}"
    assert mean <= bmean, f"{tag}: mean e {mean:.2e}"


def _sampled_rows_error(W, A, B, rows, alpha=1.0, beta=0.0, C0=None, tB=False):
    """Reference metric on sampled rows of C = alpha·A·op(B) + beta·C0 (float64)."""
    a64 = A[rows].astype(np.float64)
    b64 = (B.T if tB else B).astype(np.float64)
    ref = alpha * (a64 @ b64)
    scale = abs(alpha) * (np.abs(a64) @ np.abs(b64))
    if beta:
        c64 = C0[rows].astype(np.float64)
        ref += beta * c64
        scale += abs(beta) * np.abs(c64)
    e = np.abs(W[rows].astype(np.float64) - ref) / scale
    return float(e.mean()), float(e.max())


@pytest.mark.parametrize("kind,n", [("H", 1024), ("H", 2048), ("H", 4096), ("HS", 1024), ("HS", 2048), ("HS", 4096),
                                    ("S", 1024), ("S", 4096), ("D", 1024), ("D", 4096)])
def test_gemm_config_sizes(g9, orc, torch_dev, kind, n):
    """The benchmarked configurations: square n, NN, alpha = 1, beta = 0; FP16 inputs N(0, 1), FP32/FP64 U[-1, 1] (device buffers)."""
    torch = torch_dev
    dt = KIND_DT[kind]
    if dt == np.float16:
        A, B = orc.normal((n, n), dt, orc.SEED_A), orc.normal((n, n), dt, orc.SEED_B)
    else:
        A, B = orc.uniform((n, n), dt, orc.SEED_A), orc.uniform((n, n), dt, orc.SEED_B)
    Ad, Bd = _to_dev(torch, A), _to_dev(torch, B)
    W = g9.gemm(Ad, Bd, accurate=(kind == "HS")).cpu().numpy()
    rows = np.unique(np.r_[0, n - 1, np.random.default_rng(5).integers(0, n, 62)])
    mean, mx = _sampled_rows_error(W, A, B, rows)
    assert mx <= MAX_E[kind], f"{kind} n={n}: max e {mx:.2e}"
    assert mean <= MEAN_E[kind], f"{kind} n={n}: mean e {mean:.2e}"
    assert np.isfinite(W).all()


@pytest.mark.parametrize("K", [1000, 1024])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_sgemm_two_group_tiles(g9, orc, torch_dev, ta, tb, K):
    """2000×2048 FP32 products, alpha = 1.5, beta = 0.5, every layout, against float64 on sampled rows. K = 1000 (not a
    multiple of 32) takes the general kernel's 128×128 tiles with two k groups, whose second group's last block tile
    is partly past K, so every tile takes the checked loop; K = 1024 takes the FP32 whole-tile kernel on the
    1984×2048 interior (64×64 tiles) and the general kernel on the 16-row bottom strip. The general kernel's
    unchecked two-group loop at K = 1024 is covered by test_sgemm_generic_two_group_fast_loop."""
    torch = torch_dev
    M, N = 2000, 2048
    a = orc.uniform((K, M) if ta else (M, K), np.float32, orc.SEED_A)
    b = orc.uniform((N, K) if tb else (K, N), np.float32, orc.SEED_B)
    c0 = orc.uniform((M, N), np.float32, 3)
    Ad, Bd, Cd = _to_dev(torch, a), _to_dev(torch, b), _to_dev(torch, c0)
    W = g9.gemm(Ad.t() if ta else Ad, Bd.t() if tb else Bd, 1.5, 0.5, Cd).cpu().numpy()
    opA = a.T if ta else a
    rows = np.unique(np.r_[0, M - 1, np.random.default_rng(6).integers(0, M, 62)])
    mean, mx = _sampled_rows_error(W, opA, b, rows, 1.5, 0.5, c0, tB=bool(tb))
    assert mx <= MAX_E["S"], f"tA={ta} tB={tb} K={K}: max e {mx:.2e}"
    assert mean <= MEAN_E["S"], f"tA={ta} tB={tb} K={K}: mean e {mean:.2e}"


def test_sgemm_generic_two_group_fast_loop(tmp_path):
    """GEN9BLAS_SGEMM=generic keeps FP32 on the general kernel: 2000×2048×1024 then takes 128×128 tiles with two k
    groups, whose interior tiles run the unchecked fast loop, in every layout, alpha = 1.5, beta = 0.5, against
    float64 (full matrices, the reference metric). Runs in a child process because the variable is read once."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.realpath(__file__)))
    script = tmp_path / "generic.py"
    script.write_text(
        "import sys, numpy as np\n"
        f"sys.path.insert(0, {os.path.join(root, 'gen9-gpu-blas_amd')!r}); sys.path.insert(0, {os.path.join(root, 'oracle')!r})\n"
        "import gen9blas as g, oracle as o\n"
        "rng = np.random.default_rng(9)\n"
        "M, N, K = 2000, 2048, 1024\n"
        "for ta in (0, 1):\n"
        "    for tb in (0, 1):\n"
        "        u = rng.uniform(-1, 1, (M, K)).astype(np.float32); v = rng.uniform(-1, 1, (K, N)).astype(np.float32)\n"
        "        c0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)\n"
        "        U = np.ascontiguousarray(u.T).T if ta else u; V = np.ascontiguousarray(v.T).T if tb else v\n"
        "        W = g.gemm(U, V, 1.5, 0.5, c0.copy())\n"
        "        mean, mx = o.gemm_error(W, u, v, 1.5, 0.5, c0)\n"
        "        assert mx <= 1e-6 and mean <= 1e-6, (ta, tb, mean, mx)\n"
        "print('ok')\n")
    env = dict(os.environ)
    env["GEN9BLAS_SGEMM"] = "generic"
    r = subprocess.run([sys.executable, str(script)], env=env, capture_output=True, text=True, timeout=200)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stderr[-2000:]


def test_sgemm_odd_shape(g9, orc, torch_dev):
    """The benchmarked odd shape: M = 3000, N = 11008, K = 4096, transB (B stored N×K), beta = 0.5, C pre-filled U[-1, 1]."""
    torch = torch_dev
    M, N, K = 3000, 11008, 4096
    A = orc.uniform((M, K), np.float32, orc.SEED_A)
    B = orc.uniform((N, K), np.float32, orc.SEED_B)
    C0 = orc.uniform((M, N), np.float32, orc.SEED_C)
    Ad, Bd, Cd = _to_dev(torch, A), _to_dev(torch, B), _to_dev(torch, C0)
    g9.sgemm(Ad, Bd.t(), 1.0, 0.5, Cd)
    W = Cd.cpu().numpy()
    rows = np.unique(np.r_[0, 2999, 2944, 2943, np.random.default_rng(6).integers(0, M, 40)])
    mean, mx = _sampled_rows_error(W, A, B, rows, 1.0, 0.5, C0, tB=True)
    assert mx <= MAX_E["S"], f"odd SGEMM: max e {mx:.2e}"
    cols = [0, N - 1, 11007, 10999]
    assert np.isfinite(W[:, cols]).all()


def test_gemm_batched(g9, orc, torch_dev):
    """Batched GEMM (reference: lib/test_level3.py:48-53): 33 × (65×47×129) in every type, host and device memory."""
    rng = np.random.default_rng(9)
    for kind in ("H", "HS", "S", "D"):
        dt = KIND_DT[kind]
        A = rng.uniform(-1, 1, (33, 65, 129)).astype(dt)
        B = rng.uniform(-1, 1, (33, 129, 47)).astype(dt)
        for dev in (False, True):
            Ai, Bi = (_to_dev(torch_dev, A), _to_dev(torch_dev, B)) if dev else (A, B)
            W = g9.gemm_batched(Ai, Bi, accurate=(kind == "HS"))
            W = W.cpu().numpy() if dev else W
            for b in (0, 16, 32):
                mean, mx = orc.gemm_error(W[b], A[b], B[b])
                assert mx <= case_bounds(kind, 129)[1], f"batched {kind} dev={dev} b={b}: max e {mx:.2e}"


def test_gemm_nothing_outside_c(g9, torch_dev):
    """C as a slice of a larger array: only the slice changes (host and device)."""
    rng = np.random.default_rng(4)
    for dt in (np.float16, np.float32, np.float64):
        A = rng.uniform(-1, 1, (70, 90)).astype(dt)
        B = rng.uniform(-1, 1, (90, 50)).astype(dt)
        big = rng.uniform(-1, 1, (74, 60)).astype(dt)
        ref = big.copy()
        C = big[2:72, 3:53]
        g9.gemm(A, B, 1.0, 0.5, C)
        mask = np.ones(big.shape, bool)
        mask[2:72, 3:53] = False
        assert np.array_equal(big[mask], ref[mask]), f"{dt}: write outside the C slice"
        bigd = _to_dev(torch_dev, ref)
        g9.gemm(_to_dev(torch_dev, A), _to_dev(torch_dev, B), 1.0, 0.5, bigd[2:72, 3:53])
        got = bigd.cpu().numpy()
        assert np.array_equal(got[mask], ref[mask]), f"{dt} device: write outside the C slice"
        np.testing.assert_allclose(got[2:72, 3:53].astype(np.float64), big[2:72, 3:53].astype(np.float64),
                                   rtol=0, atol=2e-3 if dt == np.float16 else 1e-5)


def test_host_operands_staged(g9):
    """Host (pageable NumPy) operands of 4 MiB and more move through the pinned staging ring in chunks: whole spans
    (A, B, C 18-36 MB, several 8 MiB chunks each way) and re-pitched rows (A and C column slices of arrays three times
    wider, so their row gaps exceed half the span: 2D copies chunked by rows, C copied back row by row). Small-integer
    inputs make every result exact; nothing outside the C slice changes."""
    rng = np.random.default_rng(31)
    A = rng.integers(-2, 3, (3000, 1500)).astype(np.float32)
    B = rng.integers(-2, 3, (1500, 3000)).astype(np.float32)
    C0 = rng.integers(-2, 3, (3000, 3000)).astype(np.float32)
    C = C0.copy()
    g9.gemm(A, B, 1.0, 2.0, C)
    ref = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.int64) + 2 * C0.astype(np.int64)
    assert np.array_equal(C.astype(np.int64), ref), "whole spans"
    big_a = rng.integers(-2, 3, (3000, 3000)).astype(np.float32)
    big_c = rng.integers(-2, 3, (3000, 3000)).astype(np.float32)
    keep = big_c.copy()
    A2, C2 = big_a[:, 1000:2000], big_c[:, 500:1500]
    B2 = B[:1000, :1000].copy()
    g9.gemm(A2, B2, 1.0, 2.0, C2)
    ref = (A2.astype(np.float64) @ B2.astype(np.float64)).astype(np.int64) + 2 * keep[:, 500:1500].astype(np.int64)
    assert np.array_equal(big_c[:, 500:1500].astype(np.int64), ref), "re-pitched rows"
    mask = np.ones(big_c.shape, bool)
    mask[:, 500:1500] = False
    assert np.array_equal(big_c[mask], keep[mask]), "write outside the C slice"


def test_host_products_in_row_panels(g9, torch_dev):
    """Products whose C is pageable and spans two or more 8 MiB pinned chunks run in row panels of at most one chunk
    of C: each panel's rows go back on a second stream while the next panel's inputs come in. Covered: 4 FP16 panels
    of 1024 rows (A in panels); FP32 with transposed A (staged whole), transposed B, beta = 2 and C a column slice
    whose row gaps must survive the copy back, 6 panels with a last one of 40 rows; FP64 with page-locked A and a
    last panel of 252 rows; accurate FP16 in 2 panels. Small integers make the first two exact. The FP16 results must
    equal the same product on device buffers bit for bit (each panel is a band of rows, tiled like the whole); FP64
    meets the float64 bound, and so does its difference from the device result, as a 512-row panel may take tiles
    that split K differently from the whole product's."""
    torch = torch_dev
    rng = np.random.default_rng(43)

    def ints(shape, dt, lim):
        return rng.integers(-lim, lim + 1, shape).astype(dt)

    def on_device(A, B, alpha, beta, C0, accurate=False):
        Ad = _to_dev(torch, A.T).t() if A.flags.f_contiguous and not A.flags.c_contiguous else _to_dev(torch, A)
        Bd = _to_dev(torch, B.T).t() if B.flags.f_contiguous and not B.flags.c_contiguous else _to_dev(torch, B)
        Cd = _to_dev(torch, C0)
        g9.gemm(Ad, Bd, alpha, beta, Cd, accurate=accurate)
        torch.cuda.synchronize()
        return Cd.cpu().numpy()

    # FP16, NN, 4096 x 4096 x 1024 in {-1, 0, 1}: every sum is an integer of at most 1024, exact in FP16
    A, B = ints((4096, 1024), np.float16, 1), ints((1024, 4096), np.float16, 1)
    C = np.zeros((4096, 4096), np.float16)
    g9.gemm(A, B, 1.0, 0.0, C)
    ref = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.int64)
    assert np.array_equal(C.astype(np.int64), ref), "FP16 panels"
    assert np.array_equal(C, on_device(A, B, 1.0, 0.0, np.zeros_like(C))), "FP16 panels against device buffers"

    # FP32, A and B transposed views, C a 2600 x 3000 slice of 2600 x 3100 (gaps), beta = 2
    at, bt = ints((700, 2600), np.float32, 2), ints((3000, 700), np.float32, 2)
    A, B = at.T, bt.T
    big_c = ints((2600, 3100), np.float32, 2)
    keep = big_c.copy()
    C = big_c[:, :3000]
    g9.gemm(A, B, 1.0, 2.0, C)
    ref = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.int64) + 2 * keep[:, :3000].astype(np.int64)
    assert np.array_equal(C.astype(np.int64), ref), "FP32 panels, transposed, beta = 2"
    assert np.all(big_c[:, 3000:] == keep[:, 3000:]), "gap columns of C changed"
    assert np.array_equal(C, on_device(A, B, 1.0, 2.0, keep[:, :3000].copy())), "FP32 panels against device buffers"

    # FP64, page-locked A, pageable B and C, alpha = -0.5, beta = 0.25
    A = g9.empty((2300, 300), np.float64)
    A[:] = rng.uniform(-1, 1, A.shape)
    B = rng.uniform(-1, 1, (300, 2048))
    C0 = rng.uniform(-1, 1, (2300, 2048))
    C = C0.copy()
    g9.gemm(A, B, -0.5, 0.25, C)
    rows = np.unique(np.r_[0, 511, 512, 2047, 2048, 2299, rng.integers(0, 2300, 40)])
    mean, mx = _sampled_rows_error(C, np.asarray(A), B, rows, alpha=-0.5, beta=0.25, C0=C0)
    assert mx <= MAX_E["D"], f"FP64 panels: max e {mx:.2e}"
    scale = 0.5 * (np.abs(np.asarray(A)) @ np.abs(B)) + 0.25 * np.abs(C0)
    d = np.abs(C - on_device(np.asarray(A), B, -0.5, 0.25, C0)) / scale
    assert d.max() <= MAX_E["D"], f"FP64 panels against device buffers: {d.max():.2e}"

    # accurate FP16, 4096 x 2048 x 512 on N(0, 1): C is 16 MiB, two panels of 2048 rows
    A = rng.standard_normal((4096, 512)).astype(np.float16)
    B = rng.standard_normal((512, 2048)).astype(np.float16)
    C = np.zeros((4096, 2048), np.float16)
    g9.gemm(A, B, 1.0, 0.0, C, accurate=True)
    rows = np.unique(np.r_[0, 2047, 2048, 4095, rng.integers(0, 4096, 40)])
    mean, mx = _sampled_rows_error(C, A, B, rows)
    assert mx <= case_bounds("HS", 512)[1] and mean <= case_bounds("HS", 512)[0], f"HS panels: {mean:.2e} / {mx:.2e}"
    assert np.array_equal(C, on_device(A, B, 1.0, 0.0, np.zeros_like(C), accurate=True)), "HS panels against device"


def test_gemm_beta_zero_does_not_read_c(g9, torch_dev):
    """beta = 0: C is not read, NaN in C does not propagate (reference: lib/gen9blas.h:133 semantics for C)."""
    for dt in (np.float16, np.float32, np.float64):
        A = np.ones((40, 30), dt)
        B = np.ones((30, 20), dt)
        Cd = torch_dev.full((40, 20), float("nan"), dtype={np.float16: torch_dev.float16, np.float32: torch_dev.float32,
                                                           np.float64: torch_dev.float64}[dt], device="cuda")
        g9.gemm(_to_dev(torch_dev, A), _to_dev(torch_dev, B), 1.0, 0.0, Cd)
        assert (Cd.cpu().numpy() == 30).all()


def test_gemm_exact_small_integers(g9, torch_dev):
    """Exactly representable products and sums: every type must return the exact integer result (catches transposed
    operands, dropped k blocks and wrong tile offsets bit-exactly)."""
    rng = np.random.default_rng(12)
    for dt in (np.float16, np.float32, np.float64):
        for (M, N, K) in [(5, 7, 3), (257, 130, 200), (300, 520, 129)]:
            a = rng.integers(-3, 4, (M, K)).astype(dt)
            b = rng.integers(-3, 4, (K, N)).astype(dt)
            ref = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.int64)
            if dt == np.float16 and np.abs(ref).max() > 2048:
                continue
            for ta in (0, 1):
                for tb in (0, 1):
                    A = np.ascontiguousarray(a.T).T if ta else a
                    B = np.ascontiguousarray(b.T).T if tb else b
                    W = g9.gemm(A, B)
                    assert np.array_equal(W.astype(np.int64), ref), f"{dt} {M}x{N}x{K} tA={ta} tB={tb}"


@pytest.mark.parametrize("M,N,K,count", [(256, 384, 320, 1), (128, 256, 2112, 1), (384, 256, 256, 1), (128, 128, 64, 1),
                                         (1024, 1024, 64, 4), (1024, 1024, 320, 4), (1024, 1024, 192, 16)])
def test_hgemm_whole_tile_kernel(g9, torch_dev, M, N, K, count):
    """Shapes served by the whole-tile FP16 kernel (M, N multiples of 128, K of 64, 16-byte aligned operands): fewer
    128×128 tiles than CUs (64×64 tiles in every layout, the mn-contiguous operands through the 64-wide transposing
    loader, three LDS stages, fragments read a k-step ahead over an odd, even and single k-step count), 256 tiles of
    128×128 over a batch of 4 (one k-step, and five: the loaders' swizzles kept as they advance over k), and
    256×256 tiles over a batch of 16, in every transpose
    layout, through the C ABI on device memory. Small-integer inputs make every result exact, so a misplaced 16-byte
    chunk, k row or tile shows up bit-exactly; alpha/beta are then checked against float64 with the HGEMM bound."""
    import ctypes
    torch = torch_dev
    rng = np.random.default_rng(21)
    for ta in (0, 1):
        for tb in (0, 1):
            a = rng.integers(-2, 3, (count, M, K)).astype(np.float16)
            b = rng.integers(-2, 3, (count, K, N)).astype(np.float16)
            c0 = rng.uniform(-1, 1, (count, M, N)).astype(np.float16)
            A = np.ascontiguousarray(a.transpose(0, 2, 1)) if ta else a      # stored K×M when transposed
            B = np.ascontiguousarray(b.transpose(0, 2, 1)) if tb else b      # stored N×K when transposed
            Ad, Bd = _to_dev(torch, A), _to_dev(torch, B)
            ref = np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(np.int64)   # exact: |sums| < 2^53
            assert np.abs(ref).max() <= 2048
            for al, be in ((1.0, 0.0), (0.5, -1.5)):
                Cd = _to_dev(torch, c0 if be else np.zeros_like(c0))
                lda, ldb = (M if ta else K), (K if tb else N)
                rc = g9._lib.gen9blas_gemm_batched(g9.GEN9BLAS_H, ta, tb, M, N, K, al, ctypes.c_void_p(Ad.data_ptr()),
                                                   lda, M * K, ctypes.c_void_p(Bd.data_ptr()), ldb, K * N, be,
                                                   ctypes.c_void_p(Cd.data_ptr()), N, M * N, count)
                assert rc == 0, g9._lib.gen9blas_error()
                torch.cuda.synchronize()
                W = Cd.cpu().numpy()
                tag = f"{M}x{N}x{K}x{count} tA={ta} tB={tb} alpha={al} beta={be}"
                if be == 0.0:
                    assert np.array_equal(W.astype(np.int64), ref), tag
                else:
                    r64 = al * ref + be * c0.astype(np.float64)
                    scale = abs(al) * (np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))) + abs(be) * np.abs(c0.astype(np.float64))
                    e = np.abs(W.astype(np.float64) - r64) / scale
                    assert e.max() <= 2e-3, f"{tag}: max e {e.max():.2e}"


@pytest.mark.parametrize("M,N,K,count", [(1024, 1024, 96, 1), (2048, 2048, 64, 1), (4096, 4096, 160, 1),
                                         (1032, 1092, 64, 1), (512, 512, 64, 4), (1100, 1536, 96, 1),
                                         (2100, 4096, 64, 1), (1102, 1536, 64, 2), (1024, 1024, 320, 1)])
def test_sgemm_whole_tile_kernel(g9, torch_dev, M, N, K, count):
    """Shapes served by the FP32 whole-tile kernel (16-byte aligned operands, K a multiple of 32, whole tiles filling
    the CUs): 64×64 tiles with a k-step count below one 256-k block (n = 1024, K = 96), 128×128 tiles (n = 2048),
    128×256 tiles with one whole 128-k block and a shorter one (K = 160), 64×64 tiles over the interior of
    1032×1092 with the 8-row and 4-column strips on the general kernel, and a batch of 4. Bottom strips over a width of
    whole 64-column tiles take 64×64 tiles shifted up onto the last 64 rows, storing only the strip's own rows: 12
    rows under 64×64 tiles (1100×1536), 52 rows under 128×256 tiles (2100×4096), and 14 rows (1102×1536, batch of 2)
    where the shift would misalign a transposed A, so TN and TT keep the general kernel there; 1024² with K = 320
    takes 64×64 tiles with 10 k-steps, a block shorter than the 8-step sum blocks after a whole one. Every transpose layout,
    through the C ABI on device memory. Small-integer inputs make every result exact (bit-equal to the integer
    product, so a misplaced element, k row, tile or strip shows up); alpha/beta are then checked against float64 with
    the SGEMM bound."""
    import ctypes
    torch = torch_dev
    rng = np.random.default_rng(22)
    for ta in (0, 1):
        for tb in (0, 1):
            a = rng.integers(-2, 3, (count, M, K)).astype(np.float32)
            b = rng.integers(-2, 3, (count, K, N)).astype(np.float32)
            c0 = rng.uniform(-1, 1, (count, M, N)).astype(np.float32)
            A = np.ascontiguousarray(a.transpose(0, 2, 1)) if ta else a      # stored K×M when transposed
            B = np.ascontiguousarray(b.transpose(0, 2, 1)) if tb else b      # stored N×K when transposed
            Ad, Bd = _to_dev(torch, A), _to_dev(torch, B)
            ref = np.matmul(a.astype(np.float64), b.astype(np.float64))     # exact: |sums| < 2^24
            assert np.abs(ref).max() < 2 ** 24
            for al, be in ((1.0, 0.0), (0.5, -1.5)):
                Cd = _to_dev(torch, c0 if be else np.full_like(c0, np.nan))  # beta = 0: C must not be read
                lda, ldb = (M if ta else K), (K if tb else N)
                rc = g9._lib.gen9blas_gemm_batched(g9.GEN9BLAS_S, ta, tb, M, N, K, al, ctypes.c_void_p(Ad.data_ptr()),
                                                   lda, M * K, ctypes.c_void_p(Bd.data_ptr()), ldb, K * N, be,
                                                   ctypes.c_void_p(Cd.data_ptr()), N, M * N, count)
                assert rc == 0, g9._lib.gen9blas_error()
                torch.cuda.synchronize()
                W = Cd.cpu().numpy()
                tag = f"{M}x{N}x{K}x{count} tA={ta} tB={tb} alpha={al} beta={be}"
                if be == 0.0:
                    assert np.array_equal(W.astype(np.float64), ref), tag
                else:
                    r64 = al * ref + be * c0.astype(np.float64)
                    scale = abs(al) * np.matmul(np.abs(a.astype(np.float64)), np.abs(b.astype(np.float64))) + \
                        abs(be) * np.abs(c0.astype(np.float64))
                    e = np.abs(W.astype(np.float64) - r64) / scale
                    assert e.max() <= 1e-6, f"{tag}: max e {e.max():.2e}"


def _child(args, extra_env, timeout):
    """Runs tests/long_launch_child.py in a child process with the given variables (read once per process)."""
    import os
    import subprocess
    import sys
    env = dict(os.environ)
    for v in ("GEN9BLAS_MAX_LAUNCH_MS", "GEN9BLAS_SPLITK"):
        env.pop(v, None)
    env.update(extra_env)
    child = os.path.join(os.path.dirname(os.path.realpath(__file__)), "long_launch_child.py")
    r = subprocess.run([sys.executable, "-u", child, *args], env=env, capture_output=True, text=True, timeout=timeout)
    print(r.stdout[-2000:])
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-2000:])


def test_banded_launch(g9, tmp_path):
    """GEN9BLAS_MAX_LAUNCH_MS splits a long product into row bands, each its own launch (reference:
    lib/src/gemm.c:119-164). Every type, A plain and transposed (a band of op(A) is a column range of the stored
    matrix), and a strided batch of 3 with both operands transposed (bands inside every matrix of the batch):
    - the banded result meets the reference bounds against float64 (full matrices, the reference metric);
    - it equals the unbanded call's result bit for bit (GEN9BLAS_SPLITK=0 in both runs: otherwise split-K slices and
      two-k-group tiles are picked from each band's shape and may sum in another order)."""
    import numpy as np
    plain, banded = tmp_path / "plain.npz", tmp_path / "banded.npz"
    _child(["layouts", str(plain)], {"GEN9BLAS_SPLITK": "0"}, 100)
    _child(["layouts", str(banded)], {"GEN9BLAS_SPLITK": "0", "GEN9BLAS_MAX_LAUNCH_MS": "0.0001"}, 100)
    P, B = np.load(plain), np.load(banded)
    for kind in ("S", "D", "H", "HS"):
        for case in ("tA0", "tA1", "batch"):
            key = f"{kind}_{case}"
            bound = case_bounds(kind, 700)[1]
            assert float(B[key + "_err"]) <= bound, f"banded {key}: max e {float(B[key + '_err']):.2e}"
            assert float(P[key + "_err"]) <= bound, f"plain {key}: max e {float(P[key + '_err']):.2e}"
            assert np.array_equal(P[key], B[key]), f"{key}: banded result differs from the unbanded one"


@pytest.mark.parametrize("banded", [False, True])
def test_long_launch_cases(g9, tmp_path, banded):
    """The reference's long-launch sizes (reference: lib/test_long_launch.py:39-51): DGEMM n = 4096, SGEMM n = 8192,
    accurate HGEMM n = 8192 and batched DGEMM 2 × 3072, U(0, 1) inputs in pinned host memory, checked against
    float64 on sampled rows (first, middle, last, and both sides of every 256-row band boundary) with the reference's
    bounds 1e-12 / 1e-4 / 5e-3 / 1e-12 (relative to |ref|; all products are positive, so this is also the reference
    GEMM metric). Unbanded, and with GEN9BLAS_MAX_LAUNCH_MS = 1 (6-16 bands per product)."""
    import json
    out = tmp_path / "long.json"
    _child(["cases", str(out)], {"GEN9BLAS_MAX_LAUNCH_MS": "1"} if banded else {}, 110)
    res = json.loads(out.read_text())
    bounds = {"dgemm n=4096": 1e-12, "sgemm n=8192": 1e-4, "hgemm accurate n=8192": 5e-3,
              "batched dgemm 2 x 3072": 1e-12}
    for name, bound in bounds.items():
        assert res[name] <= bound, f"{name} banded={banded}: max rel err {res[name]:.2e}"


def test_gemm_split_k(tmp_path):
    """Split-K (GEN9BLAS_SPLITK=n forces n slices; by default small products split to fill the CUs): every type and
    layout, K not a multiple of the slice, alpha/beta with C read once in the reduction, exact on small integers and
    within the reference bounds on uniform inputs. Runs in a child process because the variable is read once."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.realpath(__file__)))
    script = tmp_path / "splitk.py"
    script.write_text(
        "import sys, numpy as np\n"
        f"sys.path.insert(0, {os.path.join(root, 'gen9-gpu-blas_amd')!r}); sys.path.insert(0, {os.path.join(root, 'oracle')!r})\n"
        "import gen9blas as g, oracle as o\n"
        "rng = np.random.default_rng(8)\n"
        "bound = {np.float16: 2e-3, np.float32: 1e-6, np.float64: 1e-13}\n"
        "for dt in (np.float32, np.float64, np.float16):\n"
        "    for (M, N, K) in [(200, 136, 1000), (64, 64, 777), (130, 260, 4096)]:\n"
        "        for ta in (0, 1):\n"
        "            for tb in (0, 1):\n"
        "                a = rng.integers(-2, 3, (M, K)).astype(dt); b = rng.integers(-2, 3, (K, N)).astype(dt)\n"
        "                A = np.ascontiguousarray(a.T).T if ta else a; B = np.ascontiguousarray(b.T).T if tb else b\n"
        "                ref = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.int64)\n"
        "                if np.abs(ref).max() <= 2048 or dt != np.float16:\n"
        "                    assert np.array_equal(g.gemm(A, B).astype(np.int64), ref), (dt, M, N, K, ta, tb)\n"
        "                u = rng.uniform(-1, 1, (M, K)).astype(dt); v = rng.uniform(-1, 1, (K, N)).astype(dt)\n"
        "                c0 = rng.uniform(-1, 1, (M, N)).astype(dt)\n"
        "                U = np.ascontiguousarray(u.T).T if ta else u; V = np.ascontiguousarray(v.T).T if tb else v\n"
        "                W = g.gemm(U, V, 0.75, -0.5, c0.copy())\n"
        "                mean, mx = o.gemm_error(W, u, v, 0.75, -0.5, c0)\n"
        "                assert mx <= bound[dt], (dt, M, N, K, ta, tb, mx)\n"
        "print('ok')\n")
    for forced in ("3", "8"):
        env = dict(os.environ)
        env["GEN9BLAS_SPLITK"] = forced
        r = subprocess.run([sys.executable, str(script)], env=env, capture_output=True, text=True, timeout=200)
        assert r.returncode == 0 and r.stdout.strip().endswith("ok"), f"GEN9BLAS_SPLITK={forced}: " + r.stderr[-2000:]


def test_small_host_operands_bounce_and_pinned(g9):
    """Small host operands. Pageable ones pass through the library's pinned bounce area: here views whose row gaps
    make up most of their span, so their rows are re-pitched on the way in (A, and C for beta) and on the way back
    (C), each span under 128 KiB. Page-locked ones (the module's `empty`) are copied by DMA straight from and into the
    caller's memory. Both against float64, with C's gap columns left as they were."""
    rng = np.random.default_rng(41)
    M, N, K = 24, 56, 72
    big_a = rng.standard_normal((M, 1000)).astype(np.float32)
    A = big_a[:, :K]
    B = rng.standard_normal((K, N)).astype(np.float32)
    big_c = np.full((M, 900), 7.0, np.float32)
    C = big_c[:, :N]
    ref = A.astype(np.float64) @ B.astype(np.float64)
    scale = np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64))
    g9.gemm(A, B, alpha=1.0, beta=0.5, C=C)
    e = np.abs(C.astype(np.float64) - (ref + 3.5)) / (scale + 3.5)
    assert e.max() <= 1e-6, f"pageable, re-pitched: max e {e.max():.2e}"
    assert np.all(big_c[:, N:] == 7.0), "gap columns of C changed"
    Ap, Bp, Cp = g9.empty((M, K), np.float32), g9.empty((K, N), np.float32), g9.empty((M, N), np.float32)
    Ap[:], Bp[:], Cp[:] = A, B, 1.0
    for _ in range(3):
        Cp[:] = 1.0
        g9.gemm(Ap, Bp, alpha=2.0, beta=-1.0, C=Cp)
        e = np.abs(Cp.astype(np.float64) - (2 * ref - 1.0)) / (2 * scale + 1.0)
        assert e.max() <= 1e-6, f"page-locked: max e {e.max():.2e}"
    W = g9.gemm(A, B)   # a new small result: a plain NumPy array, copied back through the bounce area
    e = np.abs(W.astype(np.float64) - ref) / scale
    assert e.max() <= 1e-6, f"new result: max e {e.max():.2e}"
