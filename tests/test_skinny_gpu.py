"""Skinny GEMM parity on the GPU (C = A·Wᵀ and the other layouts with min(M, N) ≤ 16).

Follows the reference's skinny test (reference: lib/test_skinny.py:38-63): the same shapes, both weight layouts,
transposed views, the role swap for small N, alpha/beta with C as a slice of a larger array and nothing written outside
it, host and device memory. Bound: max|C − ref| / max|ref| ≤ 4e-3 (FP16) and 2e-6 (FP32) against float64
(lib/test_skinny.py:19, 29-35); the oracle's restatement of the reference skinny kernel meets the same bound.
The 4096² decode shape of the benchmark is checked at M = 1, 2, 4, 8, 16 and with rotated weight copies.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = {np.float16: 4e-3, np.float32: 2e-6}
SHAPES = [(1, 1000, 777), (3, 517, 1029), (4, 2048, 128), (5, 64, 9), (8, 333, 4096), (9, 1500, 1500),
          (16, 4096, 1000), (1, 8, 3), (2, 7, 2000)]


def _err(W, ref):
    return float(np.max(np.abs(np.asarray(W, np.float64) - ref)) / max(1e-30, np.max(np.abs(ref))))


def _dev(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


@pytest.mark.parametrize("dt", [np.float16, np.float32])
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_skinny_reference_cases(g9, orc, torch_dev, dt, M, N, K):
    rng = np.random.default_rng(7)
    fn = g9.hgemm if dt == np.float16 else g9.sgemm
    for tA in (False, True):
        for tB in (False, True):
            a = rng.uniform(-1, 1, (K, M) if tA else (M, K)).astype(dt)
            b = rng.uniform(-1, 1, (N, K) if tB else (K, N)).astype(dt)
            A, B = (a.T if tA else a), (b.T if tB else b)
            ref = A.astype(np.float64) @ B.astype(np.float64)
            tag = f"{np.dtype(dt).name} M={M} N={N} K={K} tA={tA} tB={tB}"
            assert _err(fn(A, B), ref) <= TOL[dt], tag
            assert _err(fn(B.T, A.T), ref.T) <= TOL[dt], tag + " (small N)"
            Ad = _dev(torch_dev, a)
            Bd = _dev(torch_dev, b)
            Wd = fn(Ad.t() if tA else Ad, Bd.t() if tB else Bd)
            assert _err(Wd.cpu().numpy(), ref) <= TOL[dt], tag + " device"
    # alpha, beta, C as a slice (row stride), nothing outside the slice changes
    A = rng.uniform(-1, 1, (M, K)).astype(dt)
    W = rng.uniform(-1, 1, (N, K)).astype(dt)
    big = rng.uniform(-1, 1, (M + 2, N + 5)).astype(dt)
    C = big[1:M + 1, 2:N + 2]
    C0 = C.astype(np.float64)
    D0 = big.copy()
    fn(A, W.T, alpha=0.75, beta=-1.5, C=C)
    ref = 0.75 * A.astype(np.float64) @ W.astype(np.float64).T - 1.5 * C0
    assert _err(C, ref) <= TOL[dt]
    mask = np.ones(big.shape, bool)
    mask[1:M + 1, 2:N + 2] = False
    assert np.array_equal(big[mask], D0[mask]), "write outside the C slice"
    # the oracle's restatement of the reference skinny kernel meets the same bound
    if M * N * K <= 4e6:
        R = orc.skinny(A, W, 0.75, -1.5, C0.astype(dt), tB=True)
        assert _err(R, ref) <= TOL[dt]


@pytest.mark.parametrize("M", [1, 2, 4, 8, 16])
def test_skinny_decode_4096(g9, orc, torch_dev, M):
    """Benchmark shape: W 4096×4096 fp16 ~ N(0, 0.02), A M×4096 ~ N(0, 1), C = A·Wᵀ, rotated weight copies."""
    torch = torch_dev
    K = N = 4096
    A = orc.normal((M, K), np.float16, orc.SEED_A)
    Ad = _dev(torch, A)
    for i in range(3):
        W = orc.normal((N, K), np.float16, orc.SEED_W0 + i, 0.02)
        Wd = _dev(torch, W)
        C = g9.hgemm(Ad, Wd.t()).cpu().numpy()
        ref = A.astype(np.float64) @ W.astype(np.float64).T
        assert _err(C, ref) <= TOL[np.float16], f"M={M} copy {i}"
        # the reference metric (north_star bound for FP16 accumulation in FP32: ≤ 1e-4 relative to Σ|a·w|)
        scale = np.abs(A.astype(np.float64)) @ np.abs(W.astype(np.float64)).T
        assert float(np.max(np.abs(C - ref) / scale)) <= 1e-3, f"M={M} copy {i}: reference metric"


def test_skinny_oracle_parity_small(g9, orc):
    """GPU skinny vs the oracle's restatement on a small A·Wᵀ (both FP32-accumulated: they agree to FP16 rounding)."""
    rng = np.random.default_rng(3)
    for M in (1, 3, 16):
        A = rng.uniform(-1, 1, (M, 640)).astype(np.float16)
        W = rng.uniform(-1, 1, (300, 640)).astype(np.float16)
        G = g9.hgemm(A, W.T)
        R = orc.skinny(A, W, tB=True)
        d = np.abs(G.astype(np.float64) - R.astype(np.float64))
        ulp = np.abs(R.astype(np.float64)) * 2.0 ** -10 + 2.0 ** -24
        assert (d <= 2 * ulp).all(), f"M={M}: GPU and oracle differ by more than 2 FP16 ulp"


@pytest.mark.parametrize("M,N,K", [(3, 77, 512), (4, 2050, 1024), (5, 100, 256), (8, 4099, 512), (12, 333, 768),
                                   (16, 64, 4096), (16, 3000, 2560)])
def test_skinny_matrix_core_kernel(g9, torch_dev, M, N, K):
    """FP16 shapes that take the matrix-core skinny kernel (2 < M ≤ 16, K a multiple of 256, aligned rows): fewer
    K groups than waves, N not a multiple of 16, all three M tiles (4, 8, 16), host and device memory. Small-integer inputs give exact
    products and sums, so every result must be bit-exact; then alpha/beta on a C slice, and the role swap (small N)
    that stores through swapped strides."""
    rng = np.random.default_rng(31)
    a = rng.integers(-3, 4, (M, K)).astype(np.float16)
    w = rng.integers(-3, 4, (N, K)).astype(np.float16)
    ref = a.astype(np.int64) @ w.astype(np.int64).T
    assert np.abs(ref).max() <= 2048
    assert np.array_equal(g9.hgemm(a, w.T).astype(np.int64), ref), "host"
    Wd = g9.hgemm(_dev(torch_dev, a), _dev(torch_dev, w).t())
    assert np.array_equal(Wd.cpu().numpy().astype(np.int64), ref), "device"
    # role swap: C (N×M) = w·aᵀ takes the skinny path with a as the streamed operand and C written column-wise
    assert np.array_equal(g9.hgemm(w, a.T).astype(np.int64), ref.T), "small N"
    # alpha/beta into a slice of a larger array; nothing outside it changes
    big = rng.uniform(-1, 1, (M + 3, N + 4)).astype(np.float16)
    D0 = big.copy()
    C = big[2:M + 2, 1:N + 1]
    C0 = C.astype(np.float64)
    g9.hgemm(a, w.T, alpha=0.5, beta=-2.0, C=C)
    r64 = 0.5 * ref - 2.0 * C0
    scale = 0.5 * (np.abs(a.astype(np.float64)) @ np.abs(w.astype(np.float64)).T) + 2.0 * np.abs(C0)
    assert float(np.max(np.abs(C.astype(np.float64) - r64) / scale)) <= 2e-3
    mask = np.ones(big.shape, bool)
    mask[2:M + 2, 1:N + 1] = False
    assert np.array_equal(big[mask], D0[mask]), "write outside the C slice"


def test_skinny_forced_threshold(g9):
    """GEN9BLAS_SKINNY=64, as the reference's skinny test forces it (reference: lib/test_skinny.py:14, 43-44): every
    product with min(M, N) ≤ 64 takes a skinny kernel, so M = 17, 33, 64 (and the role-swapped small N) run in M
    tiles of 16 rows (grid.y > 1), on both the dot-product kernel and, for K a multiple of 256, the FP16 matrix-core
    kernel. All of the reference test's cases against float64 (tests/skinny_forced_child.py). The variable is read
    once per process, so the cases run in a child process (one more GPU process, sequential)."""
    import os
    import subprocess
    import sys
    env = dict(os.environ, GEN9BLAS_SKINNY="64")
    child = os.path.join(os.path.dirname(os.path.realpath(__file__)), "skinny_forced_child.py")
    r = subprocess.run([sys.executable, "-u", child], env=env, capture_output=True, text=True, timeout=110)
    print(r.stdout[-3000:])
    assert r.returncode == 0, (r.stdout[-3000:], r.stderr[-2000:])
    assert "failed 0" in r.stdout
