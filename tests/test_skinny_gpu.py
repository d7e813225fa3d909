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
    ref = (a.astype(np.float64) @ w.astype(np.float64).T).astype(np.int64)
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


# (M, N, K): weights stored K×N (N-contiguous), shapes for the FP16 matrix-core form (K a multiple of 64, N ≥ 64 and
# a multiple of 8: 64-column strips, the last one shifted back to end at N, K split in 1, 2 or 4 parts) and for the
# vector form (K or N off those multiples, N below 64, and FP32)
KN_SHAPES = [(1, 4096, 512), (2, 264, 256), (3, 77 * 8, 768), (4, 2056, 1024), (7, 16, 256), (8, 520, 2048),
             (12, 1000, 512), (16, 4096, 256), (16, 24, 4096), (1, 1000, 777), (5, 333, 300), (16, 9, 513),
             (2, 4100, 1000)]


@pytest.mark.parametrize("M,N,K", KN_SHAPES)
def test_skinny_weights_n_contiguous(g9, torch_dev, M, N, K):
    """C = a·W with W stored K×N (row-major x·W), the layout the reference sends to skinny_n4 / skinny_n2
    (reference: lib/src/gemm.c:246-261). Small integers make every product and sum exact, so FP16 (matrix-core form
    where the shape allows it, the vector form elsewhere) and FP32 (vector form) must be bit-exact; also the role swap
    (C = Wᵀ·aᵀ with op(A) = Wᵀ: the weights become the transposed A), a transposed a (gathered first), and alpha/beta
    into a slice of a larger C with nothing outside it written."""
    rng = np.random.default_rng(M * 131 + N + K)
    for dt in (np.float16, np.float32):
        fn = g9.hgemm if dt == np.float16 else g9.sgemm
        a = rng.integers(-3, 4, (M, K)).astype(dt)
        w = rng.integers(-3, 4, (K, N)).astype(dt)
        ref = (a.astype(np.float64) @ w.astype(np.float64)).astype(np.int64)
        assert np.abs(ref).max() <= 2048 or dt == np.float32
        tag = f"{np.dtype(dt).name} M={M} N={N} K={K}"
        assert np.array_equal(fn(a, w).astype(np.int64), ref), tag + " host"
        got = fn(_dev(torch_dev, a), _dev(torch_dev, w)).cpu().numpy()
        assert np.array_equal(got.astype(np.int64), ref), tag + " device"
        assert np.array_equal(fn(w.T, a.T).astype(np.int64), ref.T), tag + " small N (weights as transposed A)"
        at = np.ascontiguousarray(a.T)   # a stored K×M: op(A) = atᵀ has a k stride
        assert np.array_equal(fn(at.T, w).astype(np.int64), ref), tag + " transposed a"
        big = rng.uniform(-1, 1, (M + 2, N + 3)).astype(dt)
        D0 = big.copy()
        C = big[1:M + 1, 3:N + 3]
        C0 = C.astype(np.float64)
        fn(a, w, alpha=0.5, beta=-2.0, C=C)
        r64 = 0.5 * ref - 2.0 * C0
        scale = 0.5 * (np.abs(a.astype(np.float64)) @ np.abs(w.astype(np.float64))) + 2.0 * np.abs(C0)
        assert float(np.max(np.abs(C.astype(np.float64) - r64) / scale)) <= (2e-3 if dt == np.float16 else 1e-6), tag
        mask = np.ones(big.shape, bool)
        mask[1:M + 1, 3:N + 3] = False
        assert np.array_equal(big[mask], D0[mask]), tag + ": write outside the C slice"


@pytest.mark.parametrize("M", [1, 2, 4, 8, 16])
def test_skinny_decode_4096_weights_k_by_n(g9, orc, torch_dev, M):
    """The decode shape with W stored K×N (4096², ~N(0, 0.02)) on device memory, as the benchmark runs it: against
    float64 with the skinny bound and the reference metric, and equal to the same product with the weights stored
    N×K to within FP16 rounding and the FP32 summation bound (both sum the same exact products, in different
    orders)."""
    torch = torch_dev
    K = N = 4096
    A = orc.normal((M, K), np.float16, orc.SEED_A)
    Ad = _dev(torch, A)
    for i in range(2):
        Wt = orc.normal((N, K), np.float16, orc.SEED_W0 + i, 0.02)   # N×K as in the K-contiguous case
        W = np.ascontiguousarray(Wt.T)                                 # stored K×N
        C = g9.hgemm(Ad, _dev(torch, W)).cpu().numpy()
        ref = A.astype(np.float64) @ W.astype(np.float64)
        assert _err(C, ref) <= TOL[np.float16], f"M={M} copy {i}"
        scale = np.abs(A.astype(np.float64)) @ np.abs(W.astype(np.float64))
        assert float(np.max(np.abs(C - ref) / scale)) <= 1e-3, f"M={M} copy {i}: reference metric"
        Ck = g9.hgemm(Ad, _dev(torch, Wt).t()).cpu().numpy()
        # each result is an FP32 sum of the same exact products, rounded once to FP16: they differ by at most one FP16
        # ulp plus the two summation orders' error bounds, 2·K·2^-24·Σ|a·w|
        c64, k64 = C.astype(np.float64), Ck.astype(np.float64)
        bound = 2.0 ** -10 * np.maximum(np.abs(c64), np.abs(k64)) + 2 * K * 2.0 ** -24 * scale + 2.0 ** -24
        assert (np.abs(c64 - k64) <= bound).all(), f"M={M}: layouts differ"


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
