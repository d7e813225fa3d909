"""Run-twice bit identity of the hot-path calls on the GPU.

The reference's golden tool runs every seeded call twice and flags a call whose two results differ
(reference: tools/golden/blas_golden.py:29-61). Here each call below runs twice on the same inputs, with other
work between the two runs (a different product, so the work buffers and caches hold other data), and the result
bytes must be identical: GEMM in every type on the whole-tile kernels, the general kernel, split-K and the
two-k-group tiles (the benchmarked shapes included: FP16 n = 1024/2048/4096 in both modes, FP32 n = 4096 and the odd
3000×11008×4096 product with beta, FP64 n = 1024), the skinny kernels at M = 1..16, SDOT at 2^26 and SGEMV N/T at
16384², the skinny products with weights stored K×N, SYMV / TRMV / TRSV at n = 16384, plus the level-3 calls on
the GEMM kernels. Sums are in fixed order everywhere (split-K slices added in index
order, FP64 reduction partials summed by one block), so nothing may depend on timing.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _data(torch, seed, shape, dt):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(shape, generator=g, device="cuda", dtype=torch.float32).to(dt)


def _same(a, b):
    a, b = a.contiguous(), b.contiguous()
    return a.shape == b.shape and bool(torch_equal_bytes(a, b))


def torch_equal_bytes(a, b):
    import torch
    if a.dtype == torch.float16:
        return torch.equal(a.view(torch.int16), b.view(torch.int16))
    if a.dtype == torch.float32:
        return torch.equal(a.view(torch.int32), b.view(torch.int32))
    return torch.equal(a.view(torch.int64), b.view(torch.int64))


# (label, dtype name, M, N, K, transposed B, alpha, beta, accurate)
GEMMS = [
    ("hgemm n=4096", "f16", 4096, 4096, 4096, False, 1.0, 0.0, False),
    ("hgemm accurate n=4096", "f16", 4096, 4096, 4096, False, 1.0, 0.0, True),
    ("hgemm n=2048", "f16", 2048, 2048, 2048, False, 1.0, 0.0, False),
    ("hgemm accurate n=1024", "f16", 1024, 1024, 1024, False, 1.0, 0.0, True),
    ("hgemm general 1000x600x1000 beta", "f16", 1000, 600, 1000, True, 0.5, 2.0, False),
    ("hgemm split-K 200x136x1000", "f16", 200, 136, 1000, False, 1.0, 0.0, False),
    ("sgemm n=4096", "f32", 4096, 4096, 4096, False, 1.0, 0.0, False),
    ("sgemm odd 3000x11008x4096 tB beta", "f32", 3000, 11008, 4096, True, 1.0, 0.5, False),
    ("sgemm n=1024", "f32", 1024, 1024, 1024, False, 1.0, 0.0, False),
    ("sgemm split-K 130x260x4096", "f32", 130, 260, 4096, False, 1.0, 0.0, False),
    ("dgemm n=1024", "f64", 1024, 1024, 1024, False, 1.0, 0.0, False),
    ("dgemm 2048 small tiles", "f64", 2048, 2048, 2048, False, 1.0, 0.0, False),
    ("hgemm general split-K 2048x4096x1000", "f16", 2048, 4096, 1000, False, 1.0, 0.0, False),
    ("dgemm 640x640x1024 tB beta", "f64", 640, 640, 1024, True, -1.0, 0.25, False),
]


@pytest.mark.parametrize("case", GEMMS, ids=[c[0] for c in GEMMS])
def test_gemm_twice(g9, torch_dev, case):
    torch = torch_dev
    label, dn, M, N, K, tB, alpha, beta, acc = case
    dt = {"f16": torch.float16, "f32": torch.float32, "f64": torch.float64}[dn]
    A = _data(torch, 1, (M, K), dt)
    B = _data(torch, 2, (N, K) if tB else (K, N), dt)
    C0 = _data(torch, 3, (M, N), dt)
    Bop = B.t() if tB else B
    outs = []
    for rep in range(2):
        C = C0.clone()
        g9.gemm(A, Bop, alpha=alpha, beta=beta, C=C, accurate=acc)
        # other work in between: a different product through the same dispatch
        g9.gemm(B[:64, :64].contiguous(), A[:64, :64].contiguous(), accurate=acc)
        torch.cuda.synchronize()
        outs.append(C)
    assert _same(*outs), label + ": two runs differ"


@pytest.mark.parametrize("M", [1, 2, 4, 8, 16])
def test_skinny_twice(g9, torch_dev, M):
    """C = A·Wᵀ at W 4096² FP16 (the benchmarked skinny configuration), both roles (M×4096 and 4096×M)."""
    torch = torch_dev
    W = _data(torch, 100, (4096, 4096), torch.float16) * 0.02
    A = _data(torch, 7, (M, 4096), torch.float16)
    first, second = [], []
    for out in (first, second):
        out.append(g9.gemm(A, W.t()))
        out.append(g9.gemm(W, A.t()))
        g9.gemm(W[:M].contiguous(), W.t())
        torch.cuda.synchronize()
    for a, b in zip(first, second):
        assert _same(a, b), f"skinny M={M}: two runs differ"


@pytest.mark.parametrize("M", [1, 4, 16])
def test_skinny_weights_k_by_n_twice(g9, torch_dev, M):
    """C = A·W with W stored K×N (4096² FP16, the split-K matrix-core form and its fixed-order sum), and with a
    transposed small operand (gathered first): same bytes twice."""
    torch = torch_dev
    W = _data(torch, 101, (4096, 4096), torch.float16) * 0.02
    A = _data(torch, 8, (M, 4096), torch.float16)
    At = _data(torch, 9, (4096, M), torch.float16)
    first, second = [], []
    for out in (first, second):
        out.append(g9.gemm(A, W))
        out.append(g9.gemm(At.t(), W))
        g9.gemm(W[:M].contiguous(), W)
        torch.cuda.synchronize()
    for a, b in zip(first, second):
        assert _same(a, b), f"skinny K×N M={M}: two runs differ"


def test_level2_partials_twice(g9, torch_dev):
    """SYMV and TRMV (per-row and per-column partials summed in a fixed order by a second kernel) and TRSV on inverted
    blocks at n = 16384 FP32: same bytes twice."""
    torch = torch_dev
    n = 16384
    A = _data(torch, 30, (n, n), torch.float32) / 128
    A.diagonal().add_(4.0)
    v = _data(torch, 31, n, torch.float32)
    calls = [("symv L", lambda: g9.symv(A, v, uplo="L")), ("symv U", lambda: g9.symv(A, v, uplo="U")),
             ("trmv LT", lambda: g9.trmv(A, v.clone(), uplo="L", trans=True)),
             ("trsv LN", lambda: g9.trsv(A, v.clone(), uplo="L")),
             ("trsv UT", lambda: g9.trsv(A, v.clone(), uplo="U", trans=True))]
    for name, fn in calls:
        r1 = fn()
        g9.symv(A[:300, :300], v[:300])
        torch.cuda.synchronize()
        r2 = fn()
        torch.cuda.synchronize()
        assert _same(r1, r2), f"{name}: two runs differ"


def test_level12_twice(g9, torch_dev):
    """SDOT (2^26) returns the same float64 both times; SGEMV N and T at 16384² and SAXPY write the same bytes."""
    torch = torch_dev
    n = 1 << 26
    x, y = _data(torch, 20, n, torch.float32), _data(torch, 21, n, torch.float32)
    d = [g9.dot(x, y) for _ in range(2)]
    assert d[0] == d[1], f"sdot: {d[0]!r} then {d[1]!r}"
    m = 16384
    A = _data(torch, 22, (m, m), torch.float32)
    v = _data(torch, 23, m, torch.float32)
    for trans in (False, True):
        r = []
        for _ in range(2):
            r.append(g9.gemv(A, v, trans=trans))
            g9.gemv(A[:100, :100], v[:100], trans=not trans)
        torch.cuda.synchronize()
        assert _same(*r), f"sgemv trans={trans}: two runs differ"
    ys = [y.clone(), y.clone()]
    for t in ys:
        g9.axpy(0.75, x, t)
    torch.cuda.synchronize()
    assert _same(*ys), "saxpy: two runs differ"


@pytest.mark.parametrize("dn", ["f32", "f64"])
def test_level3_twice(g9, torch_dev, dn):
    """SYMM, SYRK, SYR2K, TRMM, TRSM at n = 1000 on the GEMM kernels: same bytes twice."""
    torch = torch_dev
    dt = torch.float32 if dn == "f32" else torch.float64
    n = 1000
    A = _data(torch, 4, (n, n), dt)
    B = _data(torch, 5, (n, 700), dt)
    T = torch.tril(A) * 0.01 + 2 * torch.eye(n, device="cuda", dtype=dt)
    calls = [("symm", lambda: g9.symm(A, B)), ("syrk", lambda: g9.syrk(B)), ("syr2k", lambda: g9.syr2k(B, B * 0.5)),
             ("trmm", lambda: g9.trmm(T, B.clone())), ("trsm", lambda: g9.trsm(T, B.clone()))]
    for name, fn in calls:
        r1 = fn()
        torch.cuda.synchronize()
        r2 = fn()
        torch.cuda.synchronize()
        assert _same(r1, r2), f"{name} {dn}: two runs differ"


def test_host_operands_twice(g9):
    """The staged path (NumPy operands: pinned ring, row panels for a 32 MiB C) gives the same bytes twice."""
    rng = np.random.default_rng(9)
    A = rng.standard_normal((4096, 1024)).astype(np.float16)
    B = rng.standard_normal((1024, 4096)).astype(np.float16)
    r = [g9.gemm(A, B) for _ in range(2)]
    assert np.array_equal(r[0].view(np.int16), r[1].view(np.int16))
