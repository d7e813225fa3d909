"""gen9blas_gemm_noalloc (the GEMM entry point that allocates nothing) against gen9blas_gemm, through the C ABI.

Same kernels and dispatch as gen9blas_gemm, so on the same device operands the results must be identical, bit for
bit: products that take split-K (whose slices then live in the entry point's static work space), the two-k-group
tiles and the whole-tile FP16 kernel, in every type, two calls in a row with the second smaller (the work space
keeps the last call's contents; a split-K slice writes every element it is later read at). The largest default
splits are included: FP16 2048×4096×1000 (128 general-kernel tiles of 256×256 split two ways: the whole 64 MiB),
FP64 640×640×1024 (split four ways) and FP16
1280×1280×1000 on the general kernel. Skinny products whose gathered operand and partial sums live in that work
space are included too. Both are also held to the GEMM bounds against float64. Host operands (checked
before any dispatch, so the staging paths never run) and a work space beyond the fixed maximum give INVALID_ARG
before any launch (the latter needs a split forced with GEN9BLAS_SPLITK, read once per process: a child process).
A fresh child process checks the property itself: the free device memory does not move across no-alloc calls,
while one gen9blas_gemm of the same product grows the library's buffers."""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

INVALID = -3
CODE = {"H": 0, "S": 1, "HS": 2, "D": 3}
DT = {"H": np.float16, "HS": np.float16, "S": np.float32, "D": np.float64}
BOUND = {"H": 2e-3, "HS": 5e-3, "S": 1e-6, "D": 1e-13}


def _sig(L):
    i, d, p = ctypes.c_int, ctypes.c_double, ctypes.c_void_p
    for name in ("gen9blas_gemm", "gen9blas_gemm_noalloc"):
        getattr(L, name).argtypes = [i, i, i, i, i, i, d, p, i, p, i, d, p, i]
        getattr(L, name).restype = i
    return L


def _run(L, torch, name, kind, tA, tB, M, N, K, alpha, beta, a, b, c0):
    dev = [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in (a, b, c0)]
    lda = M if tA else K
    ldb = K if tB else N
    rc = getattr(L, name)(CODE[kind], tA, tB, M, N, K, alpha, dev[0].data_ptr(), lda, dev[1].data_ptr(), ldb, beta,
                          dev[2].data_ptr(), N)
    assert rc == 0, (name, L.gen9blas_error())
    torch.cuda.synchronize()
    return dev[2].cpu().numpy()


def _err(W, opA, opB, alpha, beta, c0):
    a, b, c = (x.astype(np.float64) for x in (opA, opB, c0))
    ref = alpha * (a @ b) + beta * c
    scale = abs(alpha) * (np.abs(a) @ np.abs(b)) + abs(beta) * np.abs(c)
    return float(np.max(np.abs(W.astype(np.float64) - ref) / scale))


# (M, N, K, tA, tB): split-K products (few small tiles), then products that take the two-k-group tiles and the
# whole-tile FP16 kernel; each pair of rows is one call followed by a smaller one
CASES = [((200, 136, 1000, 0, 0), (100, 72, 500, 1, 1)),
         ((130, 260, 4096, 1, 0), (64, 64, 777, 0, 1)),
         ((1024, 1024, 512, 0, 0), (512, 384, 256, 0, 1))]
# skinny products (min(M, N) ≤ 16) that use the work space: weights stored K×N (FP16: K split in 4 parts, partial
# sums in the work space) and a transposed small operand (gathered into the work space), the second call smaller
SKINNY = [((4, 4096, 4096, 0, 0), (16, 2048, 1024, 1, 0)),
          ((4096, 8, 2048, 0, 0), (1000, 3, 512, 1, 1))]
# the largest default work spaces: 64 MiB (FP16 2048×4096×1000), then 12.5 MiB (FP64 640×640×1024, FP16
# 1280×1280×1000); FP64 2048³, whose big tiles are half the CUs, takes the small tiles instead of a split
LARGE = {"D": ((2048, 2048, 2048, 0, 0), (640, 640, 1024, 1, 0)),
         "H": ((2048, 4096, 1000, 0, 0), (1280, 1280, 1000, 0, 1)),
         "HS": ((1280, 1280, 1000, 1, 1), (1000, 600, 1000, 0, 0))}


def _compare(g9, torch_dev, kind, shapes, seed):
    L = _sig(g9._lib)
    rng = np.random.default_rng(seed)
    dt = DT[kind]
    for (M, N, K, tA, tB) in shapes:
        a = rng.uniform(-1, 1, (K, M) if tA else (M, K)).astype(dt)
        b = rng.uniform(-1, 1, (N, K) if tB else (K, N)).astype(dt)
        c0 = rng.uniform(-1, 1, (M, N)).astype(dt)
        W0 = _run(L, torch_dev, "gen9blas_gemm", kind, tA, tB, M, N, K, 1.5, 0.5, a, b, c0)
        W1 = _run(L, torch_dev, "gen9blas_gemm_noalloc", kind, tA, tB, M, N, K, 1.5, 0.5, a, b, c0)
        tag = f"{kind} {M}x{N}x{K} tA={tA} tB={tB}"
        assert np.array_equal(W0, W1), tag + ": no-alloc result differs from gen9blas_gemm"
        opA, opB = (a.T if tA else a), (b.T if tB else b)
        assert _err(W1, opA, opB, 1.5, 0.5, c0) <= BOUND[kind], tag


@pytest.mark.parametrize("kind", ["S", "D", "H", "HS"])
@pytest.mark.parametrize("pair", range(len(CASES)))
def test_noalloc_matches_gemm(g9, torch_dev, kind, pair):
    _compare(g9, torch_dev, kind, CASES[pair], 40 + pair)


@pytest.mark.parametrize("kind", ["S", "H", "HS"])
@pytest.mark.parametrize("pair", range(len(SKINNY)))
def test_noalloc_skinny(g9, torch_dev, kind, pair):
    _compare(g9, torch_dev, kind, SKINNY[pair], 60 + pair)


@pytest.mark.parametrize("kind", sorted(LARGE))
def test_noalloc_largest_work_space(g9, torch_dev, kind):
    _compare(g9, torch_dev, kind, LARGE[kind], 50)


def test_noalloc_rejects_host_operands(g9):
    L = _sig(g9._lib)
    a = np.ones((64, 64), np.float32)
    c = np.zeros((64, 64), np.float32)
    rc = L.gen9blas_gemm_noalloc(1, 0, 0, 64, 64, 64, 1.0, a.ctypes.data, 64, a.ctypes.data, 64, 0.0, c.ctypes.data, 64)
    assert rc == INVALID and b"device operands only" in L.gen9blas_error()
    assert (c == 0).all()


CHILD = r"""
import ctypes, sys, numpy as np, torch
sys.path.insert(0, sys.argv[1])
import gen9blas as g
L = g._lib
i, d, p = ctypes.c_int, ctypes.c_double, ctypes.c_void_p
L.gen9blas_gemm_noalloc.argtypes = [i, i, i, i, i, i, d, p, i, p, i, d, p, i]
n, K = 1024, 4096
a = torch.ones((n, K), dtype=torch.float32, device="cuda")
b = torch.ones((K, n), dtype=torch.float32, device="cuda")
c = torch.zeros((n, n), dtype=torch.float32, device="cuda")
rc = L.gen9blas_gemm_noalloc(1, 0, 0, n, n, K, 1.0, a.data_ptr(), K, b.data_ptr(), n, 0.0, c.data_ptr(), n)
msg = L.gen9blas_error().decode()
torch.cuda.synchronize()
untouched = bool((c == 0).all())
rc2 = L.gen9blas_gemm(1, 0, 0, n, n, K, 1.0, a.data_ptr(), K, b.data_ptr(), n, 0.0, c.data_ptr(), n)
torch.cuda.synchronize()
print(rc, untouched, rc2, bool((c == K).all()), msg)
"""


def test_noalloc_rejects_work_space_beyond_maximum(g9, tmp_path):
    """GEN9BLAS_SPLITK=64 on 1024² × 4096 FP32 needs 64 slices × 4 MiB of work space, beyond the 64 MiB maximum: the
    no-alloc call fails with INVALID_ARG and writes nothing; gen9blas_gemm (growing buffers) computes it."""
    script = tmp_path / "child.py"
    script.write_text(CHILD)
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.realpath(__file__))), "gen9-gpu-blas_amd")
    env = dict(os.environ, GEN9BLAS_SPLITK="64")
    r = subprocess.run([sys.executable, str(script), pkg], env=env, capture_output=True, text=True, timeout=100)
    assert r.returncode == 0, r.stderr[-2000:]
    rc, untouched, rc2, right = r.stdout.split()[:4]
    assert int(rc) == INVALID and untouched == "True", r.stdout
    assert "fixed maximum" in r.stdout
    assert int(rc2) == 0 and right == "True", r.stdout


FRESH = r"""
import ctypes, sys, numpy as np, torch
sys.path.insert(0, sys.argv[1])
import gen9blas as g
L = g._lib
i, d, p = ctypes.c_int, ctypes.c_double, ctypes.c_void_p
for name in ("gen9blas_gemm", "gen9blas_gemm_noalloc"):
    getattr(L, name).argtypes = [i, i, i, i, i, i, d, p, i, p, i, d, p, i]
assert L.gen9blas_init() == 0
dt = {0: torch.float16, 2: torch.float16, 3: torch.float64, 1: torch.float32}
cases = [(0, 2048, 4096, 1000), (3, 2048, 2048, 2048), (0, 1280, 1280, 1000), (2, 1280, 1280, 1000), (3, 640, 640, 1024), (1, 200, 136, 1000)]
bufs = [[torch.randn(s, dtype=dt[t], device="cuda") for s in ((M, K), (K, N), (M, N))] for (t, M, N, K) in cases]
small = [torch.ones((64, 64), dtype=torch.float32, device="cuda") for _ in range(3)]
def call(name, t, M, N, K, a, b, c):
    rc = getattr(L, name)(t, 0, 0, M, N, K, 1.0, a.data_ptr(), K, b.data_ptr(), N, 0.0, c.data_ptr(), N)
    assert rc == 0, (name, t, M, N, K, L.gen9blas_error())
call("gen9blas_gemm_noalloc", 1, 64, 64, 64, *small)   # warm-up: a product without split-K
torch.cuda.synchronize()
free0 = torch.cuda.mem_get_info()[0]
for k in range(2):
    for (t, M, N, K), (a, b, c) in zip(cases, bufs):
        call("gen9blas_gemm_noalloc", t, M, N, K, a, b, c)
torch.cuda.synchronize()
free1 = torch.cuda.mem_get_info()[0]
t, M, N, K = cases[0]
call("gen9blas_gemm", t, M, N, K, *bufs[0])
torch.cuda.synchronize()
free2 = torch.cuda.mem_get_info()[0]
# a pageable C of 32 MiB (the size that takes the row-panel staging in gen9blas_gemm) next to device A and B
a = torch.randn((4096, 4096), dtype=torch.float16, device="cuda")
ch = np.zeros((4096, 4096), np.float16)
rc = L.gen9blas_gemm_noalloc(0, 0, 0, 4096, 4096, 4096, 1.0, a.data_ptr(), 4096, a.data_ptr(), 4096, 0.0,
                             ch.ctypes.data, 4096)
msg = L.gen9blas_error().decode()
untouched = bool((ch == 0).all())
# afterwards gen9blas_gemm on host buffers (row panels through the pinned ring) still computes correctly
rng = np.random.default_rng(5)
ah = rng.integers(-2, 3, (4096, 256)).astype(np.float16)
bh = rng.integers(-2, 3, (256, 2048)).astype(np.float16)
ch2 = np.zeros((4096, 2048), np.float16)
rc2 = L.gen9blas_gemm(0, 0, 0, 4096, 2048, 256, 1.0, ah.ctypes.data, 256, bh.ctypes.data, 2048, 0.0,
                      ch2.ctypes.data, 2048)
exact = bool(np.array_equal(ch2.astype(np.float64), ah.astype(np.float64) @ bh.astype(np.float64)))
print(free0 - free1, free1 - free2, rc, untouched, rc2, exact, "|", msg)
"""


def test_noalloc_allocates_nothing(g9, tmp_path):
    """In a fresh process: after one warm-up call, no-alloc calls that use the whole 64 MiB work space (and smaller
    ones) leave the free device memory where it was, while one gen9blas_gemm of the largest product takes at least
    64 MiB for its split-K buffer. A pageable 32 MiB C next to device A and B gives INVALID_ARG, writes nothing, and
    leaves the host staging paths working for the next gen9blas_gemm (exact on small integers)."""
    script = tmp_path / "fresh.py"
    script.write_text(FRESH)
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.realpath(__file__))), "gen9-gpu-blas_amd")
    env = {k: v for k, v in os.environ.items() if not k.startswith("GEN9BLAS_")}
    r = subprocess.run([sys.executable, str(script), pkg], env=env, capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stderr[-2000:]
    fields = r.stdout.split("|")[0].split()
    d_noalloc, d_gemm, rc, untouched, rc2, exact = fields[:6]
    assert int(d_noalloc) < (2 << 20), f"free device memory fell by {d_noalloc} bytes across no-alloc calls"
    assert int(d_gemm) >= (64 << 20), f"gen9blas_gemm's split-K buffer not seen ({d_gemm} bytes)"
    assert int(rc) == INVALID and untouched == "True" and "device operands only" in r.stdout, r.stdout
    assert int(rc2) == 0 and exact == "True", r.stdout
