"""gen9blas_gemm_noalloc (the GEMM entry point that allocates nothing) against gen9blas_gemm, through the C ABI.

Same kernels and dispatch as gen9blas_gemm, so on the same device operands the results must be identical, bit for
bit: products that take split-K (whose slices then live in the entry point's static work space), the two-k-group
tiles and the whole-tile FP16 kernel, in every type, two calls in a row with the second smaller (the work space
keeps the last call's contents; a split-K slice writes every element it is later read at). Both are also held to the
GEMM bounds against float64. Host operands and a work space beyond the fixed maximum give INVALID_ARG before any
launch (the latter needs a split forced with GEN9BLAS_SPLITK, read once per process: a child process)."""
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


@pytest.mark.parametrize("kind", ["S", "D", "H", "HS"])
@pytest.mark.parametrize("pair", range(len(CASES)))
def test_noalloc_matches_gemm(g9, torch_dev, kind, pair):
    L = _sig(g9._lib)
    rng = np.random.default_rng(40 + pair)
    dt = DT[kind]
    for (M, N, K, tA, tB) in CASES[pair]:
        a = rng.uniform(-1, 1, (K, M) if tA else (M, K)).astype(dt)
        b = rng.uniform(-1, 1, (N, K) if tB else (K, N)).astype(dt)
        c0 = rng.uniform(-1, 1, (M, N)).astype(dt)
        W0 = _run(L, torch_dev, "gen9blas_gemm", kind, tA, tB, M, N, K, 1.5, 0.5, a, b, c0)
        W1 = _run(L, torch_dev, "gen9blas_gemm_noalloc", kind, tA, tB, M, N, K, 1.5, 0.5, a, b, c0)
        tag = f"{kind} {M}x{N}x{K} tA={tA} tB={tB}"
        assert np.array_equal(W0, W1), tag + ": no-alloc result differs from gen9blas_gemm"
        opA, opB = (a.T if tA else a), (b.T if tB else b)
        assert _err(W1, opA, opB, 1.5, 0.5, c0) <= BOUND[kind], tag


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
    """GEN9BLAS_SPLITK=64 on 1024² × 4096 FP32 needs 64 slices × 4 MiB of work space, beyond the 8 MiB maximum: the
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
