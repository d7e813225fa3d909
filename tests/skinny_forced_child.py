"""Child process of test_skinny_gpu.py::test_skinny_forced_threshold: runs with GEN9BLAS_SKINNY=64 in its environment
(read once, when the library first dispatches), so every product with min(M, N) ≤ 64 takes a skinny kernel, in every
layout, M tiles of 16 rows included.

Cases follow the reference's skinny test (reference: lib/test_skinny.py:38-63): its shapes (M = 17, 33, 64 beyond the
default threshold), both weight layouts and transposed views, the role swap for small N, alpha/beta into a slice of a
larger C with nothing written outside it, host (pageable and pinned) and device memory, FP16 and FP32. Two more shapes
with K a multiple of 256 put M > 16 on the FP16 matrix-core kernel (several M tiles). Bound: max|C − ref| / max|ref|
against float64, 4e-3 (FP16) and 2e-6 (FP32) (lib/test_skinny.py:19, 29-35). Prints one line per failure and a final
"checked N" line; exits 1 on any failure."""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.realpath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "gen9-gpu-blas_amd"))
import gen9blas  # noqa: E402
import torch  # noqa: E402

assert os.environ.get("GEN9BLAS_SKINNY") == "64"
TOL = {np.float16: 4e-3, np.float32: 2e-6}
SHAPES = [(1, 1000, 777), (3, 517, 1029), (4, 2048, 128), (5, 64, 9), (8, 333, 4096), (9, 1500, 1500),
          (16, 4096, 1000), (17, 130, 257), (33, 700, 300), (64, 256, 513), (1, 8, 3), (2, 7, 2000),
          (40, 1000, 512), (64, 2048, 1024)]
rng = np.random.default_rng(7)
failures, checked = [], 0


def err(W, ref):
    W = W.cpu().numpy() if hasattr(W, "cpu") else np.asarray(W)
    return float(np.max(np.abs(W.astype(np.float64) - ref)) / max(1e-30, np.max(np.abs(ref))))


def check(tag, dt, W, ref):
    global checked
    checked += 1
    e = err(W, ref)
    if not np.isfinite(e) or e > TOL[dt]:
        failures.append(f"{tag}: error {e:.2e}")


def mem(x, where):
    if where == "device":
        return torch.from_numpy(np.ascontiguousarray(x)).cuda()
    if where == "pinned":
        y = gen9blas.empty(x.shape, x.dtype)
        y[...] = x
        return y
    return x


def T(x):
    return x.t() if hasattr(x, "t") else x.T


for dt in (np.float16, np.float32):
    fn = gen9blas.hgemm if dt == np.float16 else gen9blas.sgemm
    for where in ("pageable", "pinned", "device"):
        for M, N, K in SHAPES:
            for tA in (False, True):
                for tB in (False, True):
                    a = rng.uniform(-1, 1, (K, M) if tA else (M, K)).astype(dt)
                    b = rng.uniform(-1, 1, (N, K) if tB else (K, N)).astype(dt)
                    A_, B_ = mem(a, where), mem(b, where)
                    A, B = (T(A_) if tA else A_), (T(B_) if tB else B_)
                    ref = (a.T if tA else a).astype(np.float64) @ (b.T if tB else b).astype(np.float64)
                    tag = f"{np.dtype(dt).name} {where} M={M} N={N} K={K} tA={tA} tB={tB}"
                    check(tag, dt, fn(A, B), ref)
                    check(tag + " (small N)", dt, fn(T(B), T(A)), ref.T)
            a = rng.uniform(-1, 1, (M, K)).astype(dt)
            w = rng.uniform(-1, 1, (N, K)).astype(dt)
            big = rng.uniform(-1, 1, (M + 2, N + 5)).astype(dt)
            keep = big.copy()
            ref = 0.75 * a.astype(np.float64) @ w.astype(np.float64).T - 1.5 * big[1:M + 1, 2:N + 2].astype(np.float64)
            B_ = mem(big, where)
            fn(mem(a, where), T(mem(w, where)), alpha=0.75, beta=-1.5, C=B_[1:M + 1, 2:N + 2])
            got = B_.cpu().numpy() if where == "device" else np.asarray(B_)
            tag = f"{np.dtype(dt).name} {where} M={M} N={N} K={K} alpha/beta into a C slice"
            check(tag, dt, got[1:M + 1, 2:N + 2], ref)
            mask = np.ones(big.shape, bool)
            mask[1:M + 1, 2:N + 2] = False
            if not np.array_equal(got[mask], keep[mask]):
                failures.append(tag + ": write outside the slice")

for f in failures:
    print("FAIL", f)
print(f"checked {checked}, failed {len(failures)}", flush=True)
sys.exit(1 if failures else 0)
