"""Child process of the long-launch and banding tests in test_gemm_gpu.py. GEN9BLAS_MAX_LAUNCH_MS and GEN9BLAS_SPLITK
are read once per process, so the parent runs this script once without and once with them.

    python long_launch_child.py cases  OUT.json    # the reference's long-launch sizes
    python long_launch_child.py layouts OUT.npz    # band offsets: transposed A, batches, every type

"cases" follows the reference's long-launch test (reference: lib/test_long_launch.py:26-58): inputs U(0, 1) from
seed 3 in pinned host memory (gen9blas.empty), DGEMM n = 4096, SGEMM n = 8192, accurate HGEMM n = 8192 and a batched
DGEMM 2 × 3072; max |C − ref| / |ref| against float64 over sampled rows. The rows are the reference's (first, middle,
last) plus both rows around every multiple of 256, since every band boundary is one. Writes {case: max error}.

"layouts" runs 1100×900×700 products with alpha = 1.5 and beta = 0.5 in FP32, FP64, FP16 (H) and FP16 (HS): A not
transposed and transposed (a band of op(A) is then a column range of the stored matrix), and a strided batch of 3
with both operands transposed, on device memory through gen9blas_gemm_batched. Writes every C and its error against
float64 (the reference metric |C − ref| / (|alpha|·Σ|a·b| + |beta·c|))."""
import ctypes
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.realpath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(HERE), "gen9-gpu-blas_amd"))
import gen9blas  # noqa: E402


def band_rows(n):
    rows = {0, n // 2, n - 1}
    for b in range(256, n, 256):
        rows.update((b - 1, b))
    return np.array(sorted(rows))


def rel_err_rows(C, A, B, rows):
    ref = A[..., rows, :].astype(np.float64) @ B.astype(np.float64)
    return float(np.max(np.abs(np.asarray(C)[..., rows, :].astype(np.float64) - ref) / np.abs(ref)))


def cases(out):
    rng = np.random.default_rng(3)

    def rand(shape, dt):
        X = gen9blas.empty(shape, dt)
        X[...] = rng.uniform(0, 1, shape)
        return X

    res = {}
    for name, dt, n in (("dgemm n=4096", np.float64, 4096), ("sgemm n=8192", np.float32, 8192),
                        ("hgemm accurate n=8192", np.float16, 8192)):
        A, B = rand((n, n), dt), rand((n, n), dt)
        C = gen9blas.gemm(A, B, accurate=(dt == np.float16))
        res[name] = rel_err_rows(C, A, B, band_rows(n))
        print(f"{name}: max rel err {res[name]:.2e}", flush=True)
        del A, B, C
        gen9blas.free_pool()
    A, B = rand((2, 3072, 3072), np.float64), rand((2, 3072, 3072), np.float64)
    C = gen9blas.gemm_batched(A, B)
    res["batched dgemm 2 x 3072"] = max(rel_err_rows(C[i], A[i], B[i], band_rows(3072)) for i in range(2))
    print(f"batched dgemm 2 x 3072: max rel err {res['batched dgemm 2 x 3072']:.2e}", flush=True)
    with open(out, "w") as f:
        json.dump(res, f)


def metric_err(W, opA, opB, alpha, beta, C0):
    a, b, c = opA.astype(np.float64), opB.astype(np.float64), C0.astype(np.float64)
    ref = alpha * (a @ b) + beta * c
    scale = abs(alpha) * (np.abs(a) @ np.abs(b)) + abs(beta) * np.abs(c)
    return float(np.max(np.abs(W.astype(np.float64) - ref) / scale))


def layouts(out):
    import torch
    rng = np.random.default_rng(4)
    M, N, K, al, be = 1100, 900, 700, 1.5, 0.5
    saved = {}
    for kind, dt in (("S", np.float32), ("D", np.float64), ("H", np.float16), ("HS", np.float16)):
        acc = kind == "HS"
        for ta in (0, 1):
            a = rng.uniform(-1, 1, (K, M) if ta else (M, K)).astype(dt)
            b = rng.uniform(-1, 1, (K, N)).astype(dt)
            c0 = rng.uniform(-1, 1, (M, N)).astype(dt)
            W = gen9blas.gemm(a.T if ta else a, b, al, be, c0.copy(), accurate=acc)
            key = f"{kind}_tA{ta}"
            saved[key] = W
            saved[key + "_err"] = metric_err(W, a.T if ta else a, b, al, be, c0)
        cnt = 3
        a = rng.uniform(-1, 1, (cnt, K, M)).astype(dt)      # stored K×M per matrix: op(A) = Aᵀ
        b = rng.uniform(-1, 1, (cnt, N, K)).astype(dt)      # stored N×K: op(B) = Bᵀ
        c0 = rng.uniform(-1, 1, (cnt, M, N)).astype(dt)
        Ad, Bd, Cd = (torch.from_numpy(x).cuda() for x in (a, b, c0))
        code = {"S": gen9blas.GEN9BLAS_S, "D": gen9blas.GEN9BLAS_D, "H": gen9blas.GEN9BLAS_H, "HS": gen9blas.GEN9BLAS_HS}
        rc = gen9blas._lib.gen9blas_gemm_batched(code[kind], 1, 1, M, N, K, al, ctypes.c_void_p(Ad.data_ptr()), M, K * M,
                                                 ctypes.c_void_p(Bd.data_ptr()), K, N * K, be,
                                                 ctypes.c_void_p(Cd.data_ptr()), N, M * N, cnt)
        assert rc == 0, gen9blas._lib.gen9blas_error()
        torch.cuda.synchronize()
        W = Cd.cpu().numpy()
        key = f"{kind}_batch"
        saved[key] = W
        saved[key + "_err"] = max(metric_err(W[i], a[i].T, b[i].T, al, be, c0[i]) for i in range(cnt))
        print(f"{kind}: errors {saved[kind + '_tA0_err']:.2e} {saved[kind + '_tA1_err']:.2e} "
              f"{saved[key + '_err']:.2e}", flush=True)
    np.savez(out, **saved)


if __name__ == "__main__":
    {"cases": cases, "layouts": layouts}[sys.argv[1]](sys.argv[2])
