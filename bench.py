"""Benchmark of the gen9blas hot path on one MI355X: SGEMM/HGEMM/DGEMM TFLOPS at n = 4096, skinny 4096² FP16 µs/call
and HBM GB/s, level 1/2 GB/s, each as a fraction of its roofline, with the reference's CPU path timed beside it.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--quick]

Prints ONE JSON line. `value` is HGEMM (GEN9BLAS_H) TFLOP/s at n = 4096 (NN, alpha = 1, beta = 0, inputs resident in
HBM); every other configuration of BASELINE.json is in `results`. A step is one library call on one configuration;
timed with HIP events recorded on the library's own stream (the stream its kernels run on) around K back-to-back calls
after W warm-up calls, in no-wait mode (device operands, no host synchronization per call).
Inputs: np.random.default_rng seeds A = 1, B = 2, C = 3, W copies 100..131, x = 20, y = 21 (synthetic, BASELINE §8d).
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.realpath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gen9-gpu-blas_amd"))

PEAK_TFLOPS = {"H": 2516.6, "HS": 2516.6, "S": 157.3, "D": 78.6}   # MI355X dense MFMA (datasheet)
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--quick", action="store_true", help="HGEMM n=4096 and skinny only, no CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the GPU boxes of this build have one GPU and the library is single-device "
              "(multi-GPU sharding is design-only). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import gen9blas as g9
    g9._init()
    L = g9._lib
    stream = torch.cuda.ExternalStream(g9.hip_stream())
    steps, warm = args.steps, args.warmup
    dev = torch.device("cuda:0")
    p, i, d = ctypes.c_void_p, ctypes.c_int, ctypes.c_double

    def to_dev(x):
        return torch.from_numpy(np.ascontiguousarray(x)).to(dev)

    def timed(fn, k=steps, w=warm):
        """ms per call: HIP events on the library stream around k back-to-back calls after w warm-ups."""
        for _ in range(w):
            fn()
        g9.flush()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(k):
            fn()
        e1.record(stream)
        e1.synchronize()
        g9.flush()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / k

    g9.set_nowait(True)
    res = {}

    # ---------------- GEMM ----------------
    def gemm_case(kind, n=None, M=None, N=None, K=None, tB=0, beta=0.0):
        M, N, K = (n, n, n) if n else (M, N, K)
        dt = {"H": np.float16, "HS": np.float16, "S": np.float32, "D": np.float64}[kind]
        typ = {"H": 0, "HS": 2, "S": 1, "D": 3}[kind]
        if dt == np.float16:
            A = np.random.default_rng(1).standard_normal((M, K), dtype=np.float32).astype(dt)
            B = np.random.default_rng(2).standard_normal((N, K) if tB else (K, N), dtype=np.float32).astype(dt)
        else:
            A = np.random.default_rng(1).uniform(-1, 1, (M, K)).astype(dt)
            B = np.random.default_rng(2).uniform(-1, 1, (N, K) if tB else (K, N)).astype(dt)
        C = np.random.default_rng(3).uniform(-1, 1, (M, N)).astype(dt) if beta else np.zeros((M, N), dt)
        Ad, Bd, Cd = to_dev(A), to_dev(B), to_dev(C)
        del A, B, C
        args_ = (typ, 0, tB, M, N, K, d(1.0), p(Ad.data_ptr()), K, p(Bd.data_ptr()), K if tB else N, d(beta),
                 p(Cd.data_ptr()), N)

        def fn():
            rc = L.gen9blas_gemm(*args_)
            if rc:
                raise RuntimeError(L.gen9blas_error().decode())
        ms = timed(fn)
        tf = 2.0 * M * N * K / (ms * 1e-3) / 1e12
        del Ad, Bd, Cd
        return {"M": M, "N": N, "K": K, "ms": round(ms, 4), "tflops": round(tf, 2),
                "frac_of_peak": round(tf / PEAK_TFLOPS[kind], 4)}

    log("HGEMM n=4096 ...")
    res["hgemm_n4096"] = gemm_case("H", 4096)
    log(res["hgemm_n4096"])
    res["hgemm_accurate_n4096"] = gemm_case("HS", 4096)
    if not args.quick:
        for n in (1024, 2048):
            res[f"hgemm_n{n}"] = gemm_case("H", n)
            res[f"hgemm_accurate_n{n}"] = gemm_case("HS", n)
        log("SGEMM / DGEMM ...")
        res["sgemm_n1024"] = gemm_case("S", 1024)
        res["sgemm_n4096"] = gemm_case("S", 4096)
        res["dgemm_n1024"] = gemm_case("D", 1024)
        res["dgemm_n4096"] = gemm_case("D", 4096)
        res["sgemm_odd_3000x11008x4096_tB_beta05"] = gemm_case("S", M=3000, N=11008, K=4096, tB=1, beta=0.5)
        for k, v in res.items():
            log(k, v)

    # ---------------- measured HBM bandwidth: streaming read of 1 GiB (> 256 MB MALL) ----------------
    nh = 1 << 28
    big = torch.empty(nh, dtype=torch.float32, device=dev).uniform_(-1, 1)
    out_d = torch.zeros(1, dtype=torch.float64, device=dev)   # device result: no host wait per call
    out_p = ctypes.cast(ctypes.c_void_p(out_d.data_ptr()), ctypes.POINTER(ctypes.c_double))

    def rd():
        rc = L.gen9blas_asum(1, nh, p(big.data_ptr()), 1, out_p)
        if rc:
            raise RuntimeError(L.gen9blas_error().decode())
    ms = timed(rd, k=10, w=2)
    hbm = 4.0 * nh / (ms * 1e-3) / 1e9
    res["hbm_read_1GiB"] = {"kernel": "gen9blas_asum FP32 2^28 (pure streaming read)", "ms": round(ms, 4),
                            "GBs": round(hbm, 1), "frac_of_datasheet": round(hbm / PEAK_HBM_GBS, 4)}
    log(res["hbm_read_1GiB"])
    del big

    # ---------------- skinny C = A·Wᵀ, W 4096² fp16, 32 rotated copies ----------------
    log("skinny ...")
    K = N = 4096
    ncopy = 32
    Wd = torch.empty((ncopy, N, K), dtype=torch.float16, device=dev)
    for c in range(ncopy):
        w = np.random.default_rng(100 + c).standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
        Wd[c].copy_(torch.from_numpy(w.astype(np.float16)))
    sk = {}
    for M in (1, 2, 4, 8, 16):
        Ah = np.random.default_rng(1).standard_normal((M, K), dtype=np.float32).astype(np.float16)
        Ad = to_dev(Ah)
        Cd = torch.empty((M, N), dtype=torch.float16, device=dev)
        wp = [Wd[c].data_ptr() for c in range(ncopy)]
        state = {"j": 0}

        def fn():
            j = state["j"]
            state["j"] = (j + 1) % ncopy
            rc = L.gen9blas_gemm(0, 0, 1, M, N, K, d(1.0), p(Ad.data_ptr()), K, p(wp[j]), K, d(0.0), p(Cd.data_ptr()), N)
            if rc:
                raise RuntimeError(L.gen9blas_error().decode())
        ms = timed(fn, k=max(steps, 32) * 2, w=max(warm, 32))
        byts = 2.0 * N * K + 2.0 * M * K + 2.0 * M * N
        gbs = byts / (ms * 1e-3) / 1e9
        sk[f"M{M}"] = {"us_per_call": round(ms * 1e3, 2), "GBs": round(gbs, 1), "frac_of_measured_hbm": round(gbs / hbm, 4),
                       "frac_of_datasheet_hbm": round(gbs / PEAK_HBM_GBS, 4)}
        log(M, sk[f"M{M}"])
    res["skinny_fp16_4096x4096"] = sk
    del Wd

    # ---------------- level 1/2 ----------------
    if not args.quick:
        log("level 1/2 ...")
        n = 1 << 26
        xd = to_dev(np.random.default_rng(20).uniform(-1, 1, n).astype(np.float32))
        yd = to_dev(np.random.default_rng(21).uniform(-1, 1, n).astype(np.float32))

        def ax():
            rc = L.gen9blas_axpy(1, n, d(0.5), p(xd.data_ptr()), 1, p(yd.data_ptr()), 1)
            if rc:
                raise RuntimeError(L.gen9blas_error().decode())
        ms = timed(ax)
        res["saxpy_2^26"] = {"ms": round(ms, 4), "GBs": round(12.0 * n / (ms * 1e-3) / 1e9, 1)}
        def dt_():
            rc = L.gen9blas_dot(1, n, p(xd.data_ptr()), 1, p(yd.data_ptr()), 1, out_p)
            if rc:
                raise RuntimeError(L.gen9blas_error().decode())
        ms = timed(dt_)
        res["sdot_2^26"] = {"ms": round(ms, 4), "GBs": round(8.0 * n / (ms * 1e-3) / 1e9, 1),
                            "note": "FP64 result written to device memory"}
        del xd, yd
        m = 16384
        Ad = to_dev(np.random.default_rng(1).uniform(-1, 1, (m, m)).astype(np.float32))
        xv = to_dev(np.random.default_rng(20).uniform(-1, 1, m).astype(np.float32))
        yv = torch.empty(m, dtype=torch.float32, device=dev)
        for tr in (0, 1):
            def gv():
                rc = L.gen9blas_gemv(1, tr, m, m, d(1.0), p(Ad.data_ptr()), m, p(xv.data_ptr()), 1, d(0.0),
                                     p(yv.data_ptr()), 1)
                if rc:
                    raise RuntimeError(L.gen9blas_error().decode())
            ms = timed(gv)
            byts = 4.0 * m * m + 8.0 * m
            res[f"sgemv_{'T' if tr else 'N'}_16384"] = {"ms": round(ms, 4), "GBs": round(byts / (ms * 1e-3) / 1e9, 1)}
        for k in ("saxpy_2^26", "sdot_2^26", "sgemv_N_16384", "sgemv_T_16384"):
            res[k]["frac_of_measured_hbm"] = round(res[k]["GBs"] / hbm, 4)
            log(k, res[k])
        del Ad

    g9.set_nowait(False)

    # ---------------- calibration: AMD's libraries through torch.matmul (hipBLASLt / rocBLAS), not this library ----
    if not args.quick:
        cal = {}
        for name, tdt in (("fp16", torch.float16), ("fp32", torch.float32), ("fp64", torch.float64)):
            a = torch.randn(4096, 4096, dtype=tdt, device=dev)
            b = torch.randn(4096, 4096, dtype=tdt, device=dev)
            for _ in range(3):
                torch.matmul(a, b)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(10):
                torch.matmul(a, b)
            e1.record()
            e1.synchronize()
            ms = e0.elapsed_time(e1) / 10
            cal[name] = round(2.0 * 4096 ** 3 / (ms * 1e-3) / 1e12, 1)
            del a, b
        res["calibration_torch_matmul_n4096_tflops"] = cal
        log("calibration", cal)

    # ---------------- CPU baseline: the reference's CPU path on the host cores ----------------
    cpu = None
    if not args.quick and not args.no_cpu:
        cpu = cpu_baseline()

    h = res["hgemm_n4096"]
    line = {
        "metric": "SGEMM/HGEMM/DGEMM TFLOPS @n=4096; skinny 4096² fp16 µs/call + HBM GB/s",
        "value": h["tflops"], "unit": "TFLOPS", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": h["ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "HGEMM FP16 (GEN9BLAS_H) n=4096 NN alpha=1 beta=0, A,B ~ N(0,1) fp16, HBM-resident",
                   "M": 4096, "N": 4096, "K": 4096, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": h["tflops"], "peak": PEAK_TFLOPS["H"], "unit": "TFLOP/s",
                     "frac": h["frac_of_peak"], "traffic": None},
        "cpu_baseline": cpu,
        "results": res,
    }
    print(json.dumps(line), flush=True)


def cpu_baseline():
    """HGEMM n=4096 on the reference's CPU path (NumPy FP32 math on the FP16 inputs = OpenBLAS sgemm), bounded sample."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    threads = min(16, os.cpu_count() or 1)
    try:
        from threadpoolctl import threadpool_limits
        lim = threadpool_limits(threads)
    except Exception:
        lim = None
    n = 4096
    A = oracle.normal((n, n), np.float16, oracle.SEED_A)
    B = oracle.normal((n, n), np.float16, oracle.SEED_B)
    oracle.cpu_path.hgemm(A[:256], B)
    ts = []
    t_end = time.perf_counter() + 20
    for _ in range(5):
        t = time.perf_counter()
        oracle.cpu_path.hgemm(A, B)
        ts.append(time.perf_counter() - t)
        if time.perf_counter() > t_end:
            break
    best = min(ts)
    ver, nth = oracle.openblas_info()
    if lim is not None:
        lim.unregister() if hasattr(lim, "unregister") else None
    return {"value": round(2.0 * n ** 3 / best / 1e12, 3), "unit": "TFLOPS", "cores": nth or threads, "kind": "port",
            "sample": f"HGEMM n=4096 on the reference CPU path: NumPy FP32 matmul (OpenBLAS {ver}) of the same FP16 "
                      f"inputs, best of {len(ts)} after 1 warm-up, {nth or threads} threads on {os.cpu_count()} cpus"}


if __name__ == "__main__":
    main()
