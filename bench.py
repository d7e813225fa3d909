"""Benchmark of the gen9blas hot path on one MI355X: SGEMM/HGEMM/DGEMM TFLOPS at n = 4096, skinny 4096² FP16 µs/call
and HBM GB/s, level 1/2 GB/s, each as a fraction of its roofline, with the reference's CPU path timed beside it.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--quick] [--no-cpu] [--case NAME ...]

Prints ONE JSON line. `value` is HGEMM (GEN9BLAS_H) TFLOP/s at n = 4096 (NN, alpha = 1, beta = 0, inputs resident in
HBM); every other configuration of BASELINE.json is in `results`. A step is one library call on one configuration,
timed with HIP events recorded on the library's own stream (the stream its kernels run on) around K back-to-back calls
after W warm-up calls, in no-wait mode (device operands, no host synchronization per call). `--case` runs only the
named cases (for profiling runs; the JSON line then carries only what was measured).
Inputs: np.random.default_rng seeds A = 1, B = 2, C = 3, W copies 100..131, x = 20, y = 21 (synthetic data).
"""
import argparse
import ctypes
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.realpath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gen9-gpu-blas_amd"))

PEAK_TFLOPS = {"H": 2516.6, "HS": 2516.6, "S": 157.3, "D": 78.6}   # MI355X dense MFMA (datasheet)
PEAK_HBM_GBS = 8000.0
# HBM bytes per launch of the headline kernel, from rocprofv3 FETCH_SIZE / WRITE_SIZE runs scaled by a copy kernel
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "hgemm_n4096_hbm_traffic.md")

GEMM_CASES = {
    "hgemm_n4096": ("H", 4096), "hgemm_accurate_n4096": ("HS", 4096),
    "hgemm_n1024": ("H", 1024), "hgemm_accurate_n1024": ("HS", 1024),
    "hgemm_n2048": ("H", 2048), "hgemm_accurate_n2048": ("HS", 2048),
    "sgemm_n1024": ("S", 1024), "sgemm_n4096": ("S", 4096),
    "dgemm_n1024": ("D", 1024), "dgemm_n4096": ("D", 4096),
    "sgemm_odd_3000x11008x4096_tB_beta05": ("S", None),
}
QUICK = ("hgemm_n4096", "hgemm_accurate_n4096", "hbm_read_1GiB", "skinny")
OTHER_CASES = ("hgemm_n4096_host", "hbm_read_1GiB", "skinny", "packed_decode", "level3_n4096", "saxpy_2^26",
               "sdot_2^26", "sgemv_16384", "level2_16384", "copy_256MiB", "calibration")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def traffic_from_summary():
    """HBM bytes per launch recorded in the committed PMC summary (line `traffic_bytes_per_launch: N`), or None."""
    try:
        with open(TRAFFIC_SUMMARY) as f:
            m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", f.read(), re.M)
        return float(m.group(1)) if m else None
    except OSError:
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--quick", action="store_true", help="HGEMM n=4096, HBM read and skinny only, no CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--case", action="append", default=[], choices=list(GEMM_CASES) + list(OTHER_CASES))
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the GPU boxes of this build have one GPU and the library is single-device "
              "(multi-GPU sharding is design-only). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    cases = set(args.case) or set(QUICK if args.quick else list(GEMM_CASES) + list(OTHER_CASES))

    import torch
    import gen9blas as g9
    g9._init()
    L = g9._lib
    stream = torch.cuda.ExternalStream(g9.hip_stream())
    steps, warm = args.steps, args.warmup
    dev = torch.device("cuda:0")
    p, d = ctypes.c_void_p, ctypes.c_double

    def to_dev(x):
        return torch.from_numpy(np.ascontiguousarray(x)).to(dev)

    def check(rc):
        if rc:
            raise RuntimeError(L.gen9blas_error().decode())

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
        ms = timed(lambda: check(L.gen9blas_gemm(*args_)))
        tf = 2.0 * M * N * K / (ms * 1e-3) / 1e12
        del Ad, Bd, Cd
        return {"M": M, "N": N, "K": K, "ms": round(ms, 4), "tflops": round(tf, 2),
                "frac_of_peak": round(tf / PEAK_TFLOPS[kind], 4)}

    for name, (kind, n) in GEMM_CASES.items():
        if name not in cases:
            continue
        if n:
            res[name] = gemm_case(kind, n)
        else:
            res[name] = gemm_case(kind, M=3000, N=11008, K=4096, tB=1, beta=0.5)
        log(name, res[name])

    # ---------------- the same HGEMM on host (pageable NumPy) buffers: PCIe-inclusive whole call, not `value` ------
    if "hgemm_n4096_host" in cases:
        n = 4096
        A = np.random.default_rng(1).standard_normal((n, n), dtype=np.float32).astype(np.float16)
        B = np.random.default_rng(2).standard_normal((n, n), dtype=np.float32).astype(np.float16)
        C = np.empty((n, n), np.float16)
        call = lambda: check(L.gen9blas_gemm(0, 0, 0, n, n, n, d(1.0), p(A.ctypes.data), n, p(B.ctypes.data), n,
                                             d(0.0), p(C.ctypes.data), n))
        g9.set_nowait(False)   # host operands: every call copies in, computes, copies back and waits
        call()
        ts = []
        for _ in range(max(3, steps // 4)):
            t = time.perf_counter()
            call()
            ts.append(time.perf_counter() - t)
        g9.set_nowait(True)
        ms = float(np.median(ts)) * 1e3
        res["hgemm_n4096_host"] = {"ms": round(ms, 3), "tflops": round(2.0 * n ** 3 / (ms * 1e-3) / 1e12, 2),
                                   "note": "whole call on pageable host buffers: 2 x 32 MiB in, 32 MiB out over PCIe"}
        log("hgemm_n4096_host", res["hgemm_n4096_host"])
        del A, B, C

    # ---------------- measured HBM bandwidth: streaming read of 1 GiB (> 256 MB MALL) ----------------
    out_d = torch.zeros(1, dtype=torch.float64, device=dev)   # device result: no host wait per call
    out_p = ctypes.cast(ctypes.c_void_p(out_d.data_ptr()), ctypes.POINTER(ctypes.c_double))
    hbm = None
    if "hbm_read_1GiB" in cases:
        nh = 1 << 28
        big = torch.empty(nh, dtype=torch.float32, device=dev).uniform_(-1, 1)
        ms = timed(lambda: check(L.gen9blas_asum(1, nh, p(big.data_ptr()), 1, out_p)), k=10, w=2)
        hbm = 4.0 * nh / (ms * 1e-3) / 1e9
        res["hbm_read_1GiB"] = {"kernel": "gen9blas_asum FP32 2^28 (pure streaming read)", "ms": round(ms, 4),
                                "GBs": round(hbm, 1), "frac_of_datasheet": round(hbm / PEAK_HBM_GBS, 4)}
        log("hbm_read_1GiB", res["hbm_read_1GiB"])
        del big

    def hbm_fracs(r):
        if hbm:
            r["frac_of_measured_hbm"] = round(r["GBs"] / hbm, 4)
        r["frac_of_datasheet_hbm"] = round(r["GBs"] / PEAK_HBM_GBS, 4)
        return r

    # ---------------- skinny C = A·Wᵀ, W 4096² fp16, 32 rotated copies (1 GiB) ----------------
    if "skinny" in cases:
        K = N = 4096
        ncopy = 32
        Wd = torch.empty((ncopy, N, K), dtype=torch.float16, device=dev)
        for c in range(ncopy):
            w = np.random.default_rng(100 + c).standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
            Wd[c].copy_(torch.from_numpy(w.astype(np.float16)))
        sk = {}
        wp = [Wd[c].data_ptr() for c in range(ncopy)]
        for M in (1, 2, 4, 8, 16):
            Ad = to_dev(np.random.default_rng(1).standard_normal((M, K), dtype=np.float32).astype(np.float16))
            Cd = torch.empty((M, N), dtype=torch.float16, device=dev)
            state = {"j": 0}

            def fn():
                j = state["j"]
                state["j"] = (j + 1) % ncopy
                check(L.gen9blas_gemm(0, 0, 1, M, N, K, d(1.0), p(Ad.data_ptr()), K, p(wp[j]), K, d(0.0),
                                      p(Cd.data_ptr()), N))
            ms = timed(fn, k=max(steps, 32) * 2, w=max(warm, 32))
            byts = 2.0 * N * K + 2.0 * M * K + 2.0 * M * N
            sk[f"M{M}"] = hbm_fracs({"us_per_call": round(ms * 1e3, 2), "GBs": round(byts / (ms * 1e-3) / 1e9, 1)})
            log("skinny", M, sk[f"M{M}"])
        res["skinny_fp16_4096x4096"] = sk
        del Wd

    # ---------------- packed weights: gemm_pb (M = 1..16) on 32 resident packed copies of a 4096² fp16 W ----------
    if "packed_decode" in cases:
        K = N = 4096
        ncopy = 32
        packs = []
        for c in range(ncopy):
            w = np.random.default_rng(100 + c).standard_normal((K, N), dtype=np.float32) * np.float32(0.02)
            Wd = to_dev(w.astype(np.float16))   # K×N, packed once (transB = 0) and then released
            torch.cuda.synchronize()            # the copy ran on torch's stream, pack_b reads on the library's
            h = L.gen9blas_pack_b(2, 0, K, N, p(Wd.data_ptr()), N)   # GEN9BLAS_HS: also what gemm_pb_skinny takes
            if not h:
                raise RuntimeError(L.gen9blas_error().decode())
            packs.append(h)
            del Wd
        pk = {}
        for M in (1, 4, 16):
            Ad = to_dev(np.random.default_rng(1).standard_normal((M, K), dtype=np.float32).astype(np.float16))
            Cd = torch.empty((M, N), dtype=torch.float16, device=dev)
            state = {"j": 0}

            def fn():
                j = state["j"]
                state["j"] = (j + 1) % ncopy
                check(L.gen9blas_gemm_pb(0, M, d(1.0), p(Ad.data_ptr()), K, p(packs[j]), d(0.0), p(Cd.data_ptr()), N))
            ms = timed(fn, k=max(steps, 32) * 2, w=max(warm, 32))
            byts = 2.0 * N * K + 2.0 * M * K + 2.0 * M * N
            pk[f"M{M}"] = hbm_fracs({"us_per_call": round(ms * 1e3, 2), "GBs": round(byts / (ms * 1e-3) / 1e9, 1)})
            log("packed_decode", M, pk[f"M{M}"])
        # gen9blas_gemm_pb_skinny: FP32 activations on the same packed FP16 weights, FP32 result. The call waits for its
        # kernel (it reports non-finite results), so this time includes the wait and the flag read; the kernel's own
        # duration is in the rocprofv3 trace (skinny_pb_kernel).
        L.gen9blas_gemm_pb_skinny.argtypes = [ctypes.c_int, p, ctypes.c_int, p, p, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]
        nfv = ctypes.c_int(0)
        for M in (1, 4, 16):
            Af = to_dev(np.random.default_rng(1).standard_normal((M, K), dtype=np.float32))
            Cf = torch.empty((M, N), dtype=torch.float32, device=dev)
            state = {"j": 0}

            def fn():
                j = state["j"]
                state["j"] = (j + 1) % ncopy
                check(L.gen9blas_gemm_pb_skinny(M, p(Af.data_ptr()), K, p(packs[j]), p(Cf.data_ptr()), N,
                                                ctypes.byref(nfv)))
            ms = timed(fn, k=max(steps, 32) * 2, w=max(warm, 32))
            byts = 2.0 * N * K + 4.0 * M * K + 4.0 * M * N
            pk[f"pb_skinny_f32_M{M}"] = hbm_fracs({"us_per_call": round(ms * 1e3, 2),
                                                   "GBs": round(byts / (ms * 1e-3) / 1e9, 1),
                                                   "note": "synchronous call (waits, reads the non-finite flag)"})
            log("packed_decode pb_skinny", M, pk[f"pb_skinny_f32_M{M}"])
        for h in packs:
            L.gen9blas_packed_b_free(p(h))
        res["packed_decode_fp16_4096x4096"] = pk

    # ---------------- level 3 beyond GEMM at n = 4096 (useful flops: SYMM 2n³, SYRK n³, SYR2K 2n³, TRMM/TRSM n³) -----
    if "level3_n4096" in cases:
        n = 4096
        l3 = {}
        for kind, typ, dt in (("S", 1, np.float32), ("D", 3, np.float64)):
            rng = np.random.default_rng(30)
            A = rng.uniform(-1, 1, (n, n)) / n
            A[np.diag_indices(n)] = 1.0            # well-conditioned triangle for TRSM
            Ad = to_dev(A.astype(dt))
            Bd = to_dev(rng.uniform(-1, 1, (n, n)).astype(dt))
            Cd = to_dev(rng.uniform(-1, 1, (n, n)).astype(dt))
            Xd = torch.empty_like(Bd)
            a, b, c, x = (p(t.data_ptr()) for t in (Ad, Bd, Cd, Xd))
            calls = {
                "symm_LL": (2.0, lambda: check(L.gen9blas_symm(typ, 0, 0, n, n, d(1.0), a, n, b, n, d(0.5), c, n))),
                "syrk_LN": (1.0, lambda: check(L.gen9blas_syrk(typ, 0, 0, n, n, d(1.0), b, n, d(0.5), c, n))),
                "syr2k_LN": (2.0, lambda: check(L.gen9blas_syr2k(typ, 0, 0, n, n, d(1.0), a, n, b, n, d(0.5), c, n))),
                # TRMM/TRSM overwrite their B: a fresh copy first, by the library on its stream (a copy of 64 / 128
                # MiB, under 1 % of the call, inside the timing)
                "trmm_LLN": (1.0, lambda: (check(L.gen9blas_copy(typ, n * n, b, 1, x, 1)),
                                           check(L.gen9blas_trmm(typ, 0, 0, 0, 0, n, n, d(1.0), a, n, x, n)))),
                "trsm_LLN": (1.0, lambda: (check(L.gen9blas_copy(typ, n * n, b, 1, x, 1)),
                                           check(L.gen9blas_trsm(typ, 0, 0, 0, 0, n, n, d(1.0), a, n, x, n)))),
            }
            for name, (mult, fn) in calls.items():
                ms = timed(fn, k=max(3, steps // 4), w=1)
                tf = mult * n ** 3 / (ms * 1e-3) / 1e12
                l3[f"{kind.lower()}{name}"] = {"ms": round(ms, 3), "tflops": round(tf, 2),
                                               "frac_of_peak": round(tf / PEAK_TFLOPS[kind], 4)}
                log("level3", kind, name, l3[f"{kind.lower()}{name}"])
            del Ad, Bd, Cd, Xd
        res["level3_n4096"] = l3

    # ---------------- level 1/2 ----------------
    n = 1 << 26
    if cases & {"saxpy_2^26", "sdot_2^26", "copy_256MiB"}:
        xd = to_dev(np.random.default_rng(20).uniform(-1, 1, n).astype(np.float32))
        yd = to_dev(np.random.default_rng(21).uniform(-1, 1, n).astype(np.float32))
        if "saxpy_2^26" in cases:
            ms = timed(lambda: check(L.gen9blas_axpy(1, n, d(0.5), p(xd.data_ptr()), 1, p(yd.data_ptr()), 1)))
            res["saxpy_2^26"] = hbm_fracs({"ms": round(ms, 4), "GBs": round(12.0 * n / (ms * 1e-3) / 1e9, 1)})
            log("saxpy_2^26", res["saxpy_2^26"])
        if "sdot_2^26" in cases:
            ms = timed(lambda: check(L.gen9blas_dot(1, n, p(xd.data_ptr()), 1, p(yd.data_ptr()), 1, out_p)))
            res["sdot_2^26"] = hbm_fracs({"ms": round(ms, 4), "GBs": round(8.0 * n / (ms * 1e-3) / 1e9, 1),
                                          "note": "FP64 result written to device memory"})
            log("sdot_2^26", res["sdot_2^26"])
        if "copy_256MiB" in cases:
            # known-size copy (reads 256 MiB, writes 256 MiB): the reference point for the HBM byte counters
            ms = timed(lambda: check(L.gen9blas_copy(1, n, p(xd.data_ptr()), 1, p(yd.data_ptr()), 1)))
            res["copy_256MiB"] = hbm_fracs({"ms": round(ms, 4), "GBs": round(8.0 * n / (ms * 1e-3) / 1e9, 1)})
            log("copy_256MiB", res["copy_256MiB"])
        del xd, yd
    if "sgemv_16384" in cases:
        m = 16384
        Ad = to_dev(np.random.default_rng(1).uniform(-1, 1, (m, m)).astype(np.float32))
        xv = to_dev(np.random.default_rng(20).uniform(-1, 1, m).astype(np.float32))
        yv = torch.empty(m, dtype=torch.float32, device=dev)
        for tr in (0, 1):
            ms = timed(lambda: check(L.gen9blas_gemv(1, tr, m, m, d(1.0), p(Ad.data_ptr()), m, p(xv.data_ptr()), 1,
                                                     d(0.0), p(yv.data_ptr()), 1)))
            byts = 4.0 * m * m + 8.0 * m
            k = f"sgemv_{'T' if tr else 'N'}_16384"
            res[k] = hbm_fracs({"ms": round(ms, 4), "GBs": round(byts / (ms * 1e-3) / 1e9, 1)})
            log(k, res[k])
        del Ad

    if "level2_16384" in cases:
        # FP32 n = 16384 on device buffers. Algorithmic bytes: the stored triangle once (n(n+1)/2 elements, 512 MiB)
        # plus the vectors; SYR2 reads and writes the triangle. TRSV restores its right-hand side by a library copy
        # on the same stream before each solve (64 KiB, inside the timing).
        m = 16384
        rng = np.random.default_rng(31)
        A = rng.uniform(-1, 1, (m, m)).astype(np.float32) / np.float32(m)
        A[np.diag_indices(m)] = 1.0
        Ad = to_dev(A)
        del A
        Apd = to_dev(np.random.default_rng(32).uniform(-1, 1, m * (m + 1) // 2).astype(np.float32))
        xv = to_dev(np.random.default_rng(20).uniform(-1, 1, m).astype(np.float32))
        yv = to_dev(np.random.default_rng(21).uniform(-1, 1, m).astype(np.float32))
        wv = torch.empty_like(xv)
        a, ap, x, y, w = (p(t.data_ptr()) for t in (Ad, Apd, xv, yv, wv))
        tri = 4.0 * m * (m + 1) / 2
        calls = {
            "ssymv_L": (tri + 12.0 * m, lambda: check(L.gen9blas_symv(1, 0, m, d(1.0), a, m, x, 1, d(0.0), y, 1))),
            "ssymv_U": (tri + 12.0 * m, lambda: check(L.gen9blas_symv(1, 1, m, d(1.0), a, m, x, 1, d(0.0), y, 1))),
            "strmv_LN": (tri + 8.0 * m, lambda: (check(L.gen9blas_copy(1, m, x, 1, w, 1)),
                                                 check(L.gen9blas_trmv(1, 0, 0, 0, m, a, m, w, 1)))),
            "strmv_LT": (tri + 8.0 * m, lambda: (check(L.gen9blas_copy(1, m, x, 1, w, 1)),
                                                 check(L.gen9blas_trmv(1, 0, 1, 0, m, a, m, w, 1)))),
            "strsv_LN": (tri + 8.0 * m, lambda: (check(L.gen9blas_copy(1, m, x, 1, w, 1)),
                                                 check(L.gen9blas_trsv(1, 0, 0, 0, m, a, m, w, 1)))),
            "strsv_LT": (tri + 8.0 * m, lambda: (check(L.gen9blas_copy(1, m, x, 1, w, 1)),
                                                 check(L.gen9blas_trsv(1, 0, 1, 0, m, a, m, w, 1)))),
            "sspmv_L": (tri + 12.0 * m, lambda: check(L.gen9blas_spmv(1, 0, m, d(1.0), ap, x, 1, d(0.0), y, 1))),
            "ssyr2_L": (2 * tri + 8.0 * m, lambda: check(L.gen9blas_syr2(1, 0, m, d(1e-3), x, 1, y, 1, a, m))),
        }
        l2 = {}
        for name, (byts, fn) in calls.items():
            ms = timed(fn, k=max(5, steps // 2), w=2)
            l2[name] = hbm_fracs({"ms": round(ms, 4), "GBs": round(byts / (ms * 1e-3) / 1e9, 1)})
            log("level2", name, l2[name])
        res["level2_16384"] = l2
        del Ad, Apd

    g9.set_nowait(False)

    # ---------------- calibration: AMD's libraries through torch.matmul (hipBLASLt / rocBLAS), not this library ----
    if "calibration" in cases:
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
    if not args.quick and not args.no_cpu and not args.case:
        cpu = cpu_baseline()

    h = res.get("hgemm_n4096")
    line = {
        "metric": "SGEMM/HGEMM/DGEMM TFLOPS @n=4096; skinny 4096² fp16 µs/call + HBM GB/s",
        "value": h["tflops"] if h else None, "unit": "TFLOPS", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": h["ms"] if h else None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "HGEMM FP16 (GEN9BLAS_H) n=4096 NN alpha=1 beta=0, A,B ~ N(0,1) fp16, HBM-resident",
                   "M": 4096, "N": 4096, "K": 4096, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": h["tflops"] if h else None, "peak": PEAK_TFLOPS["H"],
                     "unit": "TFLOP/s", "frac": h["frac_of_peak"] if h else None, "traffic": traffic_from_summary(),
                     "traffic_unit": "bytes per launch (HBM, FETCH_SIZE + WRITE_SIZE scaled by a known-size copy)",
                     "algorithmic_bytes": 3 * 2 * 4096 * 4096},
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
