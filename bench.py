"""Benchmark of the gen9blas hot path on one MI355X: SGEMM/HGEMM/DGEMM TFLOPS at n = 4096, skinny 4096² FP16 µs/call
and HBM GB/s, level 1/2 GB/s, each as a fraction of its roofline, with the reference's CPU path timed beside it.

    python bench.py [--steps K] [--warmup W] [--settle S] [--gpus 1] [--quick] [--no-cpu] [--case NAME ...]

Prints ONE JSON line. `value` is HGEMM (GEN9BLAS_H) TFLOP/s at n = 4096 (NN, alpha = 1, beta = 0, inputs resident in
HBM); every other configuration of BASELINE.json is in `results`. A step is one library call on one configuration,
timed with HIP events recorded on the library's own stream (the stream its kernels run on) around K back-to-back calls
after W warm-up calls, in no-wait mode (device operands, no host synchronization per call). Before the W warm-ups each
case runs the same call for S seconds (default 1.5): the MI355X clock climbs for about a second after the GPU has been
idle (measured 1.7 → 2.4 GHz over 1.2 s) and then settles under the board's power limit, so shorter runs measure the
ramp, not the sustained rate. The hipBLASLt calibration is timed the same way. `--case` runs only the named cases (for
profiling runs; the JSON line then carries only what was measured).
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
QUICK = ("hgemm_n4096", "hgemm_accurate_n4096", "hbm_read_1GiB", "skinny", "skinny_kn")
OTHER_CASES = ("hgemm_n4096_host", "hbm_read_1GiB", "skinny", "skinny_kn", "skinny_read_floor", "packed_decode", "level3_n4096",
               "saxpy_2^26", "sdot_2^26", "sgemv_16384", "level2_16384", "copy_256MiB", "calibration", "mfma_ceiling")
# Opt-in cases (--case only): the headline product on low-entropy operands, whose matrix cores draw less power than
# on N(0, 1) data, so the board's power limit lowers the clock less (power-cap evidence for the headline kernel)
OPT_CASES = ("hgemm_n4096_zeros", "hgemm_n4096_ternary")
CALIB_LIB = os.path.join(ROOT, "gen9-gpu-blas_amd", "libgen9blas_calib.so")   # calibration kernels (calib/calibrate.hip)


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
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--settle", type=float, default=1.5, help="seconds of the same call before each case's warm-ups")
    ap.add_argument("--quick", action="store_true", help="HGEMM n=4096, HBM read and skinny only, no CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--case", action="append", default=[], choices=list(GEMM_CASES) + list(OTHER_CASES) + list(OPT_CASES))
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
    cal = ctypes.CDLL(CALIB_LIB)
    cal.g9cal_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    cal.g9cal_mfma.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int,
                               ctypes.c_int, ctypes.c_void_p]
    cal.g9cal_touch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    cal.g9cal_round_trip_us.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    cal.g9cal_round_trip_us.restype = ctypes.c_double
    lib_stream = ctypes.c_void_p(g9.hip_stream())
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    p, d = ctypes.c_void_p, ctypes.c_double

    def to_dev(x):
        return torch.from_numpy(np.ascontiguousarray(x)).to(dev)

    def check(rc):
        if rc:
            raise RuntimeError(L.gen9blas_error().decode())

    def settle(fn, seconds):
        """Runs fn back to back for `seconds` (waiting every 64 calls, so the queue stays short)."""
        t_end = time.perf_counter() + seconds
        while time.perf_counter() < t_end:
            for _ in range(64):
                fn()
            g9.flush()
            torch.cuda.synchronize()

    def timed(fn, k=steps, w=warm):
        """ms per call: HIP events on the library stream around k back-to-back calls after the settle period and w
        warm-ups."""
        settle(fn, args.settle)
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
    # calls timed for kernels of a few µs (skinny, its read floor, packed decode): about 4.5 ms at 7 µs, so the first
    # launch after the drained queue weighs under 1 %
    kshort = max(2 * steps, 640)

    # ---------------- GEMM ----------------
    def gemm_case(kind, n=None, M=None, N=None, K=None, tB=0, beta=0.0, headline=False, operands="normal"):
        """The headline case times exactly `steps` calls; the others at least `steps`, and as many as fill about 5 ms
        at the expected rate, so that the first launch after the drained queue weighs under 1 % (n = 1024: 50 calls
        are 0.28 ms)."""
        M, N, K = (n, n, n) if n else (M, N, K)
        dt = {"H": np.float16, "HS": np.float16, "S": np.float32, "D": np.float64}[kind]
        typ = {"H": 0, "HS": 2, "S": 1, "D": 3}[kind]
        if operands == "zeros":
            A, B = np.zeros((M, K), dt), np.zeros((N, K) if tB else (K, N), dt)
        elif operands == "ternary":   # entries in {-1, 0, 1}
            A = np.random.default_rng(1).integers(-1, 2, (M, K)).astype(dt)
            B = np.random.default_rng(2).integers(-1, 2, (N, K) if tB else (K, N)).astype(dt)
        elif dt == np.float16:
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
        est_s = 2.0 * M * N * K / {"H": 1.2e15, "HS": 1.2e15, "S": 1.4e14, "D": 7e13}[kind]
        k = steps if headline else max(steps, int(5e-3 / est_s))
        ms = timed(lambda: check(L.gen9blas_gemm(*args_)), k=k)
        tf = 2.0 * M * N * K / (ms * 1e-3) / 1e12
        del Ad, Bd, Cd
        return {"M": M, "N": N, "K": K, "ms": round(ms, 4), "tflops": round(tf, 2),
                "frac_of_peak": round(tf / PEAK_TFLOPS[kind], 4), "calls": k}

    for name, (kind, n) in GEMM_CASES.items():
        if name not in cases:
            continue
        if n:
            res[name] = gemm_case(kind, n, headline=name == "hgemm_n4096")
        else:
            res[name] = gemm_case(kind, M=3000, N=11008, K=4096, tB=1, beta=0.5)
        log(name, res[name])
    for name in OPT_CASES:
        if name in cases:
            res[name] = gemm_case("H", 4096, operands=name.rsplit("_", 1)[1])
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
    if "hbm_read_1GiB" in cases:
        nh = 1 << 28
        big = torch.empty(nh, dtype=torch.float32, device=dev).uniform_(-1, 1)
        ms = timed(lambda: check(L.gen9blas_asum(1, nh, p(big.data_ptr()), 1, out_p)), k=20, w=2)
        hbm = 4.0 * nh / (ms * 1e-3) / 1e9
        res["hbm_read_1GiB"] = {"kernel": "gen9blas_asum FP32 2^28 (pure streaming read)", "ms": round(ms, 4),
                                "GBs": round(hbm, 1), "frac_of_datasheet": round(hbm / PEAK_HBM_GBS, 4)}
        log("hbm_read_1GiB", res["hbm_read_1GiB"])
        sink = torch.empty(4 * ncu, dtype=torch.float32, device=dev)
        ms = timed(lambda: check(cal.g9cal_stream_read(big.data_ptr(), 4 * nh, sink.data_ptr(), 4 * ncu, lib_stream)),
                   k=20, w=2)
        gbs = 4.0 * nh / (ms * 1e-3) / 1e9
        res["calib_stream_read_1GiB"] = {"kernel": "calibration streaming read (8 loads of 16 B in flight per lane)",
                                         "ms": round(ms, 4), "GBs": round(gbs, 1),
                                         "frac_of_datasheet": round(gbs / PEAK_HBM_GBS, 4)}
        log("calib_stream_read_1GiB", res["calib_stream_read_1GiB"])
        del big, sink

    hbm_rated = []   # streaming results whose fraction of the measured HBM bandwidth is filled in at the end

    def hbm_fracs(r):
        r["frac_of_datasheet_hbm"] = round(r["GBs"] / PEAK_HBM_GBS, 4)
        hbm_rated.append(r)
        return r

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
    # ---------------- skinny C = A·Wᵀ, W 4096² fp16, 32 rotated copies (1 GiB); then W stored K×N ----------------
    if cases & {"skinny", "skinny_kn", "skinny_read_floor"}:
        K = N = 4096
        ncopy = 32
        Wd = torch.empty((ncopy, N, K), dtype=torch.float16, device=dev)
        for c in range(ncopy):
            w = np.random.default_rng(100 + c).standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
            Wd[c].copy_(torch.from_numpy(w.astype(np.float16)))
        sk = {}
        wp = [Wd[c].data_ptr() for c in range(ncopy)]
        for M in ((1, 2, 4, 8, 16) if "skinny" in cases else ()):
            Ad = to_dev(np.random.default_rng(1).standard_normal((M, K), dtype=np.float32).astype(np.float16))
            Cd = torch.empty((M, N), dtype=torch.float16, device=dev)
            state = {"j": 0}

            def fn():
                j = state["j"]
                state["j"] = (j + 1) % ncopy
                check(L.gen9blas_gemm(0, 0, 1, M, N, K, d(1.0), p(Ad.data_ptr()), K, p(wp[j]), K, d(0.0),
                                      p(Cd.data_ptr()), N))
            ms = timed(fn, k=kshort, w=max(warm, 32))
            byts = 2.0 * N * K + 2.0 * M * K + 2.0 * M * N
            sk[f"M{M}"] = hbm_fracs({"us_per_call": round(ms * 1e3, 2), "GBs": round(byts / (ms * 1e-3) / 1e9, 1)})
            log("skinny", M, sk[f"M{M}"])
        if sk:
            res["skinny_fp16_4096x4096"] = sk
        if "skinny_kn" in cases:
            # the same products with W stored K×N (row-major x·W, weights contiguous along N): the same 32 copies,
            # transposed on the device
            Wkn = Wd.transpose(1, 2).contiguous()
            torch.cuda.synchronize()
            wq = [Wkn[c].data_ptr() for c in range(ncopy)]
            skn = {}
            for M in (1, 2, 4, 8, 16):
                Ad = to_dev(np.random.default_rng(1).standard_normal((M, K), dtype=np.float32).astype(np.float16))
                Cd = torch.empty((M, N), dtype=torch.float16, device=dev)
                state = {"j": 0}

                def fn():
                    j = state["j"]
                    state["j"] = (j + 1) % ncopy
                    check(L.gen9blas_gemm(0, 0, 0, M, N, K, d(1.0), p(Ad.data_ptr()), K, p(wq[j]), N, d(0.0),
                                          p(Cd.data_ptr()), N))
                ms = timed(fn, k=kshort, w=max(warm, 32))
                byts = 2.0 * N * K + 2.0 * M * K + 2.0 * M * N
                skn[f"M{M}"] = hbm_fracs({"us_per_call": round(ms * 1e3, 2), "GBs": round(byts / (ms * 1e-3) / 1e9, 1)})
                log("skinny_kn", M, skn[f"M{M}"])
            res["skinny_kn_fp16_4096x4096"] = skn
            del Wkn
        if "skinny_read_floor" in cases:
            # the floor of one skinny call: a pure read of the same 32 MiB weight copy per call, over the same 32
            # rotated copies, by the calibration streaming-read kernel (one kernel per call, as the skinny product) with
            # 512 and 1024 blocks, and by the library's own asum (two kernels per call: partial sums, then their sum)
            sink = torch.empty(1024, dtype=torch.float32, device=dev)
            byts = 2.0 * N * K
            floor = {}
            for blocks in (512, 1024):
                state = {"j": 0}

                def fn():
                    j = state["j"]
                    state["j"] = (j + 1) % ncopy
                    check(cal.g9cal_stream_read(wp[j], N * K * 2, sink.data_ptr(), blocks, lib_stream))
                ms = timed(fn, k=kshort, w=max(warm, 32))
                floor[f"calib_read_{blocks}_blocks"] = hbm_fracs({"us_per_call": round(ms * 1e3, 2),
                                                                  "GBs": round(byts / (ms * 1e-3) / 1e9, 1)})
            state = {"j": 0}

            def fn():
                j = state["j"]
                state["j"] = (j + 1) % ncopy
                check(L.gen9blas_asum(0, N * K, p(wp[j]), 1, out_p))
            ms = timed(fn, k=kshort, w=max(warm, 32))
            floor["gen9blas_asum_fp16"] = hbm_fracs({"us_per_call": round(ms * 1e3, 2),
                                                     "GBs": round(byts / (ms * 1e-3) / 1e9, 1)})
            floor["note"] = "a pure read of one 4096x4096 fp16 copy per call, 32 copies rotated (1 GiB)"
            res["skinny_read_floor_32MiB"] = floor
            log("skinny_read_floor", floor)
            # Decomposition of the one-pass floor into a fixed part per call and a streaming part: the calibration
            # read (1024 blocks) over S MiB per call, each call a new region of the same 1 GiB (beyond the 256 MB
            # MALL), S = 4 .. 128; t(S) = t0 + S / bw fitted over S = 16 .. 128. Beside it: the same 32 MiB region read
            # by every call (served from the MALL), and the one-word kernel back to back (the launch-to-launch floor
            # of dependent kernels on one stream).
            flat = Wd.view(-1)
            total = flat.numel() * 2
            dec = {}
            for mib in (4, 8, 16, 32, 64, 128):
                size = mib << 20
                nreg = total // size
                state = {"j": 0}

                def fn():
                    j = state["j"]
                    state["j"] = (j + 1) % nreg
                    check(cal.g9cal_stream_read(flat.data_ptr() + j * size, size, sink.data_ptr(), 1024, lib_stream))
                ms = timed(fn, k=kshort, w=max(warm, 32))
                dec[f"{mib}MiB"] = {"us_per_call": round(ms * 1e3, 2), "GBs": round(size / (ms * 1e-3) / 1e9, 1)}

            def fn():
                check(cal.g9cal_stream_read(flat.data_ptr(), 32 << 20, sink.data_ptr(), 1024, lib_stream))
            ms = timed(fn, k=kshort, w=max(warm, 32))
            dec["32MiB_same_region_MALL"] = {"us_per_call": round(ms * 1e3, 2),
                                             "GBs": round((32 << 20) / (ms * 1e-3) / 1e9, 1)}
            ms = timed(lambda: check(cal.g9cal_touch(sink.data_ptr(), lib_stream)), k=kshort, w=max(warm, 32))
            dec["empty_kernel_us"] = round(ms * 1e3, 2)
            xs = np.array([16.0, 32.0, 64.0, 128.0]) * (1 << 20)
            ys = np.array([dec[f"{int(x) >> 20}MiB"]["us_per_call"] for x in xs])
            slope, t0 = np.polyfit(xs, ys, 1)
            dec["fit_16_128MiB"] = {"t0_us": round(float(t0), 2), "streaming_GBs": round(1e-3 / float(slope), 1),
                                    "model_32MiB_us": round(float(t0 + slope * (32 << 20)), 2)}
            res["skinny_floor_decomposition"] = dec
            log("skinny_floor_decomposition", dec)
            del sink
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
            ms = timed(fn, k=kshort, w=max(warm, 32))
            byts = 2.0 * N * K + 2.0 * M * K + 2.0 * M * N
            pk[f"M{M}"] = hbm_fracs({"us_per_call": round(ms * 1e3, 2), "GBs": round(byts / (ms * 1e-3) / 1e9, 1)})
            log("packed_decode", M, pk[f"M{M}"])
        # gen9blas_gemm_pb_skinny: FP32 activations on the same packed FP16 weights, FP32 result. The call waits for its
        # kernel (it reports non-finite results), so this time includes the launch, the wait and the flag read; the
        # kernel's own duration is in the rocprofv3 trace (skinny_pb_lds_kernel). For scale: the launch-and-wait round
        # trip of a one-word kernel on the same stream, measured here.
        touch = torch.zeros(1, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        rt = cal.g9cal_round_trip_us(touch.data_ptr(), 2000, lib_stream)
        if rt < 0:
            raise RuntimeError("round-trip probe failed")
        pk["sync_round_trip_one_word_kernel_us"] = round(rt, 2)
        log("packed_decode round trip", rt)
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

    # ---------------- the matrix cores' sustained FP16 rate on random operands, with no data movement ----------------
    if "mfma_ceiling" in cases:
        src = torch.from_numpy(np.random.default_rng(1).standard_normal(8 << 20, dtype=np.float32).astype(np.float16)).to(dev)
        blocks, iters = 2 * ncu, 2000                 # 8 waves per CU; about 2 ms per call
        outb = torch.empty(blocks * 256, dtype=torch.float32, device=dev)
        flop = blocks * 4 * iters * float(1 << 20)
        mc = {}
        for shape in (32, 16):
            ms = timed(lambda: check(cal.g9cal_mfma(shape, src.data_ptr(), src.numel() * 2, outb.data_ptr(), blocks,
                                                    iters, lib_stream)), k=20, w=2)
            mc[f"mfma_f32_{shape}x{shape}x{512 // shape}_f16"] = round(flop / (ms * 1e-3) / 1e12, 1)
        mc["note"] = ("calibration loop of MFMAs on random FP16 register operands (8 waves per CU, no memory traffic): "
                      "the rate the matrix cores sustain under the board's power limit")
        res["mfma_ceiling_fp16_tflops"] = mc
        log("mfma_ceiling", mc)
        del src, outb

    # ---------------- calibration: AMD's libraries through torch.matmul (hipBLASLt / rocBLAS), not this library ----
    if "calibration" in cases:
        cal = {}
        for name, tdt in (("fp16", torch.float16), ("fp32", torch.float32), ("fp64", torch.float64)):
            if tdt == torch.float16:
                a = torch.from_numpy(np.random.default_rng(1).standard_normal((4096, 4096), dtype=np.float32)).to(dev, tdt)
                b = torch.from_numpy(np.random.default_rng(2).standard_normal((4096, 4096), dtype=np.float32)).to(dev, tdt)
            else:
                a = torch.empty(4096, 4096, dtype=tdt, device=dev).uniform_(-1, 1)
                b = torch.empty(4096, 4096, dtype=tdt, device=dev).uniform_(-1, 1)
            c = torch.empty(4096, 4096, dtype=tdt, device=dev)
            t_end = time.perf_counter() + args.settle
            while time.perf_counter() < t_end:
                for _ in range(16):
                    torch.matmul(a, b, out=c)
                torch.cuda.synchronize()
            for _ in range(warm):
                torch.matmul(a, b, out=c)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(steps):
                torch.matmul(a, b, out=c)
            e1.record()
            e1.synchronize()
            ms = e0.elapsed_time(e1) / steps
            cal[name] = round(2.0 * 4096 ** 3 / (ms * 1e-3) / 1e12, 1)
            del a, b, c
        res["calibration_torch_matmul_n4096_tflops"] = cal
        log("calibration", cal)

    # ---------------- fractions of the measured HBM bandwidth ----------------
    # The reference point is the fastest streaming kernel over working sets beyond the MALL: the library's 1 GiB read
    # (asum), the calibration read of the same 1 GiB, SDOT (2 × 256 MiB read) and the copy (256 MiB read + written).
    ref_keys = ("hbm_read_1GiB", "calib_stream_read_1GiB", "sdot_2^26", "copy_256MiB")
    streams = [res[k]["GBs"] for k in ref_keys if k in res]
    if streams:
        hbm_ref = max(streams)
        res["measured_hbm_GBs"] = {"GBs": round(hbm_ref, 1), "of": "max of " + ", ".join(k for k in ref_keys if k in res)}
        for r in hbm_rated:
            r["frac_of_measured_hbm"] = round(r["GBs"] / hbm_ref, 4)

    # ---------------- CPU baseline: the reference's CPU path on the host cores ----------------
    cpu = None
    if not args.quick and not args.no_cpu and not args.case:
        cpu, per_config = cpu_baselines()
        for k, v in per_config.items():
            res.setdefault("cpu_path", {})[k] = v
            log("cpu", k, v)

    h = res.get("hgemm_n4096")
    line = {
        "metric": "SGEMM/HGEMM/DGEMM TFLOPS @n=4096; skinny 4096² fp16 µs/call + HBM GB/s",
        "value": h["tflops"] if h else None, "unit": "TFLOPS", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": h["ms"] if h else None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "HGEMM FP16 (GEN9BLAS_H) n=4096 NN alpha=1 beta=0, A,B ~ N(0,1) fp16, HBM-resident",
                   "M": 4096, "N": 4096, "K": 4096, "parallelism": "single GPU", "settle_s": args.settle},
        "roofline": {"bound": "mfma", "achieved": h["tflops"] if h else None, "peak": PEAK_TFLOPS["H"],
                     "unit": "TFLOP/s", "frac": h["frac_of_peak"] if h else None, "traffic": traffic_from_summary(),
                     "traffic_unit": "bytes per launch (HBM, FETCH_SIZE + WRITE_SIZE scaled by a known-size copy)",
                     "algorithmic_bytes": 3 * 2 * 4096 * 4096},
        "cpu_baseline": cpu,
        "results": res,
    }
    summary = config_summary(res)
    line["summary"] = summary   # last key: the end of the line (what a tail keeps) holds every configuration
    print(json.dumps(line), flush=True)
    for s in summary:
        log(s)


def config_summary(res):
    """One short line per benchmarked configuration (GPU rate, fraction of its roofline, the CPU path's rate),
    printed last so that a truncated log still holds every configuration."""
    cpu = res.get("cpu_path", {})

    def cpu_of(key, unit):
        v = cpu.get(key)
        return f" | cpu {v['value']:g} {unit}" if v else ""
    out = []
    for name, (kind, n) in GEMM_CASES.items():
        r = res.get(name)
        if r:
            cname = name.replace("_accurate", "")
            out.append(f"{name} {r['tflops']:.1f} TF/s {r['frac_of_peak']:.3f} of peak{cpu_of(cname, 'TF/s')}")
    hbm = res.get("measured_hbm_GBs", {}).get("GBs")
    if hbm:
        out.append(f"measured_hbm {hbm:.0f} GB/s")
    for M, r in res.get("skinny_fp16_4096x4096", {}).items():
        out.append(f"skinny_{M} {r['us_per_call']:.2f} us {r['GBs']:.0f} GB/s {r.get('frac_of_measured_hbm', 0):.3f} of "
                   f"hbm{cpu_of('skinny_' + M, 'us')}")
    for M, r in res.get("skinny_kn_fp16_4096x4096", {}).items():
        out.append(f"skinny_kn_{M} {r['us_per_call']:.2f} us {r['GBs']:.0f} GB/s {r.get('frac_of_measured_hbm', 0):.3f} "
                   f"of hbm")
    for key in ("saxpy_2^26", "sdot_2^26", "sgemv_N_16384", "sgemv_T_16384"):
        r = res.get(key)
        if r:
            out.append(f"{key} {r['GBs']:.0f} GB/s {r.get('frac_of_measured_hbm', 0):.3f} of hbm{cpu_of(key, 'GB/s')}")
    return out


def cpu_baselines(budget_s=40.0):
    """The reference's CPU path (its BLAS layer forwards to OpenBLAS; HGEMM and skinny are NumPy FP32 math on the
    FP16 inputs, reference: lib/src/cblas.c:43-56, bench/gemm_cpu.py:33-37, bench/l12_cpu.py:13-16) on the host
    cores, for every benchmarked configuration: best of up to 5 timed runs after one warm-up, on the same inputs as the
    GPU cases. Returns (the HGEMM n = 4096 entry, which is `cpu_baseline`, {config: entry}). Bounded: each config stops
    after ~3 s of runs and the whole set after `budget_s`."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    from scipy.linalg import blas
    threads = min(16, os.cpu_count() or 1)
    try:
        from threadpoolctl import threadpool_limits
        lim = threadpool_limits(threads)
    except Exception:
        lim = None
    ver, nth = oracle.openblas_info()
    cores = nth or threads
    t_all = time.perf_counter() + budget_s
    out = {}

    def best_of(fn, per_s=3.0):
        fn()
        ts, t_end = [], time.perf_counter() + per_s
        for _ in range(5):
            t = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t)
            if time.perf_counter() > t_end:
                break
        return min(ts), len(ts)

    def entry(name, value, unit, sample):
        out[name] = {"value": value, "unit": unit, "cores": cores, "kind": "port",
                     "sample": f"{sample}; OpenBLAS {ver}, {cores} threads on {os.cpu_count()} cpus"}

    rng = np.random.default_rng
    for n in (4096, 1024, 2048):
        if time.perf_counter() > t_all:
            break
        A = oracle.normal((n, n), np.float16, oracle.SEED_A)
        B = oracle.normal((n, n), np.float16, oracle.SEED_B)
        t, k = best_of(lambda: oracle.cpu_path.hgemm(A, B))
        entry(f"hgemm_n{n}", round(2.0 * n ** 3 / t / 1e12, 4), "TFLOPS",
              f"NumPy FP32 matmul of the FP16 inputs (H and HS alike), n={n}, best of {k}")
    for kind, dt in (("sgemm", np.float32), ("dgemm", np.float64)):
        for n in (1024, 4096):
            if time.perf_counter() > t_all:
                break
            A = rng(1).uniform(-1, 1, (n, n)).astype(dt)
            B = rng(2).uniform(-1, 1, (n, n)).astype(dt)
            t, k = best_of(lambda: A @ B)
            entry(f"{kind}_n{n}", round(2.0 * n ** 3 / t / 1e12, 4), "TFLOPS", f"NumPy {kind} n={n}, best of {k}")
    if time.perf_counter() < t_all:
        M, N, K = 3000, 11008, 4096
        A = rng(1).uniform(-1, 1, (M, K)).astype(np.float32)
        Bt = rng(2).uniform(-1, 1, (N, K)).astype(np.float32)
        C0 = rng(3).uniform(-1, 1, (M, N)).astype(np.float32)
        # one OpenBLAS sgemm with beta, in place: C (column-major view Cᵀ, N×M) = Bt·Aᵀ + 0.5·Cᵀ
        Cw = np.array(C0.T, order="F")
        t, k = best_of(lambda: blas.sgemm(1.0, Bt.T, A.T, beta=0.5, c=Cw, trans_a=1, overwrite_c=1))
        entry("sgemm_odd_3000x11008x4096_tB_beta05", round(2.0 * M * N * K / t / 1e12, 4), "TFLOPS",
              f"scipy.linalg.blas.sgemm (beta = 0.5), best of {k}")
    if time.perf_counter() < t_all:
        K = N = 4096
        Ws = [oracle.normal((N, K), np.float16, 100 + c, 0.02) for c in range(4)]
        for M in (1, 2, 4, 8, 16):
            A = oracle.normal((M, K), np.float16, oracle.SEED_A)
            state = {"j": 0}

            def call():
                state["j"] = (state["j"] + 1) % len(Ws)
                oracle.cpu_path.skinny(A, Ws[state["j"]])
            t, k = best_of(call, per_s=1.0)
            entry(f"skinny_M{M}", round(t * 1e6, 1), "us_per_call",
                  f"NumPy FP32 A·Wᵀ of the FP16 inputs (FP16→FP32 conversion of W included), 4 rotated W copies, "
                  f"best of {k}")
    if time.perf_counter() < t_all:
        n = 1 << 26
        x = rng(20).uniform(-1, 1, n).astype(np.float32)
        y = rng(21).uniform(-1, 1, n).astype(np.float32)
        t, k = best_of(lambda: blas.saxpy(x, y, a=0.5))
        entry("saxpy_2^26", round(12.0 * n / t / 1e9, 1), "GB/s", f"scipy.linalg.blas.saxpy, best of {k}")
        t, k = best_of(lambda: blas.sdot(x, y))
        entry("sdot_2^26", round(8.0 * n / t / 1e9, 1), "GB/s", f"scipy.linalg.blas.sdot, best of {k}")
        del x, y
    if time.perf_counter() < t_all:
        m = 16384
        A = rng(1).uniform(-1, 1, (m, m)).astype(np.float32)
        xv = rng(20).uniform(-1, 1, m).astype(np.float32)
        for tr in (0, 1):
            t, k = best_of(lambda: A.T @ xv if tr else A @ xv)
            entry(f"sgemv_{'T' if tr else 'N'}_16384", round((4.0 * m * m + 8.0 * m) / t / 1e9, 1), "GB/s",
                  f"NumPy float32 matrix-vector (OpenBLAS sgemv), best of {k}")
        del A
    if lim is not None and hasattr(lim, "unregister"):
        lim.unregister()
    head = out.get("hgemm_n4096")
    if head:
        head = dict(head, sample="HGEMM n=4096 on the reference CPU path: " + head["sample"])
    return head, out


if __name__ == "__main__":
    main()
