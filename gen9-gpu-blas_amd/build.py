"""Builds libgen9blas.so (HIP, gfx950) and libgen9blas_blas.so (CBLAS/BLAS shim) in this directory.

    python gen9-gpu-blas_amd/build.py            # rebuild what changed
    python gen9-gpu-blas_amd/build.py --force    # rebuild everything

The libraries are written next to this file (git-ignored), object files under _build/; libgen9blas_calib.so holds
the calibration kernels bench.py measures ceilings with and is not part of the library. hipcc cross-compiles for gfx950
without a GPU. Replaces the reference's CMake + ocloc kernel-table build (reference: lib/CMakeLists.txt): the HIP
kernels are compiled into the library, there is no separate kernel table.
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.realpath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
INCLUDE = os.path.join(ROOT, "include")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
LIB = os.path.join(HERE, "libgen9blas.so")
BLAS_LIB = os.path.join(HERE, "libgen9blas_blas.so")
CALIB_LIB = os.path.join(HERE, "libgen9blas_calib.so")   # bench.py's calibration kernels, not part of the library

HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++20", "-fPIC", "-fvisibility=hidden", "-I" + INCLUDE, "-I" + CSRC,
             # packed FP32 VALU forms are kept out of the generated code
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wall", "-Wno-unused-function"]
HIP_SOURCES = ["runtime.hip", "gemm.hip", "gemm_kernels.hip", "skinny.hip", "level12.hip", "level12_kernels.hip",
               "packed.hip", "level3.hip", "level2.hip", "noalloc.hip"]
# every header of csrc/ counts as a dependency of every object: a new header cannot be left out
HEADERS = sorted(f for f in os.listdir(CSRC) if f.endswith(".h"))


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    return err


def _stale(target, deps):
    if not os.path.exists(target):
        return True
    t = os.path.getmtime(target)
    return any(os.path.getmtime(d) > t for d in deps)


def build(force=False, jobs=None, verbose=True):
    os.makedirs(BUILD, exist_ok=True)
    hdr = [os.path.join(CSRC, h) for h in HEADERS] + [os.path.join(INCLUDE, h) for h in ("gen9blas.h", "gen9blas_hip.h", "gen9blas_ml.h")]
    objs, todo = [], []
    for s in HIP_SOURCES:
        src, obj = os.path.join(CSRC, s), os.path.join(BUILD, s.replace(".hip", ".o"))
        objs.append(obj)
        if force or _stale(obj, [src] + hdr):
            todo.append([HIPCC] + HIP_FLAGS + ["-c", src, "-o", obj])
    jobs = jobs or min(len(todo) or 1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 8)
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        for out in ex.map(_run, todo):
            if out.strip() and verbose:
                print(out, file=sys.stderr)
    if force or todo or _stale(LIB, objs + [os.path.join(CSRC, "exports.map")]):
        _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,-soname,libgen9blas.so",
              "-Wl,--version-script=" + os.path.join(CSRC, "exports.map"), "-o", LIB + ".tmp"] + objs)
        os.replace(LIB + ".tmp", LIB)
    _build_blas(force)
    _build_calib(force)
    return LIB


def _build_calib(force):
    """libgen9blas_calib.so: the calibration kernels bench.py measures ceilings with (calib/calibrate.hip)."""
    src = os.path.join(HERE, "calib", "calibrate.hip")
    if force or _stale(CALIB_LIB, [src]):
        _run([HIPCC] + HIP_FLAGS + ["-shared", "-o", CALIB_LIB + ".tmp", src])
        os.replace(CALIB_LIB + ".tmp", CALIB_LIB)


def _build_blas(force):
    """libgen9blas_blas.so: the BLAS / CBLAS shim (blas_shim/blas_shim.c) plus its generated forwarding stubs."""
    src = os.path.join(HERE, "blas_shim", "blas_shim.c")
    gen = os.path.join(HERE, "blas_shim", "gen_forward.py")
    hdr = [os.path.join(INCLUDE, h) for h in ("gen9blas.h", "gen9blas_hip.h")]
    obj = os.path.join(BUILD, "blas_shim.o")
    fwd_c, fwd_o = os.path.join(BUILD, "blas_forward.c"), os.path.join(BUILD, "blas_forward.o")
    cflags = ["gcc", "-O2", "-fPIC", "-std=gnu11", "-Wall", "-fvisibility=hidden", "-I" + INCLUDE]
    if force or _stale(obj, [src] + hdr):
        _run(cflags + ["-c", src, "-o", obj])
    if force or _stale(fwd_c, [obj, gen]):
        out = subprocess.run([sys.executable, gen, obj], capture_output=True, text=True, check=True).stdout
        with open(fwd_c, "w") as f:
            f.write(out)
    if force or _stale(fwd_o, [fwd_c]):
        _run(cflags + ["-c", fwd_c, "-o", fwd_o])
    if force or _stale(BLAS_LIB, [obj, fwd_o, LIB]):
        _run(["gcc", "-shared", "-fPIC", "-Wl,-soname,libgen9blas_blas.so", "-o", BLAS_LIB + ".tmp", obj, fwd_o,
              "-L" + HERE, "-lgen9blas", "-Wl,-rpath,$ORIGIN", "-ldl", "-lpthread"])
        os.replace(BLAS_LIB + ".tmp", BLAS_LIB)


if __name__ == "__main__":
    print(build(force="--force" in sys.argv))
