"""The C ABI surface of libgen9blas.so, checked without a GPU.

- Every function declared in include/*.h is exported, and nothing else is (kernel stubs and C++ internals stay local).
- The version is 0.2.0 (reference: lib/gen9blas.h:20-23) and the ctypes module loads the library.
- Without a usable device, every entry point reports GEN9BLAS_ERR_NO_DEVICE (-5), permanently, with a message
  (reference status codes: lib/gen9blas.h:38-46); pointer-returning functions return NULL and set the last status;
  a host result pointer of a reduction is zeroed first (reference: lib/src/level12.c:172).
No kernel is launched: these tests run in a container without a GPU (they skip where one is present).
"""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.realpath(__file__)))
LIB = os.path.join(ROOT, "gen9-gpu-blas_amd", "libgen9blas.so")
HEADERS = [os.path.join(ROOT, "include", h) for h in ("gen9blas.h", "gen9blas_hip.h", "gen9blas_ml.h")]


def declared():
    names = set()
    for h in HEADERS:
        text = open(h).read()
        names |= set(re.findall(r"GEN9BLAS_API\s+[\w\s\*]+?\b(gen9blas_\w+)\s*\(", text))
    return names


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if l.strip()}


def gpu_present():
    return os.path.exists("/dev/kfd")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail("libgen9blas.so is not built: run python gen9-gpu-blas_amd/build.py")
    L = ctypes.CDLL(LIB)
    L.gen9blas_error.restype = ctypes.c_char_p
    L.gen9blas_alloc.restype = ctypes.c_void_p
    L.gen9blas_alloc.argtypes = [ctypes.c_size_t]
    L.gen9blas_pack_b.restype = ctypes.c_void_p
    L.gen9blas_device_alloc.restype = ctypes.c_void_p
    L.gen9blas_device_alloc.argtypes = [ctypes.c_size_t]
    L.gen9blas_hip_stream.restype = ctypes.c_void_p
    return L


def test_header_declares_the_reference_surface():
    names = declared()
    # the hot-path entry points of the reference header, with the library-state functions around them
    for f in ("gen9blas_gemm", "gen9blas_gemm_batched", "gen9blas_hgemm", "gen9blas_sgemm", "gen9blas_axpy",
              "gen9blas_dot", "gen9blas_gemv", "gen9blas_version", "gen9blas_init", "gen9blas_device_gen",
              "gen9blas_has", "gen9blas_error", "gen9blas_last_status", "gen9blas_last_time_ms",
              "gen9blas_last_zero_copy", "gen9blas_alloc", "gen9blas_free", "gen9blas_is_usm"):
        assert f in names, f
    assert "gen9blas_gemm_pb_skinny" in names   # the packed-weight decode entry of the reference's ML header
    assert "gen9blas_gemm_noalloc" in names     # MI355X addition: gen9blas_gemm without allocations
    assert len(names) == 61


def test_exports_exactly_the_header(lib):
    names, syms = declared(), exported()
    missing = names - syms
    assert not missing, f"declared but not exported: {sorted(missing)}"
    extra = {s for s in syms if not s.startswith("gen9blas_")}
    assert not extra, f"exported beyond the C ABI: {sorted(extra)[:10]}"
    assert syms - names == set(), f"exported but not declared: {sorted(syms - names)}"
    for f in names:
        assert hasattr(lib, f)


def test_version_and_constants(lib):
    assert lib.gen9blas_version() == 200
    text = open(HEADERS[0]).read()
    for name, val in (("GEN9BLAS_H", 0), ("GEN9BLAS_S", 1), ("GEN9BLAS_HS", 2), ("GEN9BLAS_D", 3)):
        assert re.search(rf"\b{name} = {val}\b", text), name
    for name, val in (("GEN9BLAS_OK", 0), ("GEN9BLAS_DECLINED", 1), ("GEN9BLAS_ERR", -1),
                      ("GEN9BLAS_ERR_UNSUPPORTED", -2), ("GEN9BLAS_ERR_INVALID_ARG", -3),
                      ("GEN9BLAS_ERR_OUT_OF_MEMORY", -4), ("GEN9BLAS_ERR_NO_DEVICE", -5)):
        assert re.search(rf"\b{name} = {val}\b", text), name
    assert re.search(r"#define GEN9BLAS_KC 32", text)


def test_ctypes_module_loads():
    import gen9blas
    assert gen9blas._lib.gen9blas_version() // 100 == 2
    for f in ("hgemm", "sgemm", "gemm", "gemm_batched", "gemv", "dot", "axpy", "asum", "nrm2", "iamax",
              "scal", "copy", "swap", "rot", "ger", "empty", "set_nowait", "flush", "hip_stream"):
        assert callable(getattr(gen9blas, f)), f


@pytest.mark.skipif(gpu_present(), reason="a GPU is present: the no-device path is not reachable")
def test_no_device_status(lib):
    NO_DEV = -5
    assert lib.gen9blas_init() == NO_DEV
    msg = lib.gen9blas_error()
    assert msg and b"device" in msg.lower()
    assert lib.gen9blas_init() == NO_DEV          # permanent for the process
    assert lib.gen9blas_device_gen() == 0
    assert lib.gen9blas_device_arch() == 0
    assert lib.gen9blas_has(0) == 0
    d = ctypes.c_double
    assert lib.gen9blas_gemm(1, 0, 0, 8, 8, 8, d(1.0), None, 8, None, 8, d(0.0), None, 8) == NO_DEV
    assert lib.gen9blas_last_status() == NO_DEV
    assert lib.gen9blas_axpy(1, 8, d(1.0), None, 1, None, 1) == NO_DEV
    r = ctypes.c_double(5.0)
    assert lib.gen9blas_dot(1, 4, None, 1, None, 1, ctypes.byref(r)) == NO_DEV
    assert r.value == 0.0                          # host result zeroed before anything else
    assert lib.gen9blas_alloc(64) is None
    assert lib.gen9blas_last_status() == NO_DEV
    assert lib.gen9blas_device_alloc(64) is None
    assert lib.gen9blas_pack_b(1, 0, 8, 8, None, 8) is None
    assert lib.gen9blas_last_status() == NO_DEV
    assert lib.gen9blas_flush() in (0, NO_DEV)
