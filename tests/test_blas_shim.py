"""libgen9blas_blas.so (the BLAS / CBLAS shim) without a GPU: every call must reach the CPU BLAS with BLAS results.

Checks the reference BLAS layer's contract (reference: lib/src/cblas.c:1-562, lib/test_blas.py, lib/test_blas_d.py)
on the CPU side: the library loads and finds a CPU BLAS, it exports its own S/D entry points plus a forwarding stub
for every other BLAS/CBLAS symbol of that CPU BLAS, row- and column-major CBLAS calls and Fortran calls give the
float64 closed-form results (bounds 1e-5 FP32 / 1e-12 FP64 as in the reference's tests), the level-3 functions the
shim routes itself (SYMM, SYRK, SYR2K, TRMM, TRSM and the symmetric / triangular / band / packed level 2) pass every
option through, and forwarded functions (here complex GEMV) work. Without a device the routing sends everything to the CPU, so these run anywhere.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import blas_shim_util as U

rng = np.random.default_rng(5)
TOL = {"s": 1e-5, "d": 1e-12}
DT = {"s": np.float32, "d": np.float64}


@pytest.fixture(scope="module")
def L():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present: the GPU module covers the shim there")
    if not os.path.exists(U.SHIM):
        pytest.fail("libgen9blas_blas.so is not built: run python gen9-gpu-blas_amd/build.py")
    return U.load()


def test_exports(L):
    out = subprocess.run(["nm", "-D", "--defined-only", U.SHIM], capture_output=True, text=True, check=True).stdout
    syms = {l.split()[-1] for l in out.splitlines() if l.strip()}
    assert U.OWN <= syms
    blas = {s for s in syms if s.startswith("cblas_") or s.endswith("_") or s == "__xerbla"}
    assert len(blas) == len(syms), f"non-BLAS exports: {sorted(syms - blas)[:10]}"
    for s in ("cblas_zgemm", "cblas_csyrk", "dtrsm_", "cblas_sgbmv", "xerbla_", "__xerbla", "cblas_dtrsv", "zdotc_"):
        assert s in syms, s
    assert len(syms) > 300


@pytest.mark.parametrize("P", ["s", "d"])
@pytest.mark.parametrize("order", [U.ROW, U.COL])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_cblas_gemm(L, P, order, ta, tb):
    dt = DT[P]
    M, N, K = 37, 29, 45
    opA = rng.uniform(-1, 1, (M, K)).astype(dt)
    opB = rng.uniform(-1, 1, (K, N)).astype(dt)
    C0 = rng.uniform(-1, 1, (M, N)).astype(dt)
    A = opA.T.copy() if ta else opA
    B = opB.T.copy() if tb else opB
    if order == U.COL:   # column-major storage of the same matrices
        Af, Bf, C = np.asfortranarray(A), np.asfortranarray(B), np.asfortranarray(C0.copy())
        lda, ldb, ldc = A.shape[0], B.shape[0], M
    else:
        Af, Bf, C = A, B, C0.copy()
        lda, ldb, ldc = A.shape[1], B.shape[1], N
    getattr(L, f"cblas_{P}gemm")(order, U.T if ta else U.NT, U.T if tb else U.NT, M, N, K, 1.5, U.ptr(Af), lda,
                                 U.ptr(Bf), ldb, -0.5, U.ptr(C), ldc)
    ref = 1.5 * opA.astype(np.float64) @ opB + -0.5 * C0
    scale = 1.5 * np.abs(opA.astype(np.float64)) @ np.abs(opB) + 0.5 * np.abs(C0)
    assert U.ref_error(C, ref, scale) <= TOL[P]


@pytest.mark.parametrize("P", ["s", "d"])
def test_fortran_gemm(L, P):
    dt = DT[P]
    M, N, K = 20, 33, 17
    A = np.asfortranarray(rng.uniform(-1, 1, (K, M)).astype(dt))    # op(A) = Aᵀ
    B = np.asfortranarray(rng.uniform(-1, 1, (K, N)).astype(dt))
    C = np.asfortranarray(np.zeros((M, N), dt))
    U.fortran_gemm(L, P, "t", "N", M, N, K, 2.0, A, K, B, K, 0.0, C, M)
    ref = 2.0 * A.T.astype(np.float64) @ B
    assert U.ref_error(C, ref, 2.0 * np.abs(A.T.astype(np.float64)) @ np.abs(B)) <= TOL[P]


@pytest.mark.parametrize("P", ["s", "d"])
def test_gemv_ger_level1(L, P):
    dt = DT[P]
    M, N = 50, 70
    A = rng.uniform(-1, 1, (M, N)).astype(dt)
    x, y = rng.uniform(-1, 1, N).astype(dt), rng.uniform(-1, 1, M).astype(dt)
    y0 = y.copy()
    getattr(L, f"cblas_{P}gemv")(U.ROW, U.NT, M, N, 1.0, U.ptr(A), N, U.ptr(x), 1, 0.5, U.ptr(y), 1)
    ref = A.astype(np.float64) @ x + 0.5 * y0
    assert U.ref_error(y, ref, np.abs(A.astype(np.float64)) @ np.abs(x) + 0.5 * np.abs(y0)) <= TOL[P]
    A2 = A.copy()
    getattr(L, f"cblas_{P}ger")(U.COL, N, M, -1.0, U.ptr(x), 1, U.ptr(y0), 1, U.ptr(A2), N)   # Aᵀ col-major = A
    assert U.ref_error(A2, A - np.outer(y0, x), np.abs(A) + np.abs(np.outer(y0, x))) <= TOL[P]
    v, w = rng.uniform(-1, 1, 1000).astype(dt), rng.uniform(-1, 1, 1000).astype(dt)
    V, W = v.astype(np.float64), w.astype(np.float64)
    assert abs(getattr(L, f"cblas_{P}dot")(1000, U.ptr(v), 1, U.ptr(w), 1) - V @ W) <= TOL[P] * (abs(V) @ abs(W))
    assert abs(getattr(L, f"cblas_{P}asum")(1000, U.ptr(v), 1) - abs(V).sum()) <= TOL[P] * abs(V).sum()
    assert abs(getattr(L, f"cblas_{P}nrm2")(1000, U.ptr(v), 1) - np.linalg.norm(V)) <= TOL[P] * np.linalg.norm(V)
    assert getattr(L, f"cblas_i{P}amax")(1000, U.ptr(v), 1) == int(np.argmax(abs(V)))
    getattr(L, f"cblas_{P}axpy")(1000, 0.25, U.ptr(v), 1, U.ptr(w), 1)
    assert U.ref_error(w, 0.25 * V + W, 0.25 * abs(V) + abs(W)) <= TOL[P]
    getattr(L, f"cblas_{P}scal")(500, -2.0, U.ptr(v), 2)
    assert np.array_equal(v[::2], (-2.0 * V[::2]).astype(dt)) and np.array_equal(v[1::2], V[1::2].astype(dt))


def test_mixed_precision_dots(L):
    """On the CPU these are the CPU BLAS's own (SciPy's OpenBLAS sums dsdot in FP32: 1e-6, not FP64 accuracy)."""
    v, w = rng.uniform(-1, 1, 999).astype(np.float32), rng.uniform(-1, 1, 999).astype(np.float32)
    exact = v.astype(np.float64) @ w.astype(np.float64)
    scale = np.abs(v).astype(np.float64) @ np.abs(w)
    assert abs(L.cblas_dsdot(999, U.ptr(v), 1, U.ptr(w), 1) - exact) <= 1e-5 * scale
    assert abs(L.cblas_sdsdot(999, 0.5, U.ptr(v), 1, U.ptr(w), 1) - (0.5 + exact)) <= 1e-5 * scale


@pytest.mark.parametrize("P", ["c", "z"])
def test_forwarded_complex_gemv(L, P):
    """A function the shim forwards to the CPU BLAS by a tail jump (complex GEMV: not routed): results as BLAS."""
    dt = np.complex64 if P == "c" else np.complex128
    A = (rng.uniform(-1, 1, (30, 20)) + 1j * rng.uniform(-1, 1, (30, 20))).astype(dt)
    x = (rng.uniform(-1, 1, 20) + 1j * rng.uniform(-1, 1, 20)).astype(dt)
    y = np.zeros(30, dt)
    one, zero = np.array([1.0 + 0j], dt), np.array([0j], dt)
    fn = getattr(L, f"cblas_{P}gemv")
    fn.argtypes = [U.i, U.i, U.i, U.i, U.p, U.p, U.i, U.p, U.i, U.p, U.p, U.i]
    fn(U.ROW, U.NT, 30, 20, U.ptr(one), U.ptr(A), 20, U.ptr(x), 1, U.ptr(zero), U.ptr(y), 1)
    A64 = A.astype(np.complex128)
    assert U.ref_error(np.abs(y - A64 @ x), 0, np.abs(A64) @ np.abs(x)) <= (1e-5 if P == "c" else 1e-12)


@pytest.mark.parametrize("P", ["s", "d"])
@pytest.mark.parametrize("op", U.L3)
def test_level3_routed_functions_on_cpu(L, P, op):
    """SYMM/SYRK/SYR2K/TRMM/TRSM through the shim's own entry points (CBLAS row- and column-major, Fortran), every
    side / triangle / transpose / diagonal: without a device they reach the CPU BLAS with arguments intact."""
    dt = DT[P]
    dims = (23, 31) if op in ("syrk", "syr2k") else (29, 19)
    for opt in U.L3_OPTS[op]:
        for order in (U.ROW, U.COL, "F"):
            A, B, C0 = U.l3_case(rng, dt, op, opt, dims)
            a, b = U.to_mem(A, order), U.to_mem(B, order)
            c = U.to_mem(C0, order)
            tgt = c if op in ("symm", "syrk", "syr2k") else b
            U.call_l3(L, P, order, op, opt, dims, 0.75, -0.5, a[:2], b[:2], c[:2])
            got = tgt[2](tgt[0])
            ref, scale, mask = U.l3_ref(op, opt, 0.75, -0.5, A, B, C0)
            tol = U.L3_TRSM_TOL[P] if op == "trsm" else U.L3_TOL[P]
            assert U.l3_error(op, got, ref, scale, mask) <= tol, (opt, order)
            if mask is not None:
                assert np.array_equal(got[~mask], C0.astype(np.float64)[~mask]), (opt, order)


@pytest.mark.parametrize("P", ["s", "d"])
@pytest.mark.parametrize("op", U.L2)
def test_level2_every_option_cpu(L, P, op):
    """SYMV/SBMV/SPMV, TRMV/TRSV/TBMV/TBSV/TPMV/TPSV, SYR/SYR2/SPR/SPR2 and GBMV through the shim in CBLAS row- and
    column-major and Fortran, every triangle / transpose / diagonal: without a device every call reaches the CPU BLAS
    with its own arguments, and the results match the float64 closed forms (this also pins the tests' storage
    builders against OpenBLAS, the reference's CPU path)."""
    tol = 1e-4 if P == "s" else 1e-12
    for o in U.l2_opts(op):
        for order in (U.ROW, U.COL, "F"):
            err = U.l2_run(L, P, op, o, order, 30, 4, rng, DT[P])
            assert err <= tol, (o, order, err)


def test_ld_preload_interposition(L, tmp_path):
    """An unmodified program linked against another BLAS (a stub whose GEMMs write -1) gets the shim's cblas_sgemm and
    sgemm_ once libgen9blas_blas.so is in LD_PRELOAD (reference: README.md:9-10). Without a GPU the shim routes them
    to the CPU BLAS, and the routing log (GEN9BLAS_BLAS_INFO) says so; the results match float64 to 1e-5."""
    prog = U.build_preload_program(tmp_path)
    plain, _ = U.run_preload_program(prog, preload=False)
    assert plain["cblas_sgemm"] > 1e-2 and plain["sgemm_"] > 1e-2        # the stub ran (it writes -1)
    errs, log = U.run_preload_program(prog, preload=True)
    assert errs["cblas_sgemm"] <= 1e-5 and errs["sgemm_"] <= 1e-5, errs
    assert "cblas_sgemm -> CPU" in log and "sgemm_ -> CPU" in log, log[-1000:]
