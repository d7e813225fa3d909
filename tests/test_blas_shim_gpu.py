"""libgen9blas_blas.so on a GPU (GEN9BLAS_BLAS=auto): where each call runs, and its results.

Routing (GEN9BLAS_BLAS_INFO=1 names the side of every routed call): host-memory level 3 above the flop threshold
(1e9) and any call of 2^16 elements or more with device operands run on the GPU; smaller level 3 and host-memory
level 1-2 stay on the CPU BLAS. Results
against float64 closed forms under the reference's BLAS-test bounds (reference: lib/test_blas.py, lib/test_blas_d.py:
1e-5 FP32, 1e-12 FP64), the mixed dots under FP64 accuracy (the GPU accumulates in FP64).
"""
import os

import numpy as np
import pytest

import blas_shim_util as U

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(6)
TOL = {"s": 1e-5, "d": 1e-12}
DT = {"s": np.float32, "d": np.float64}


@pytest.fixture(scope="module")
def L(g9):
    os.environ["GEN9BLAS_BLAS_INFO"] = "1"   # read at the shim's first routed call
    os.environ.pop("GEN9BLAS_BLAS", None)
    os.environ.pop("GEN9BLAS_BLAS_L3_MIN", None)
    return U.load()


def routes(capfd):
    return [l.split("-> ")[1] for l in capfd.readouterr().err.splitlines() if l.startswith("gen9blas_blas:") and "->" in l]


@pytest.mark.parametrize("P", ["s", "d"])
@pytest.mark.parametrize("order", [U.ROW, U.COL])
def test_gemm_host_routes_by_size(L, capfd, P, order):
    dt = DT[P]
    for n, side in ((96, "CPU"), (512, "CPU"), (1024, "GPU")):
        A, B = rng.uniform(-1, 1, (n, n)).astype(dt), rng.uniform(-1, 1, (n, n)).astype(dt)
        C0 = rng.uniform(-1, 1, (n, n)).astype(dt)
        C = C0.copy()
        capfd.readouterr()
        # column-major call on the same buffers computes Cᵀ = Aᵀ·Bᵀ... in row-major terms: C = B·A for these arrays
        getattr(L, f"cblas_{P}gemm")(order, U.NT, U.T, n, n, n, 1.0, U.ptr(A), n, U.ptr(B), n, 0.5, U.ptr(C), n)
        assert routes(capfd) == [side], (n, side)
        Ad, Bd = A.astype(np.float64), B.astype(np.float64)
        if order == U.ROW:
            ref, scale = Ad @ Bd.T, np.abs(Ad) @ np.abs(Bd.T)
        else:
            ref, scale = (Ad.T @ Bd).T, (np.abs(Ad.T) @ np.abs(Bd)).T
        assert U.ref_error(C, ref + 0.5 * C0, scale + 0.5 * np.abs(C0)) <= TOL[P]


@pytest.mark.parametrize("P", ["s", "d"])
def test_fortran_gemm_on_gpu(L, capfd, P):
    dt = DT[P]
    M, N, K = 1000, 1100, 900   # 2e9 flops: above the host-memory threshold
    A = np.asfortranarray(rng.uniform(-1, 1, (M, K)).astype(dt))
    B = np.asfortranarray(rng.uniform(-1, 1, (N, K)).astype(dt))    # op(B) = Bᵀ
    C = np.asfortranarray(np.zeros((M, N), dt))
    capfd.readouterr()
    U.fortran_gemm(L, P, "N", "T", M, N, K, 1.0, A, M, B, N, 0.0, C, M)
    assert routes(capfd) == ["GPU"]
    Ad, Bd = A.astype(np.float64), B.astype(np.float64)
    assert U.ref_error(C, Ad @ Bd.T, np.abs(Ad) @ np.abs(Bd.T)) <= TOL[P]


@pytest.mark.parametrize("P", ["s", "d"])
def test_level12_host_stays_on_cpu_device_goes_to_gpu(L, capfd, torch_dev, P):
    torch = torch_dev
    dt = DT[P]
    n = 1 << 20
    x, y = rng.uniform(-1, 1, n).astype(dt), rng.uniform(-1, 1, n).astype(dt)
    X, Y = x.astype(np.float64), y.astype(np.float64)
    capfd.readouterr()
    got = getattr(L, f"cblas_{P}dot")(n, U.ptr(x), 1, U.ptr(y), 1)
    assert routes(capfd) == ["CPU"]
    assert abs(got - X @ Y) <= TOL[P] * (abs(X) @ abs(Y))
    xd, yd = torch.from_numpy(x).cuda(), torch.from_numpy(y).cuda()
    got = getattr(L, f"cblas_{P}dot")(n, U.ptr(xd), 1, U.ptr(yd), 1)
    getattr(L, f"cblas_{P}axpy")(n, 0.5, U.ptr(xd), 1, U.ptr(yd), 1)
    assert routes(capfd) == ["GPU", "GPU"]
    # FP64 accumulation on the GPU, then (sdot) one rounding of the result to float
    assert abs(got - X @ Y) <= 1e-12 * (abs(X) @ abs(Y)) + (6e-8 * abs(X @ Y) if P == "s" else 0)
    assert U.ref_error(yd.cpu().numpy(), 0.5 * X + Y, 0.5 * abs(X) + abs(Y)) <= TOL[P]
    M, N = 1000, 3000
    A = rng.uniform(-1, 1, (M, N)).astype(dt)
    v = rng.uniform(-1, 1, M).astype(dt)
    Ad, vd = torch.from_numpy(A).cuda(), torch.from_numpy(v).cuda()
    out = torch.zeros(N, dtype=Ad.dtype, device="cuda")
    # column-major view of the row-major A is Aᵀ (N×M, lda = N): y = Aᵀ·v
    getattr(L, f"cblas_{P}gemv")(U.COL, U.NT, N, M, 1.0, U.ptr(Ad), N, U.ptr(vd), 1, 0.0, U.ptr(out), 1)
    assert routes(capfd) == ["GPU"]
    Af = A.astype(np.float64)
    assert U.ref_error(out.cpu().numpy(), Af.T @ v, np.abs(Af.T) @ np.abs(v.astype(np.float64))) <= TOL[P]


def test_mixed_dots_fp64_on_device(L, capfd, torch_dev):
    torch = torch_dev
    v, w = rng.uniform(-1, 1, 100003).astype(np.float32), rng.uniform(-1, 1, 100003).astype(np.float32)
    exact = v.astype(np.float64) @ w.astype(np.float64)
    vd, wd = torch.from_numpy(v).cuda(), torch.from_numpy(w).cuda()
    capfd.readouterr()
    assert abs(L.cblas_dsdot(v.size, U.ptr(vd), 1, U.ptr(wd), 1) - exact) <= 1e-12 * (np.abs(v) @ np.abs(w))
    got = L.cblas_sdsdot(v.size, 0.25, U.ptr(vd), 1, U.ptr(wd), 1)   # FP64 sum, one rounding to float
    assert abs(got - (0.25 + exact)) <= 6e-8 * abs(0.25 + exact)
    assert routes(capfd) == ["GPU", "GPU"]


L3_BIG = {"symm": (800, 800), "syrk": (800, 1600), "syr2k": (800, 800), "trmm": (1000, 1000), "trsm": (1000, 1000)}


def _l3_run(L, P, op, opt, order, dims, torch=None):
    """One level-3 call through the shim on fresh random operands; returns the error against the float64 closed form
    and whether the entries outside the defined triangle stayed as they were."""
    dt = DT[P]
    A, B, C0 = U.l3_case(rng, dt, op, opt, dims)
    a, b, c = (U.to_mem(X, order, torch) for X in (A, B, C0))
    U.call_l3(L, P, order, op, opt, dims, 0.75, -0.5, a[:2], b[:2], c[:2])
    if torch is not None:
        torch.cuda.synchronize()
    tgt = c if op in ("symm", "syrk", "syr2k") else b
    got = tgt[2](tgt[0])
    ref, scale, mask = U.l3_ref(op, opt, 0.75, -0.5, A, B, C0)
    kept = mask is None or np.array_equal(got[~mask], C0.astype(np.float64)[~mask])
    return U.l3_error(op, got, ref, scale, mask), kept


@pytest.mark.parametrize("P", ["s", "d"])
@pytest.mark.parametrize("op", U.L3)
def test_level3_host_routes_by_size(L, capfd, P, op):
    """Host-memory SYMM/SYRK/SYR2K/TRMM/TRSM: the GPU from 1e9 flops, the CPU BLAS below; CBLAS both orders and
    Fortran give BLAS results either way."""
    tol = U.L3_TRSM_TOL[P] if op == "trsm" else U.L3_TOL[P]
    opt = U.L3_OPTS[op][-1]
    big = L3_BIG[op]
    for dims, side in ((big, "GPU"), ((big[0] // 4, big[1] // 4), "CPU")):
        for order in (U.ROW, U.COL, "F"):
            capfd.readouterr()
            err, kept = _l3_run(L, P, op, opt, order, dims)
            assert routes(capfd) == [side], (dims, order)
            assert err <= tol and kept, (dims, order, err)


@pytest.mark.parametrize("P", ["s", "d"])
@pytest.mark.parametrize("op", U.L3)
def test_level3_device_operands_every_option(L, capfd, torch_dev, P, op):
    """Device operands go to the GPU at any size over 2^16 elements: every side / triangle / transpose / diagonal in
    CBLAS row- and column-major and Fortran, i.e. every mapping of a column-major call onto the row-major library."""
    tol = U.L3_TRSM_TOL[P] if op == "trsm" else U.L3_TOL[P]
    dims = (280, 200) if op in ("syrk", "syr2k") else (300, 260)
    for opt in U.L3_OPTS[op]:
        for order in (U.ROW, U.COL, "F"):
            capfd.readouterr()
            err, kept = _l3_run(L, P, op, opt, order, dims, torch_dev)
            assert routes(capfd) == ["GPU"], (opt, order)
            assert err <= tol and kept, (opt, order, err)


L2_DIMS = {"symv": (300, 0), "trmv": (300, 0), "trsv": (300, 0), "syr": (300, 0), "syr2": (300, 0),
           "sbmv": (1500, 50), "tbmv": (1500, 50), "tbsv": (1500, 50), "gbmv": (1500, 50),
           "spmv": (400, 0), "tpmv": (400, 0), "tpsv": (400, 0), "spr": (400, 0), "spr2": (400, 0)}


@pytest.mark.parametrize("P", ["s", "d"])
@pytest.mark.parametrize("op", U.L2)
def test_level2_device_operands_every_option(L, capfd, torch_dev, P, op):
    """Symmetric / triangular / band / packed level 2 with device operands (2^16 elements and more) run on the GPU:
    every triangle / transpose / diagonal in CBLAS row- and column-major and Fortran, i.e. every mapping of a
    column-major call onto the row-major library. Host operands stay on the CPU BLAS (one pass over host memory)."""
    n, K = L2_DIMS[op]
    tol = 1e-4 if P == "s" else 1e-12
    for o in U.l2_opts(op):
        for order in (U.ROW, U.COL, "F"):
            capfd.readouterr()
            err = U.l2_run(L, P, op, o, order, n, K, rng, DT[P], torch_dev)
            assert routes(capfd) == ["GPU"], (o, order)
            assert err <= tol, (o, order, err)
    capfd.readouterr()
    err = U.l2_run(L, P, op, U.l2_opts(op)[0], U.ROW, n, K, rng, DT[P])
    assert routes(capfd) == ["CPU"] and err <= tol


def test_ld_preload_interposition_gpu(g9, tmp_path):
    """An unmodified program linked against another BLAS (a stub whose GEMMs write -1) gets the shim's cblas_sgemm and
    sgemm_ once libgen9blas_blas.so is in LD_PRELOAD (reference: README.md:9-10); both products are above the shim's
    level-3 threshold, so they run on the GPU (routing log, GEN9BLAS_BLAS_INFO) and match float64 to the SGEMM bound;
    with GEN9BLAS_BLAS=cpu the same program runs them on the CPU BLAS."""
    prog = U.build_preload_program(tmp_path)
    plain, _ = U.run_preload_program(prog, preload=False)
    assert plain["cblas_sgemm"] > 1e-2 and plain["sgemm_"] > 1e-2        # the stub ran (it writes -1)
    errs, log = U.run_preload_program(prog, preload=True)
    assert errs["cblas_sgemm"] <= 1e-6 and errs["sgemm_"] <= 1e-6, errs
    assert log.count("sgemm -> GPU") == 2, log[-1000:]                    # both calls (the log names the routine)
    errs, log = U.run_preload_program(prog, preload=True, extra_env={"GEN9BLAS_BLAS": "cpu"})
    assert errs["cblas_sgemm"] <= 1e-5 and errs["sgemm_"] <= 1e-5, errs
    assert "-> GPU" not in log
