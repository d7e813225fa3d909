"""Level 1-2 parity on the GPU: axpy, scal, copy, swap, rot, dot, asum, nrm2, iamax, gemv (N and T), ger.

Follows the reference's level 1-2 test (reference: lib/test_level12.py:27-97): lengths 1, 5, 255, 256, 1000, 100003;
strides (1, 1), (1, 1) shifted, (3, −2), (−1, 1); GEMV on odd shapes, with beta, transposed views and submatrices.
Error relative to the formula scale (e.g. |a·x| + |y| for axpy, |A|·|x| for gemv): FP32 ≤ 1e-6, FP16 ≤ 2e-3,
FP64 ≤ 1e-13; reductions (FP64 on the GPU) ≤ 1e-6. The dot product is also compared with the oracle's FP64
restatement (reference: lib/kernels/level12.cl:189-214): both are FP64 sums of exact products and agree to 1e-12.
"""
import numpy as np
import pytest

from l12_util import assert_close, strided

pytestmark = pytest.mark.gpu

TOL = {np.float32: 1e-6, np.float16: 2e-3, np.float64: 1e-13}
REDUCTION_TOL = 1e-6   # FP64 sums on the GPU, returned as float64
rng = np.random.default_rng(11)

# (inc_x, inc_y, lead of x): the reference's stride cases (reference: lib/test_level12.py:49); y always starts one
# element into its array
STRIDES = [(1, 1, 0), (1, 1, 1), (3, -2, 5), (-1, 1, 2)]


def _both(X, Y):
    return np.concatenate([X, Y])


# Level-1 calls on the pair (x, y), each from the same starting values X, Y (float64): what the call is, which
# operand(s) it leaves its result in ("y", "xy": x then y, "ret": the return value), and the float64 result with its
# error scale. Tolerance: the type's for vectors, 0 for pure data movement, REDUCTION_TOL for the FP64 sums.
LEVEL1 = [
    ("axpy", lambda g, x, y: g.axpy(0.75, x, y), "y", lambda X, Y: (0.75 * X + Y, 0.75 * abs(X) + abs(Y)), None),
    ("scal", lambda g, x, y: g.scal(-1.5, y), "y", lambda X, Y: (-1.5 * Y, 1.5 * abs(Y)), None),
    ("copy", lambda g, x, y: g.copy(x, y), "y", lambda X, Y: (X, 1.0), 0.0),
    ("swap", lambda g, x, y: g.swap(x, y), "xy", lambda X, Y: (_both(Y, X), 1.0), 0.0),
    ("rot", lambda g, x, y: g.rot(x, y, 0.6, 0.8), "xy",
     lambda X, Y: (_both(0.6 * X + 0.8 * Y, 0.6 * Y - 0.8 * X), _both(abs(X) + abs(Y), abs(X) + abs(Y))), None),
    ("dot", lambda g, x, y: g.dot(x, y), "ret", lambda X, Y: (X @ Y, abs(X) @ abs(Y)), REDUCTION_TOL),
    ("asum", lambda g, x, y: g.asum(x), "ret", lambda X, Y: (abs(X).sum(), abs(X).sum()), REDUCTION_TOL),
    ("nrm2", lambda g, x, y: g.nrm2(x), "ret", lambda X, Y: (np.sqrt(X @ X), np.sqrt(X @ X)), REDUCTION_TOL),
]


@pytest.mark.parametrize("dt", [np.float32, np.float16, np.float64])
@pytest.mark.parametrize("n", [1, 5, 255, 256, 1000, 100003])
def test_level1(g9, orc, dt, n):
    """Every level-1 call of the table on every stride case; iamax exact; the dot product also against the
    oracle's FP64 restatement."""
    for inc_x, inc_y, lead in STRIDES:
        x, y = strided(rng, n, dt, inc_x, lead), strided(rng, n, dt, inc_y, 1)
        X, Y = x.astype(np.float64), y.astype(np.float64)
        where = f"{np.dtype(dt).name} n={n} inc {inc_x},{inc_y} lead {lead}"
        for name, call, out, expect, tol in LEVEL1:
            x[:], y[:] = X, Y
            ret = call(g9, x, y)
            got = {"y": y, "xy": _both(x, y), "ret": ret}[out]
            ref, scale = expect(X, Y)
            assert_close(f"{name} {where}", got, ref, scale, TOL[dt] if tol is None else tol)
        x[:], y[:] = X, Y
        assert abs(g9.dot(x, y) - orc.dot(x, y)) <= 1e-12 * max(1.0, abs(X) @ abs(Y)), "dot vs oracle " + where
        assert g9.iamax(x) == int(np.argmax(abs(X))), "iamax " + where


@pytest.mark.parametrize("dt", [np.float32, np.float16, np.float64])
def test_level1_shared_pages(g9, dt):
    """Operands that share an array: y right behind x, and dot(x, x)."""
    v = rng.uniform(-1, 1, 3000).astype(dt)
    V = v.astype(np.float64)
    g9.axpy(2.0, v[:1000], v[1000:2000])
    assert_close("axpy shared pages", v[1000:2000], 2 * V[:1000] + V[1000:2000], 3, TOL[dt])
    v[:] = V
    assert_close("dot x·x", g9.dot(v, v), V @ V, V @ V, REDUCTION_TOL)


# GEMV calls on one M×N matrix A (reference: lib/test_level12.py:72-88 for the cases): (label, op(A) as passed, the
# trans flag, alpha, beta, x's (inc, lead), y's (inc, lead) or None for a new vector).
GEMV = [
    ("N", lambda A: A, False, 1.5, 0.0, (1, 0), None),
    ("N beta", lambda A: A, False, 0.5, -2.0, (1, 0), (2, 0)),
    ("T flag", lambda A: A, True, 0.5, 1.0, (-2, 3), (1, 0)),
    ("A.T view", lambda A: A.T, False, 1.0, 0.0, (1, 0), None),
]


@pytest.mark.parametrize("dt", [np.float32, np.float16, np.float64])
@pytest.mark.parametrize("M,N", [(1, 1), (7, 3), (64, 64), (257, 1031), (1000, 2), (3, 5000), (2048, 1536)])
def test_gemv_ger(g9, orc, dt, M, N):
    """The GEMV table against the oracle's float64 product and scale, GER with a reversed y, and the oracle's own
    restatement of the reference GEMV under the same bound."""
    tol = TOL[dt]
    A = rng.uniform(-1, 1, (M, N)).astype(dt)
    Ad = A.astype(np.float64)
    for label, view, trans, alpha, beta, xs, ys in GEMV:
        Av = view(A)
        Op = view(Ad).T if trans else view(Ad)
        x = strided(rng, Op.shape[1], dt, *xs)
        y = strided(rng, Op.shape[0], dt, *ys) if ys else None
        ref, scale = orc.mv(Op, x, alpha, beta, y)
        got = g9.gemv(Av, x, alpha=alpha, beta=beta, y=y, trans=trans)
        assert_close(f"gemv {label} {M}x{N}", got, ref, scale, tol)
    xg, yg = strided(rng, M, dt, 1, 1), strided(rng, N, dt, -3, 0)
    Xg, Yg = xg.astype(np.float64), yg.astype(np.float64)
    Aw = A.copy()
    g9.ger(-0.5, xg, yg, Aw)
    assert_close(f"ger {M}x{N}", Aw, Ad - 0.5 * np.outer(Xg, Yg), abs(Ad) + 0.5 * np.outer(abs(Xg), abs(Yg)), tol)
    if M * N <= 1 << 20:
        x = strided(rng, N, dt)
        ref, scale = orc.mv(Ad, x, 1.5)
        assert_close(f"oracle gemv N {M}x{N}", orc.gemv(A, x, alpha=1.5), ref, scale, tol)


@pytest.mark.parametrize("dt", [np.float32, np.float16, np.float64])
def test_gemv_submatrix(g9, orc, dt):
    """A submatrix view (row stride beyond its width) whose x is a row of the same array."""
    B = rng.uniform(-1, 1, (300, 400)).astype(dt)
    ref, scale = orc.mv(B[10:200, 5:305].astype(np.float64), B[0, :300])
    assert_close("gemv submatrix", g9.gemv(B[10:200, 5:305], B[0, :300]), ref, scale, TOL[dt])


def test_level2_config_device(g9, orc, torch_dev):
    """The benchmarked level 1/2 configuration at full size on device buffers: SAXPY, SDOT (2^26), SGEMV N/T (16384²)."""
    torch = torch_dev
    n = 1 << 26
    x = orc.uniform(n, np.float32, orc.SEED_X)
    y = orc.uniform(n, np.float32, orc.SEED_Y)
    xd, yd = torch.from_numpy(x).cuda(), torch.from_numpy(y).cuda()
    d = g9.dot(xd, yd)
    ref = float(np.dot(x.astype(np.float64), y.astype(np.float64)))
    assert abs(d - ref) <= 1e-12 * float(np.abs(x).astype(np.float64) @ np.abs(y).astype(np.float64))
    g9.axpy(0.5, xd, yd)
    got = yd.cpu().numpy()
    exp = np.float32(0.5) * x + y   # single rounding of a·x + y differs from fma by ≤ 1 ulp
    assert np.max(np.abs(got.astype(np.float64) - exp) / (0.5 * np.abs(x) + np.abs(y) + 1e-30)) <= 1e-6
    m = 16384
    A = orc.uniform((m, m), np.float32, orc.SEED_A)
    xv = orc.uniform(m, np.float32, orc.SEED_X)
    Ad, xvd = torch.from_numpy(A).cuda(), torch.from_numpy(xv).cuda()
    for trans in (False, True):
        yv = g9.gemv(Ad, xvd, trans=trans).cpu().numpy()
        rows = np.random.default_rng(8).integers(0, m, 64)
        Asub = (A.T if trans else A)[rows].astype(np.float64)
        ref = Asub @ xv.astype(np.float64)
        scale = np.abs(Asub) @ np.abs(xv.astype(np.float64))
        assert float(np.max(np.abs(yv[rows] - ref) / scale)) <= 1e-6, f"sgemv trans={trans}"


def test_reduction_device_result(g9, orc, torch_dev):
    """dot / asum / nrm2 with the result pointer in device memory (written in place, no host wait), also in
    no-wait mode; must equal the host-result call bit for bit."""
    import ctypes
    torch = torch_dev
    x = rng.uniform(-1, 1, 300001).astype(np.float32)
    y = rng.uniform(-1, 1, 300001).astype(np.float32)
    xd, yd = torch.from_numpy(x).cuda(), torch.from_numpy(y).cuda()
    out = torch.zeros(3, dtype=torch.float64, device="cuda")
    L = g9._lib

    def p(addr):   # device address as the double* the signature declares
        return ctypes.cast(ctypes.c_void_p(addr), ctypes.POINTER(ctypes.c_double))
    for nowait in (False, True):
        g9.set_nowait(nowait)
        assert L.gen9blas_dot(1, x.size, xd.data_ptr(), 1, yd.data_ptr(), 1, p(out.data_ptr())) == 0
        assert L.gen9blas_asum(1, x.size, xd.data_ptr(), 1, p(out.data_ptr() + 8)) == 0
        assert L.gen9blas_nrm2(1, x.size, xd.data_ptr(), 1, p(out.data_ptr() + 16)) == 0
        g9.flush()
        g9.set_nowait(False)
        got = out.cpu().numpy()
        assert got[0] == g9.dot(xd, yd) and got[1] == g9.asum(xd) and got[2] == g9.nrm2(xd)
        assert abs(got[0] - orc.dot(x, y)) <= 1e-12 * float(np.abs(x) @ np.abs(y))


@pytest.mark.parametrize("reps", [1, 40])
def test_host_result_waits_for_queued_work(g9, torch_dev, reps):
    """A host-result reduction issued right behind products queued in no-wait mode reads their finished output.
    With one product the call waits by spinning on the completion word that a kernel queued behind its work sets;
    40 FP32 products at n = 2048 put several ms of work ahead, so the spin gives up after 2 ms and falls back to
    hipStreamSynchronize. C starts as NaN and the products are of small integers, so the FP64 sum of |C| is exact
    and any read of an unfinished C shows."""
    import ctypes
    torch = torch_dev
    n = 2048
    r = np.random.default_rng(31)
    a = r.integers(-2, 3, (n, n)).astype(np.float32)
    b = r.integers(-2, 3, (n, n)).astype(np.float32)
    ref = float(np.abs(a.astype(np.float64) @ b.astype(np.float64)).sum())
    A, B = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    L = g9._lib
    for trial in range(3):
        C = torch.full((n, n), float("nan"), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        g9.set_nowait(True)
        try:
            for _ in range(reps):
                rc = L.gen9blas_gemm(g9.GEN9BLAS_S, 0, 0, n, n, n, 1.0, ctypes.c_void_p(A.data_ptr()), n,
                                     ctypes.c_void_p(B.data_ptr()), n, 0.0, ctypes.c_void_p(C.data_ptr()), n)
                assert rc == 0, g9._lib.gen9blas_error()
            got = g9.asum(C.reshape(-1))
        finally:
            g9.set_nowait(False)
        assert got == ref, f"reps={reps} trial={trial}: {got} against {ref}"



def _l12_cases(seed, count):
    """Seeded random level-1/2 calls: operation, type, sizes (1-2999, often small), vector strides (negative ones
    on the host only: torch has no negative strides), a column offset for A's view, and residency."""
    r = np.random.default_rng(seed)

    def size():
        return int(r.integers(1, 64)) if r.integers(0, 2) else int(r.integers(64, 3000))
    out = []
    for _ in range(count):
        dev = bool(r.integers(0, 2))
        steps = [1, 2] if dev else [1, 2, -1, -3]
        out.append((str(r.choice(["gemv_n", "gemv_t", "axpy", "dot", "ger"])), int(r.integers(0, 3)), size(), size(),
                    int(r.choice(steps)), int(r.choice(steps)), int(r.integers(0, 6)), dev))
    return out


@pytest.mark.parametrize("case", _l12_cases(2029, 150), ids=lambda c: "-".join(str(v) for v in c))
def test_level12_random(g9, torch_dev, case):
    """150 seeded random GEMV (N and T, on a submatrix view), AXPY, DOT and GER calls in every type, with strided and
    reversed vectors, host or device, against float64 with the bounds above."""
    op, ti, M, N, sx, sy, off, dev = case
    dt = [np.float16, np.float32, np.float64][ti]
    tol = TOL[dt]
    r = np.random.default_rng(M * 7 + N * 13 + ti)

    def vec(n, step):
        """(float64 copy of the values, the operand): a strided view of a host array, or of its device copy."""
        base = r.uniform(-1, 1, n * abs(step) + 2).astype(dt)
        v = base[1:1 + n * abs(step):abs(step)]
        v = v[::-1] if step < 0 else v
        if dev:
            return v.astype(np.float64), torch_dev.from_numpy(base).cuda()[1:1 + n * step:step]
        return v.astype(np.float64), v

    def host(t):
        return t.cpu().numpy() if hasattr(t, "cpu") else t
    tag = f"{op} {np.dtype(dt).name} {M}x{N} sx={sx} sy={sy} off={off} dev={dev}"
    big = r.uniform(-1, 1, (M, N + off + 3)).astype(dt)
    Ad = big[:, off:off + N].astype(np.float64)
    Abig = torch_dev.from_numpy(big.copy()).cuda() if dev else big.copy()
    A = Abig[:, off:off + N]
    if op in ("gemv_n", "gemv_t"):
        tr = op == "gemv_t"
        X, x = vec(M if tr else N, sx)
        Y, y = vec(N if tr else M, sy)
        g9.gemv(A, x, alpha=0.75, beta=-1.25, y=y, trans=tr)
        opA = Ad.T if tr else Ad
        assert_close(tag, host(y), 0.75 * opA @ X - 1.25 * Y, 0.75 * np.abs(opA) @ np.abs(X) + 1.25 * np.abs(Y), tol)
    elif op == "axpy":
        X, x = vec(M, sx)
        Y, y = vec(M, sy)
        g9.axpy(-1.5, x, y)
        assert_close(tag, host(y), Y - 1.5 * X, np.abs(Y) + 1.5 * np.abs(X), tol)
    elif op == "dot":
        X, x = vec(M, sx)
        Y, y = vec(M, sy)
        got = g9.dot(x, y)
        assert abs(got - float(X @ Y)) <= 1e-6 * max(float(np.abs(X) @ np.abs(Y)), 1e-30), tag
    else:
        X, x = vec(M, sx)
        Y, y = vec(N, sy)
        g9.ger(0.5, x, y, A)
        W = host(Abig)
        assert_close(tag, W[:, off:off + N], Ad + 0.5 * np.outer(X, Y), np.abs(Ad) + 0.5 * np.outer(np.abs(X), np.abs(Y)),
              tol)
        assert np.array_equal(W[:, :off], big[:, :off]) and np.array_equal(W[:, off + N:], big[:, off + N:]), tag
