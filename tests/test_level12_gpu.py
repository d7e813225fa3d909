"""Level 1-2 parity on the GPU: axpy, scal, copy, swap, rot, dot, asum, nrm2, iamax, gemv (N and T), ger.

Follows the reference's level 1-2 test (reference: lib/test_level12.py:27-97): lengths 1, 5, 255, 256, 1000, 100003;
strides (1, 1), (1, 1) shifted, (3, −2), (−1, 1); GEMV on odd shapes, with beta, transposed views and submatrices.
Error relative to the formula scale (e.g. |a·x| + |y| for axpy, |A|·|x| for gemv): FP32 ≤ 1e-6, FP16 ≤ 2e-3,
FP64 ≤ 1e-13; reductions (FP64 on the GPU) ≤ 1e-6. The dot product is also compared with the oracle's FP64
restatement (reference: lib/kernels/level12.cl:189-214): both are FP64 sums of exact products and agree to 1e-12.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = {np.float32: 1e-6, np.float16: 2e-3, np.float64: 1e-13}
rng = np.random.default_rng(11)


def check(name, W, ref, scale, tol):
    e = float(np.max(np.abs(np.asarray(W, np.float64) - ref) / np.maximum(scale, 6.2e-5 if tol > 1e-5 else 1e-30)))
    assert e <= tol, f"{name}: {e:.1e} > {tol:.0e}"


def vector(n, dt, step=1, shift=0):
    base = rng.uniform(-1, 1, n * abs(step) + shift + 3).astype(dt)
    v = base[shift:shift + n * abs(step):abs(step)]
    return v[::-1] if step < 0 else v


@pytest.mark.parametrize("dt", [np.float32, np.float16, np.float64])
@pytest.mark.parametrize("n", [1, 5, 255, 256, 1000, 100003])
def test_level1(g9, orc, dt, n):
    tol = TOL[dt]
    for kx, ky, px in ((1, 1, 0), (1, 1, 1), (3, -2, 5), (-1, 1, 2)):
        label = f"{np.dtype(dt).name} n={n} strides {kx},{ky} shift {px}"
        x, y = vector(n, dt, kx, px), vector(n, dt, ky, 1)
        X, Y = x.astype(np.float64), y.astype(np.float64)
        g9.axpy(0.75, x, y)
        check("axpy " + label, y, 0.75 * X + Y, 0.75 * abs(X) + abs(Y), tol)
        y[:] = Y
        g9.scal(-1.5, y)
        check("scal " + label, y, -1.5 * Y, 1.5 * abs(Y), tol)
        y[:] = Y
        g9.copy(x, y)
        check("copy " + label, y, X, 1, 0)
        y[:] = Y
        g9.swap(x, y)
        check("swap " + label, np.concatenate([x, y]), np.concatenate([Y, X]), 1, 0)
        x[:], y[:] = X, Y
        g9.rot(x, y, 0.6, 0.8)
        check("rot " + label, np.concatenate([x, y]), np.concatenate([0.6 * X + 0.8 * Y, 0.6 * Y - 0.8 * X]),
              np.concatenate([abs(X) + abs(Y)] * 2), tol)
        x[:], y[:] = X, Y
        d = g9.dot(x, y)
        check("dot " + label, d, X @ Y, abs(X) @ abs(Y), 1e-6)
        assert abs(d - orc.dot(x, y)) <= 1e-12 * max(1.0, abs(X) @ abs(Y)), "dot vs oracle " + label
        check("asum " + label, g9.asum(x), abs(X).sum(), abs(X).sum(), 1e-6)
        check("nrm2 " + label, g9.nrm2(x), np.linalg.norm(X), np.linalg.norm(X), 1e-6)
        assert g9.iamax(x) == int(np.argmax(abs(X))), "iamax " + label


@pytest.mark.parametrize("dt", [np.float32, np.float16, np.float64])
def test_level1_shared_pages(g9, dt):
    v = rng.uniform(-1, 1, 3000).astype(dt)
    V = v.astype(np.float64)
    g9.axpy(2.0, v[:1000], v[1000:2000])
    check("axpy shared pages", v[1000:2000], 2 * V[:1000] + V[1000:2000], 3, TOL[dt])
    v[:] = V
    check("dot x·x", g9.dot(v, v), V @ V, V @ V, 1e-6)


@pytest.mark.parametrize("dt", [np.float32, np.float16, np.float64])
@pytest.mark.parametrize("M,N", [(1, 1), (7, 3), (64, 64), (257, 1031), (1000, 2), (3, 5000), (2048, 1536)])
def test_gemv_ger(g9, orc, dt, M, N):
    tol = TOL[dt]
    A = rng.uniform(-1, 1, (M, N)).astype(dt)
    Ad = A.astype(np.float64)
    x, xt = vector(N, dt), vector(M, dt, -2, 3)
    y0, yt0 = vector(M, dt, 2), vector(N, dt)
    Y0, YT0 = y0.astype(np.float64), yt0.astype(np.float64)
    y = g9.gemv(A, x, alpha=1.5)
    check(f"gemv N {M}x{N}", y, 1.5 * Ad @ x.astype(np.float64), 1.5 * abs(Ad) @ abs(x.astype(np.float64)), tol)
    g9.gemv(A, x, alpha=0.5, beta=-2.0, y=y0)
    check(f"gemv N beta {M}x{N}", y0, 0.5 * Ad @ x.astype(np.float64) - 2 * Y0,
          0.5 * abs(Ad) @ abs(x.astype(np.float64)) + 2 * abs(Y0), tol)
    g9.gemv(A, xt, alpha=0.5, beta=1.0, y=yt0, trans=True)
    Xt = xt.astype(np.float64)
    check(f"gemv T {M}x{N}", yt0, 0.5 * Ad.T @ Xt + YT0, 0.5 * abs(Ad.T) @ abs(Xt) + abs(YT0), tol)
    xv = vector(M, dt)
    Xv = xv.astype(np.float64)
    yv = g9.gemv(A.T, xv)
    check(f"gemv A.T {M}x{N}", yv, Ad.T @ Xv, abs(Ad.T) @ abs(Xv), tol)
    xg, yg = vector(M, dt, 1, 1), vector(N, dt, -3, 0)
    Xg, Yg = xg.astype(np.float64), yg.astype(np.float64)
    A2 = A.copy()
    g9.ger(-0.5, xg, yg, A2)
    check(f"ger {M}x{N}", A2, Ad - 0.5 * np.outer(Xg, Yg), abs(Ad) + 0.5 * np.outer(abs(Xg), abs(Yg)), tol)
    # the oracle's restatement of the reference GEMV meets the same bound
    if M * N <= 1 << 20:
        R = orc.gemv(A, x, alpha=1.5)
        check(f"oracle gemv N {M}x{N}", R, 1.5 * Ad @ x.astype(np.float64), 1.5 * abs(Ad) @ abs(x.astype(np.float64)), tol)


@pytest.mark.parametrize("dt", [np.float32, np.float16, np.float64])
def test_gemv_submatrix(g9, dt):
    B = rng.uniform(-1, 1, (300, 400)).astype(dt)
    Bd = B.astype(np.float64)
    y = g9.gemv(B[10:200, 5:305], B[0, :300])
    check("gemv submatrix", y, Bd[10:200, 5:305] @ Bd[0, :300], abs(Bd[10:200, 5:305]) @ abs(Bd[0, :300]), TOL[dt])


def test_level2_config_device(g9, orc, torch_dev):
    """BASELINE level 1/2 config at full size on device buffers: SAXPY, SDOT (2^26), SGEMV N/T (16384²)."""
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
        check(tag, host(y), 0.75 * opA @ X - 1.25 * Y, 0.75 * np.abs(opA) @ np.abs(X) + 1.25 * np.abs(Y), tol)
    elif op == "axpy":
        X, x = vec(M, sx)
        Y, y = vec(M, sy)
        g9.axpy(-1.5, x, y)
        check(tag, host(y), Y - 1.5 * X, np.abs(Y) + 1.5 * np.abs(X), tol)
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
        check(tag, W[:, off:off + N], Ad + 0.5 * np.outer(X, Y), np.abs(Ad) + 0.5 * np.outer(np.abs(X), np.abs(Y)),
              tol)
        assert np.array_equal(W[:, :off], big[:, :off]) and np.array_equal(W[:, off + N:], big[:, off + N:]), tag
