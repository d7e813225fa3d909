"""Packed B kept on the GPU (gen9blas_pack_b / gen9blas_gemm_pb / gen9blas_packed_b_free) on a GPU.

Follows the reference's packed-B test (reference: lib/test_packed.py:63-110): transposed and plain B, shapes that are
not tile multiples, alpha/beta, FP16 (both modes), FP32 and FP64, one packed B reused with several A, and B
overwritten after packing (the packed copy must not change). Each product is compared with the float64 product of the
same inputs under the reference's error metric and bounds (lib/test_packed.py:27: H 3e-3, HS 3e-4, S 1e-6, D 1e-14),
and, where K is a multiple of 64 (so the packed rows need no padding), with gen9blas_gemm on the same data with
transB = 1, which then runs the same kernels on the same layout and must give identical bits. Added here: M ≤ 16 products (the skinny kernels streaming the packed weights), device-resident A and
C, and the argument checks of pack_b.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

H, S, HS, D = 0, 1, 2, 3
DT = {H: np.float16, S: np.float32, HS: np.float16, D: np.float64}
TOL = {H: 3e-3, S: 1e-6, HS: 3e-4, D: 1e-14}


def _err(C, A, Bkn, alpha=1.0, beta=0.0, C0=None):
    a64, b64 = A.astype(np.float64), Bkn.astype(np.float64)
    ref = alpha * (a64 @ b64)
    mag = abs(alpha) * (np.abs(a64) @ np.abs(b64))
    if beta:
        ref += beta * C0.astype(np.float64)
        mag += abs(beta) * np.abs(C0.astype(np.float64))
    return float(np.max(np.abs(np.asarray(C, np.float64) - ref) / np.maximum(mag, 1e-30)))


def _pack(L, t, B, transB):
    K, N = (B.shape[1], B.shape[0]) if transB else B.shape
    P = L.gen9blas_pack_b(t, transB, K, N, B.ctypes.data, B.shape[1])
    assert P, L.gen9blas_error()
    return P, K, N


def _gemm_pb(L, t, A, P, N, alpha=1.0, beta=0.0, C=None):
    if C is None:
        C = np.zeros((A.shape[0], N), DT[t])
    rc = L.gen9blas_gemm_pb(0, A.shape[0], alpha, A.ctypes.data, A.shape[1], P, beta, C.ctypes.data, N)
    assert rc == 0, L.gen9blas_error()
    return C


@pytest.mark.parametrize("t,M,N,K,transB,alpha,beta", [
    (S, 512, 1536, 1536, 1, 1.0, 0.0), (S, 33, 100, 2051, 1, 1.0, 0.0), (S, 37, 1000, 300, 0, 1.0, 0.0),
    (S, 64, 1536, 1536, 1, 0.5, -2.0), (H, 256, 1024, 1024, 1, 1.0, 0.0), (HS, 256, 1024, 2048, 1, 1.0, 0.0),
    (D, 64, 512, 512, 1, 1.0, 0.0), (H, 8, 4096, 4096, 1, 1.0, 0.0), (HS, 1, 1000, 777, 0, 1.0, 0.0),
    (S, 16, 333, 1024, 1, 2.0, 0.5), (H, 128, 384, 320, 0, 1.0, 0.0)])
def test_gemm_pb(g9, t, M, N, K, transB, alpha, beta):
    L = g9._lib
    rng = np.random.default_rng(7)
    dt = DT[t]
    A = rng.uniform(-1, 1, (M, K)).astype(dt)
    B = rng.uniform(-1, 1, (N, K) if transB else (K, N)).astype(dt)
    Bkn = B.T if transB else B
    C0 = rng.uniform(-1, 1, (M, N)).astype(dt)
    P, _, _ = _pack(L, t, B, transB)
    try:
        C = _gemm_pb(L, t, A, P, N, alpha, beta, C0.copy())
        assert np.isfinite(C).all()
        e = _err(C, A, Bkn, alpha, beta, C0)
        assert e <= TOL[t], f"rel err {e:.2e}"
        if K % 64:
            return   # the packed rows are padded to 64 elements: another leading dimension, maybe another code path
        # the same product through gen9blas_gemm on B stored N×K (transB = 1): same layout, same kernels, same bits
        Bt = np.ascontiguousarray(Bkn.T)
        C2 = C0.copy()
        assert L.gen9blas_gemm(t, 0, 1, M, N, K, ctypes.c_double(alpha), A.ctypes.data, K, Bt.ctypes.data, K,
                               ctypes.c_double(beta), C2.ctypes.data, N) == 0
        assert np.array_equal(C, C2), "gemm_pb differs from gemm with transB = 1"
    finally:
        L.gen9blas_packed_b_free(P)


def test_packed_b_reuse_and_independence(g9, torch_dev):
    """Pack once, overwrite B, multiply with different A (host and device memory): the packed copy is what counts."""
    L = g9._lib
    rng = np.random.default_rng(11)
    B = rng.uniform(-1, 1, (1536, 1536)).astype(np.float32)
    Bkn = B.T.copy()
    P, K, N = _pack(L, S, B, 1)
    B[:] = 0.0
    try:
        for M in (128, 512, 4, 128):
            A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
            assert _err(_gemm_pb(L, S, A, P, N), A, Bkn) <= TOL[S], f"M={M}"
        # device-resident A and C: C is written in place
        A = rng.uniform(-1, 1, (64, K)).astype(np.float32)
        Ad = torch_dev.from_numpy(A).cuda()
        Cd = torch_dev.zeros((64, N), dtype=torch_dev.float32, device="cuda")
        assert L.gen9blas_gemm_pb(0, 64, 1.0, ctypes.c_void_p(Ad.data_ptr()), K, P, 0.0,
                                  ctypes.c_void_p(Cd.data_ptr()), N) == 0
        torch_dev.cuda.synchronize()
        assert _err(Cd.cpu().numpy(), A, Bkn) <= TOL[S]
        assert g9.last_zero_copy() == 7
        # transposed A (stored K×M)
        At = np.ascontiguousarray(A.T)
        C = np.zeros((64, N), np.float32)
        assert L.gen9blas_gemm_pb(1, 64, 1.0, At.ctypes.data, 64, P, 0.0, C.ctypes.data, N) == 0
        assert _err(C, A, Bkn) <= TOL[S]
    finally:
        L.gen9blas_packed_b_free(P)


def test_pack_b_arguments(g9):
    L = g9._lib
    b = np.ones((8, 8), np.float32)
    assert L.gen9blas_pack_b(S, 0, 8, 8, b.ctypes.data, 4) is None          # ldb < N
    assert L.gen9blas_last_status() == -3
    assert L.gen9blas_pack_b(S, 1, 8, 8, None, 8) is None                   # NULL B
    assert L.gen9blas_last_status() == -3
    assert L.gen9blas_pack_b(S, 0, 8, -1, b.ctypes.data, 8) is None
    assert L.gen9blas_last_status() == -3
    L.gen9blas_packed_b_free(None)                                          # no-op
    P = L.gen9blas_pack_b(S, 0, 8, 8, b.ctypes.data, 8)
    assert P
    c = np.full((8, 8), -1, np.float32)
    assert L.gen9blas_gemm_pb(0, 0, 1.0, b.ctypes.data, 8, P, 0.0, c.ctypes.data, 8) == 0   # M = 0: no-op
    assert (c == -1).all()
    L.gen9blas_packed_b_free(P)


def _skinny_pb(L, M, A, P, N, C=None, ldc=None):
    C = np.full((M, N), np.nan, np.float32) if C is None else C
    nf = ctypes.c_int(-1)
    rc = L.gen9blas_gemm_pb_skinny(M, A.ctypes.data, A.shape[1], P, C.ctypes.data, ldc or N, ctypes.byref(nf))
    return rc, C, nf.value


@pytest.mark.parametrize("N,K", [(1024, 1024), (256, 1024), (3072, 1024), (1024, 3072), (1000, 1000), (37, 96),
                                 (4096, 4096)])
def test_gemm_pb_skinny(g9, N, K):
    """gen9blas_gemm_pb_skinny (reference: lib/test_skinny_pb.py:52-75): weights W[N][K] FP16 packed as GEN9BLAS_HS with
    transB = 1, FP32 activations, M = 1..16; error against the float64 product relative to |A|·|Wᵀ| under 1e-5 (the
    reference's bound), no non-finite result."""
    L = g9._lib
    assert L.gen9blas_has(3) == 1   # GEN9BLAS_FEAT_SKINNY_PB
    rng = np.random.default_rng(11)
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float16)
    P, _, _ = _pack(L, HS, W, 1)
    try:
        W64 = W.astype(np.float64)
        for M in (1, 2, 3, 4, 5, 8, 9, 12, 16):
            A = rng.standard_normal((M, K)).astype(np.float32)
            rc, C, nf = _skinny_pb(L, M, A, P, N)
            assert rc == 0, L.gen9blas_error()
            ref = A.astype(np.float64) @ W64.T
            mag = np.abs(A.astype(np.float64)) @ np.abs(W64.T)
            err = float(np.max(np.abs(C - ref) / mag))
            assert err < 1e-5 and nf == 0 and np.isfinite(C).all(), f"M={M}: rel err {err:.1e}, nonfinite {nf}"
    finally:
        L.gen9blas_packed_b_free(P)


def test_gemm_pb_skinny_flags_and_arguments(g9, torch_dev):
    """A non-finite result sets *nonfinite and the next call starts clean; M outside 1..16 is DECLINED (1) with nothing
    written; a B packed as another type is INVALID_ARG; device-resident A and C are used in place, with row strides."""
    L = g9._lib
    rng = np.random.default_rng(3)
    N, K = 300, 520
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float16)
    P, _, _ = _pack(L, HS, W, 1)
    Ph, _, _ = _pack(L, H, W, 1)
    try:
        A = rng.standard_normal((4, K)).astype(np.float32)
        A[2, 17] = np.inf
        rc, C, nf = _skinny_pb(L, 4, A, P, N)
        assert rc == 0 and nf == 1 and not np.isfinite(C[2]).all() and np.isfinite(C[[0, 1, 3]]).all()
        A[2, 17] = 1.0
        rc, C, nf = _skinny_pb(L, 4, A, P, N)
        assert rc == 0 and nf == 0 and np.isfinite(C).all()
        for M in (0, 17):
            Z = np.zeros((max(M, 1), K), np.float32)
            rc, C, nf = _skinny_pb(L, M, Z, P, N, C=np.full((max(M, 1), N), 7.0, np.float32))
            assert rc == 1 and (C == 7.0).all()
        rc, _, _ = _skinny_pb(L, 4, A, Ph, N)
        assert rc == -3
        torch = torch_dev
        Ab = rng.standard_normal((16, K + 12)).astype(np.float32)
        Ad = torch.from_numpy(Ab).cuda()
        Cd = torch.full((16, N + 5), 3.0, dtype=torch.float32, device="cuda")
        nf = ctypes.c_int(-1)
        assert L.gen9blas_gemm_pb_skinny(16, ctypes.c_void_p(Ad.data_ptr()), K + 12, P, ctypes.c_void_p(Cd.data_ptr()),
                                         N + 5, ctypes.byref(nf)) == 0 and nf.value == 0
        C = Cd.cpu().numpy()
        ref = Ab[:, :K].astype(np.float64) @ W.astype(np.float64).T
        mag = np.abs(Ab[:, :K].astype(np.float64)) @ np.abs(W.astype(np.float64)).T
        assert float(np.max(np.abs(C[:, :N] - ref) / mag)) < 1e-5 and (C[:, N:] == 3.0).all()
    finally:
        L.gen9blas_packed_b_free(P)
        L.gen9blas_packed_b_free(Ph)
