"""Decode GEMV parity (M <= 8 rows) on the GPU: the HBM-bound kernels.

FP32 against the reference-order restatement of matvec/proj_token
(generate.c:95-107, transformer.c:174-195) and the f64 truth, <= 1e-4; the
split-K path (partial sums, then an ordered reduction kernel) is exercised by
long-K shapes and must give identical bits on repeated calls.
"""
import numpy as np
import pytest

import binding as ob
import pcl
from gpu_util import FP32_TOL, announce, rel, require_device

pytestmark = pytest.mark.gpu
p = ob.p


@pytest.fixture(scope="module", autouse=True)
def _device():
    require_device()


def sgemv(opW, X, W, bias=None, Y0=None):
    M, K = X.shape
    N = W.shape[1] if opW == pcl.OP_N else W.shape[0]
    dX, dW = pcl.dev(X), pcl.dev(W)
    db = pcl.dev(bias) if bias is not None else None
    dY = pcl.dev(Y0) if Y0 is not None else pcl.empty((M, N), np.float32)
    pcl.check(pcl.lib.pcl_sgemv(opW, M, N, K, dX.ptr, K, dW.ptr, W.shape[1], db.ptr if db else None,
                                0 if Y0 is None else 1, dY.ptr, N, None))
    pcl.sync()
    return dY.download((M, N), np.float32)


# grown-model decode shapes (D=512, FF=2048, V=2048), 350M-class ones, odd
# sizes (scalar tail path) and long-K shapes (split-K reduction)
N_SHAPES = [(512, 1536), (512, 512), (512, 2048), (2048, 512), (1024, 4096), (4096, 1024),
            (77, 131), (5000, 64), (3, 1)]
T_SHAPES = [(512, 2048), (1024, 50257), (1536, 2048), (77, 131), (8192, 64), (100, 3)]


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
def test_sgemv_n(M):
    for K, N in N_SHAPES:
        X = ob.normal((M, K), 10 + K)
        W = ob.normal((K, N), 11 + N, 0.0, 0.02)
        b = ob.normal((N,), 12)
        announce("sgemv_n", M, K, N)
        Y = sgemv(pcl.OP_N, X, W, b)
        Rr = np.empty((M, N), np.float32)
        ob.oracle().orc_matvec(p(Rr), p(X), p(W), p(b), M, K, N)
        assert rel(Y, Rr) <= FP32_TOL
        assert rel(Y, ob.gemm_f64(X, W, bias=b)) <= FP32_TOL


@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_sgemv_t(M):
    for K, N in T_SHAPES:
        X = ob.normal((M, K), 20 + K)
        W = ob.normal((N, K), 21 + N, 0.0, 0.02)
        announce("sgemv_t", M, K, N)
        Y = sgemv(pcl.OP_T, X, W)
        Rr = np.empty((M, N), np.float32)
        ob.oracle().orc_lm_head(p(Rr), p(X), p(W), M, K, N)
        assert rel(Y, Rr) <= FP32_TOL


def test_sgemv_accumulate_and_determinism():
    M, K, N = 4, 8192, 96  # long K: several splits per column strip
    X = ob.normal((M, K), 30)
    W = ob.normal((K, N), 31, 0, 0.02)
    b = ob.normal((N,), 32)
    Y0 = ob.normal((M, N), 33)
    announce("sgemv accumulate x3")
    outs = [sgemv(pcl.OP_N, X, W, b, Y0) for _ in range(3)]
    assert rel(outs[0], ob.gemm_f64(X, W, bias=b, C0=Y0)) <= FP32_TOL
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])


@pytest.mark.parametrize("opW", [pcl.OP_N, pcl.OP_T])
@pytest.mark.parametrize("M,K,ldx", [(3, 130, 136), (8, 2050, 2052), (5, 61, 64)])
def test_sgemv_padded_rows(opW, M, K, ldx):
    # 16-byte aligned activation rows whose K is not a multiple of 4: the
    # staging's vector loads stop at K and assemble the last chunk by element
    N = 70
    Xp = ob.normal((M, ldx), 70 + K)
    X = np.ascontiguousarray(Xp[:, :K])
    W = ob.normal((K, N) if opW == pcl.OP_N else (N, K), 71, 0.0, 0.02)
    dX, dW, dY = pcl.dev(Xp), pcl.dev(W), pcl.empty((M, N), np.float32)
    announce("sgemv padded rows", opW, M, K, ldx)
    pcl.check(pcl.lib.pcl_sgemv(opW, M, N, K, dX.ptr, ldx, dW.ptr, W.shape[1], None, 0, dY.ptr, N, None))
    pcl.sync()
    R = ob.gemm_f64(X, W, transB=opW == pcl.OP_T)
    assert rel(dY.download((M, N), np.float32), R) <= FP32_TOL


@pytest.mark.parametrize("opW", [pcl.OP_N, pcl.OP_T])
def test_sgemv_k0(opW):
    # K == 0 reads no operand (NULL X and W): Y = Y0 + bias
    M, N = 3, 50
    b = ob.normal((N,), 60)
    Y0 = ob.normal((M, N), 61)
    db, dY = pcl.dev(b), pcl.dev(Y0)
    announce("sgemv K=0", opW)
    pcl.check(pcl.lib.pcl_sgemv(opW, M, N, 0, None, 1, None, N, db.ptr, 1, dY.ptr, N, None))
    pcl.sync()
    np.testing.assert_array_equal(dY.download((M, N), np.float32), Y0 + b)
    dY2 = pcl.dev(Y0)
    pcl.check(pcl.lib.pcl_sgemv(opW, M, N, 0, None, 1, None, N, None, 0, dY2.ptr, N, None))
    pcl.sync()
    np.testing.assert_array_equal(dY2.download((M, N), np.float32), np.zeros((M, N), np.float32))
    ddb = pcl.dev(b)
    pcl.check(pcl.lib.pcl_bias_bwd(ddb.ptr, None, 0, N, N, None))  # sum over no rows
    pcl.sync()
    np.testing.assert_array_equal(ddb.download((N,), np.float32), b)


def test_sgemm_routes_small_m_to_gemv():
    # pcl_sgemm with M <= 8 and opA == N takes the GEMV kernels
    M, K, N = 6, 640, 1000
    X = ob.normal((M, K), 40)
    W = ob.normal((N, K), 41, 0, 0.02)
    dX, dW, dY = pcl.dev(X), pcl.dev(W), pcl.empty((M, N), np.float32)
    announce("sgemm->gemv")
    pcl.check(pcl.lib.pcl_sgemm(pcl.OP_N, pcl.OP_T, M, N, K, dX.ptr, K, dW.ptr, K, None, 0, dY.ptr, N, None))
    pcl.sync()
    assert rel(dY.download((M, N), np.float32), ob.gemm_f64(X, W, transB=True)) <= FP32_TOL


@pytest.mark.parametrize("M,N", [(4096, 1536), (1, 7), (37, 300), (100000, 64)])
def test_bias_bwd(M, N):
    dY = ob.normal((M, N), 50, 0.0, 1e-3)
    db0 = ob.normal((N,), 51, 0.0, 1e-3)
    ddY, ddb = pcl.dev(dY), pcl.dev(db0)
    announce("bias_bwd", M, N)
    pcl.check(pcl.lib.pcl_bias_bwd(ddb.ptr, ddY.ptr, M, N, N, None))
    pcl.sync()
    got = ddb.download((N,), np.float32)
    want = db0.copy()
    ob.oracle().orc_bias_bwd(p(want), p(dY), M, N)
    truth = db0.astype(np.float64) + dY.astype(np.float64).sum(0)
    assert rel(got, truth) <= FP32_TOL
    assert rel(got, want) <= FP32_TOL
