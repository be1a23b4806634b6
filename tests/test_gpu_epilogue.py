"""Fused GEMM epilogues on the GPU: pcl_sgemm_ex against the oracle's GEMM (f64,
one rounding) followed by the oracle's elementwise step (train.c:314-333 GELU,
the residual add of train.c:522/527), and the reference GPU API's elementwise
drop-ins gelu_fwd / gelu_bwd / vec_add (gpu_kernels.cu:228-251).

Fused cases (NN and NT products on grids that take the LDS-DMA kernel or the
16x16x4 kernel without a K split, ragged last tiles included) and fallback cases (TN, unaligned K, split-K grids) must give the
same values; tolerance max|X-R|/max|R| <= 1e-4.
"""
import numpy as np
import pytest

import binding as ob
import pcl
from gpu_util import FP32_TOL, announce, rel, require_device

pytestmark = pytest.mark.gpu
N_, T_ = pcl.OP_N, pcl.OP_T


@pytest.fixture(scope="module", autouse=True)
def _device():
    require_device()


def run_ex(opA, opB, A, B, M, N, K, bias, epi, aux_in=None, want_aux_out=False):
    dA, dB, dbias = pcl.dev(A), pcl.dev(B), pcl.dev(bias)
    dC = pcl.dev(np.full((M, N), np.nan, np.float32))
    din = pcl.dev(aux_in) if aux_in is not None else None
    dout = pcl.dev(np.full((M, N), np.nan, np.float32)) if want_aux_out else None
    pcl.check(pcl.lib.pcl_sgemm_ex(opA, opB, M, N, K, dA.ptr, A.shape[1], dB.ptr, B.shape[1], dbias.ptr,
                                   epi, din.ptr if din else None, dout.ptr if dout else None, N,
                                   dC.ptr, N, None))
    pcl.sync()
    C = dC.download((M, N), np.float32)
    return C, (dout.download((M, N), np.float32) if dout else None)


# (M, N, K, opA, opB, path): "fused" grids take the LDS-DMA kernel unsplit
CASES = [(1024, 1024, 256, N_, N_, "fused 64x64"), (2048, 2048, 128, N_, N_, "fused 128x128"),
         (1024, 1024, 256, N_, T_, "fused NT"), (300, 500, 200, N_, N_, "small grid, K % 32 != 0"),
         (300, 500, 1024, N_, N_, "split K"), (300, 500, 1024, T_, N_, "split K TN"),
         (250, 700, 480, N_, N_, "16x16 kernel, 32x64, ragged"),
         (250, 700, 480, N_, T_, "16x16 kernel, 32x64 NT, ragged"),
         (1024, 1024, 250, N_, N_, "K % 32 != 0"), (1024, 1024, 256, T_, N_, "TN"),
         (1000, 1030, 256, N_, N_, "ragged edges"),
         (4100, 4100, 64, N_, N_, "16x16 kernel, 128x128, ragged"),
         (4100, 4100, 64, N_, T_, "16x16 kernel, 128x128 NT, ragged"),
         (2900, 2980, 96, N_, N_, "16x16 kernel, 128x192, ragged"),
         (2900, 2980, 96, N_, T_, "16x16 kernel, 8-wave 256x192 NT, ragged"),
         (4000, 4000, 96, N_, N_, "16x16 kernel, 8-wave 128x256, ragged"),
         (4000, 3000, 64, N_, N_, "16x16 kernel, 128x192, ragged"),
         (4000, 3000, 64, N_, T_, "16x16 kernel, 8-wave 256x192 NT, ragged"),
         (4000, 1000, 64, N_, N_, "16x16 kernel, 8-wave 128x128, ragged"),
         (4000, 1000, 64, N_, T_, "16x16 kernel, 8-wave 128x128 NT, ragged"),
         (2000, 1100, 160, N_, N_, "16x16 kernel, 64x64, ragged"),
         (2000, 1100, 160, N_, T_, "16x16 kernel, 64x64 NT, ragged")]


@pytest.mark.parametrize("M,N,K,opA,opB,path", CASES)
@pytest.mark.parametrize("epi", [pcl.EPI_GELU, pcl.EPI_RESID, pcl.EPI_GELU_BWD])
def test_sgemm_epilogues(M, N, K, opA, opB, path, epi):
    announce("sgemm_ex", epi, M, N, K, opA, opB, path)
    seed = 700 + M + N + K + 10 * epi
    A = ob.normal((M, K) if opA == N_ else (K, M), seed, 0.0, 1.0)
    B = ob.normal((K, N) if opB == N_ else (N, K), seed + 1, 0.0, 0.05)
    bias = ob.normal((N,), seed + 2, 0.0, 0.1)
    v = ob.gemm_f64(A, B, transA=opA == T_, transB=opB == T_, bias=bias)
    aux = ob.normal((M, N), seed + 3) if epi != pcl.EPI_GELU else None
    C, pre = run_ex(opA, opB, A, B, M, N, K, bias, epi, aux, want_aux_out=epi == pcl.EPI_GELU)
    if epi == pcl.EPI_GELU:
        want = ob.gelu(v)
        assert rel(pre, v) <= FP32_TOL
    elif epi == pcl.EPI_RESID:
        want = aux + v
    else:
        want = ob.gelu_backward(v, aux)
    assert rel(C, want) <= FP32_TOL


def test_sgemm_ex_gelu_without_preactivation_and_none():
    M, N, K = 1024, 1024, 256
    announce("sgemm_ex gelu no aux / none")
    A, B = ob.normal((M, K), 760), ob.normal((K, N), 761, 0.0, 0.05)
    bias = ob.normal((N,), 762, 0.0, 0.1)
    C1, _ = run_ex(N_, N_, A, B, M, N, K, bias, pcl.EPI_GELU)
    C2, pre = run_ex(N_, N_, A, B, M, N, K, bias, pcl.EPI_GELU, want_aux_out=True)
    np.testing.assert_array_equal(C1, C2)
    C0, _ = run_ex(N_, N_, A, B, M, N, K, bias, pcl.EPI_NONE)
    np.testing.assert_array_equal(C0, pre)


def test_sgemm_ex_argument_errors():
    d = pcl.empty((64, 64), np.float32)
    assert pcl.lib.pcl_sgemm_ex(0, 0, 64, 64, 64, d.ptr, 64, d.ptr, 64, None, 9, None, None, 64, d.ptr,
                                64, None) == pcl.PCL_ERR_INVALID_ARG
    pcl.lib.pcl_clear_error()
    assert pcl.lib.pcl_sgemm_ex(0, 0, 64, 64, 64, d.ptr, 64, d.ptr, 64, None, pcl.EPI_RESID, None, None,
                                64, d.ptr, 64, None) == pcl.PCL_ERR_INVALID_ARG
    pcl.lib.pcl_clear_error()


def test_elementwise_dropins():
    n = 100003
    announce("gelu_fwd / gelu_bwd / vec_add", n)
    x, g, y = ob.normal((n,), 780, 0.0, 2.0), ob.normal((n,), 781), ob.normal((n,), 782)
    dx, dg, dy = pcl.dev(x), pcl.dev(g), pcl.dev(y)
    out = pcl.empty((n,), np.float32)
    pcl.lib.gelu_fwd(out.ptr, dx.ptr, n)
    pcl.check_void()
    pcl.sync()
    assert rel(out.download((n,), np.float32), ob.gelu(x)) <= 1e-6
    pcl.lib.gelu_bwd(out.ptr, dg.ptr, dx.ptr, n)
    pcl.check_void()
    pcl.sync()
    assert rel(out.download((n,), np.float32), ob.gelu_backward(g, x)) <= 1e-6
    pcl.lib.vec_add(out.ptr, dx.ptr, dy.ptr, n)
    pcl.check_void()
    pcl.sync()
    np.testing.assert_array_equal(out.download((n,), np.float32), x + y)
