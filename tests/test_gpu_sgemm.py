"""FP32 GEMM parity on the GPU: libpcl_hip (f32 MFMA) vs the CPU oracle.

Tolerance: max|C-R|/max|R| <= 1e-4 against both
the reference-order fp32 restatement (tensor.c:34-53) and the f64 truth.
Full 350M-class shapes are checked on sampled rows against f64 numpy.
"""
import numpy as np
import pytest

import binding as ob
import pcl
from gpu_util import FP32_TOL, announce, rel, require_device, sampled_rows_f64, sgemm

pytestmark = pytest.mark.gpu

N_, T_ = pcl.OP_N, pcl.OP_T


@pytest.fixture(scope="module", autouse=True)
def _device():
    require_device()


def _operands(opA, opB, M, N, K, seed):
    A = ob.frand((M, K) if opA == N_ else (K, M), seed)
    B = ob.frand((K, N) if opB == N_ else (N, K), seed + 1)
    return A, B


SHAPES = [(17, 33, 65), (64, 64, 64), (128, 128, 128), (1000, 1001, 999), (256, 1536, 512),
          (9, 5, 1), (33, 260, 300), (130, 70, 4),
          # small grids with a short K: 32x64 tiles in one launch for row-major A
          # (ragged M and N, K a multiple of 32 up to 512, and one past it)
          (250, 700, 480), (256, 512, 512), (100, 2000, 32), (256, 512, 544)]


@pytest.mark.parametrize("opA,opB", [(N_, N_), (N_, T_), (T_, N_), (T_, T_)])
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_sgemm_layouts(opA, opB, M, N, K):
    announce("sgemm", opA, opB, M, N, K)
    A, B = _operands(opA, opB, M, N, K, 1000 + M + N + K)
    C = sgemm(opA, opB, A, B, M, N, K)
    R = ob.gemm_f64(A, B, transA=opA == T_, transB=opB == T_)
    assert rel(C, R) <= FP32_TOL


def test_sgemm_nn_matches_reference_order_restatement():
    M, K, N = 1024, 1024, 1024  # gemm_bench FP32 config, A,B ~ U[-1,1]
    announce("sgemm nn 1024^3 vs ikj")
    A, B = ob.frand((M, K), 1234), ob.frand((K, N), 1235)
    C = sgemm(N_, N_, A, B, M, N, K)
    assert rel(C, ob.matmul_ikj(A, B)) <= FP32_TOL


def test_sgemm_tensor_kat():
    # tensor.c:204-205 / 237-241: C[0,0] = 0.07 on the 1024^3 mod pattern
    M = K = N = 1024
    A = np.empty(M * K, np.float32)
    B = np.empty(K * N, np.float32)
    ob.oracle().orc_fill_kat_tensor(ob.p(A), A.size, ob.p(B), B.size)
    announce("sgemm tensor KAT")
    C = sgemm(N_, N_, A.reshape(M, K), B.reshape(K, N), M, N, K)
    assert abs(float(C[0, 0]) - 0.07) < 1e-5


def test_sgemm_bias_accumulate_and_k0():
    M, N, K = 70, 90, 50
    A, B = _operands(N_, N_, M, N, K, 77)
    bias = ob.normal((N,), 78)
    C0 = ob.normal((M, N), 79)
    announce("sgemm bias+accumulate")
    C = sgemm(N_, N_, A, B, M, N, K, bias=bias, C0=C0)
    assert rel(C, ob.gemm_f64(A, B, bias=bias, C0=C0)) <= FP32_TOL
    # K == 0: C = bias (or C0 + bias)
    A0, B0 = np.zeros((M, 0), np.float32), np.zeros((0, N), np.float32)
    dA, dB, dbias = pcl.empty((1,), np.float32), pcl.empty((1,), np.float32), pcl.dev(bias)
    dC = pcl.dev(C0)
    pcl.check(pcl.lib.pcl_sgemm(N_, N_, M, N, 0, dA.ptr, 1, dB.ptr, N, dbias.ptr, 1, dC.ptr, N, None))
    pcl.sync()
    np.testing.assert_array_equal(dC.download((M, N), np.float32), C0 + bias)
    del A0, B0


@pytest.mark.parametrize("opA,opB", [(N_, N_), (N_, T_), (T_, N_)])
@pytest.mark.parametrize("M,N,K", [(256, 512, 2048), (256, 512, 512), (100, 200, 1000), (64, 96, 4100),
                                   (640, 1024, 4096), (1000, 600, 2100)])
def test_sgemm_split_k_bias_accumulate(opA, opB, M, N, K):
    # grids of fewer than 256 64x64 tiles split K over workgroups (grids of
    # 129-255 tiles with K >= 2048 into 2+ workgroups per CU); the partial
    # products are added in split order, then bias, then the old C
    A, B = _operands(opA, opB, M, N, K, 3000 + M + K)
    bias = ob.normal((N,), 3001)
    C0 = ob.normal((M, N), 3002)
    announce("sgemm split-K", opA, opB, M, N, K)
    C = sgemm(opA, opB, A, B, M, N, K, bias=bias, C0=C0)
    R = ob.gemm_f64(A, B, transA=opA == T_, transB=opB == T_, bias=bias, C0=C0)
    assert rel(C, R) <= FP32_TOL


@pytest.mark.parametrize("opA,opB", [(N_, N_), (N_, T_), (T_, N_), (T_, T_)])
@pytest.mark.parametrize("M,N,K", [(200, 260, 320), (132, 68, 96), (1000, 1004, 992)])
def test_sgemm_lds_dma_edges(opA, opB, M, N, K):
    # aligned operands with K % 32 == 0 take the LDS-DMA pipeline: ragged M
    # and N (clamped rows / column chunks), all four layouts, padded leading
    # dimensions, bias and accumulate
    A = ob.frand((M, K + 8) if opA == N_ else (K, M + 12), 4000 + M)
    B = ob.frand((K, N + 4) if opB == N_ else (N, K + 8), 4001 + N)
    bias = ob.normal((N,), 4002)
    C0 = ob.normal((M, N + 4), 4003)
    dA, dB, db, dC = pcl.dev(A), pcl.dev(B), pcl.dev(bias), pcl.dev(C0)
    announce("sgemm lds-dma", opA, opB, M, N, K)
    pcl.check(pcl.lib.pcl_sgemm(opA, opB, M, N, K, dA.ptr, A.shape[1], dB.ptr, B.shape[1], db.ptr, 1, dC.ptr,
                                N + 4, None))
    pcl.sync()
    C = dC.download((M, N + 4), np.float32)
    Av = A[:, :K] if opA == N_ else A[:, :M]
    Bv = B[:, :N] if opB == N_ else B[:, :K]
    R = ob.gemm_f64(np.ascontiguousarray(Av), np.ascontiguousarray(Bv), transA=opA == T_, transB=opB == T_,
                    bias=bias, C0=np.ascontiguousarray(C0[:, :N]))
    assert rel(C[:, :N], R) <= FP32_TOL
    np.testing.assert_array_equal(C[:, N:], C0[:, N:])  # padding columns untouched


@pytest.mark.parametrize("opA,opB", [(N_, N_), (N_, T_), (T_, N_), (T_, T_)])
@pytest.mark.parametrize("M,N,K", [(4100, 4100, 64), (2900, 2980, 96), (4000, 4000, 64), (4000, 3000, 96),
                                   (4000, 1000, 64), (4100, 1000, 352), (2000, 1100, 160)])
def test_sgemm_16x16_grid_edges(opA, opB, M, N, K):
    # grids of >= 512 tiles take the 16x16x4 kernel: 128x128 tiles on 16-deep
    # stages (4100 x 4100, and 4000 x 4000 in the layouts other than NN); NN
    # grids that fill whole rounds of 128x256 tiles (4000 x 4000) one 8-wave
    # 128x256 workgroup per CU; grids that fill the
    # chip better with 192-wide tiles (4000 x 3000, 2900 x 2980) two 4-wave 128x192
    # workgroups per CU, for NT one 8-wave 256x192 on 32-deep stages; grids of one 128x128
    # tile per CU (4000 x 1000, 4100 x 1000) an 8-wave 128x128 workgroup on
    # 16-deep stages (NN, TN) or 32-deep ones (NT), and for TT 128x64 tiles on
    # 32-deep stages; 64x64 tiles on 16-deep stages (2000 x 1100); with ragged
    # last tile rows and columns (the bounds-checked epilogue beside the
    # unchecked one of interior tiles), padded leading dimensions,
    # bias and accumulate, all four layouts, against the f64 product
    A = ob.frand((M, K + 8) if opA == N_ else (K, M + 12), 4100 + M)
    B = ob.frand((K, N + 4) if opB == N_ else (N, K + 8), 4101 + N)
    bias = ob.normal((N,), 4102)
    C0 = ob.normal((M, N + 4), 4103)
    dA, dB, db, dC = pcl.dev(A), pcl.dev(B), pcl.dev(bias), pcl.dev(C0)
    announce("sgemm 16x16 edges", opA, opB, M, N, K)
    pcl.check(pcl.lib.pcl_sgemm(opA, opB, M, N, K, dA.ptr, A.shape[1], dB.ptr, B.shape[1], db.ptr, 1, dC.ptr,
                                N + 4, None))
    pcl.sync()
    C = dC.download((M, N + 4), np.float32)
    Av = A[:, :K] if opA == N_ else A[:, :M]
    Bv = B[:, :N] if opB == N_ else B[:, :K]
    R = ob.gemm_f64(np.ascontiguousarray(Av), np.ascontiguousarray(Bv), transA=opA == T_, transB=opB == T_,
                    bias=bias, C0=np.ascontiguousarray(C0[:, :N]))
    assert rel(C[:, :N], R) <= FP32_TOL
    np.testing.assert_array_equal(C[:, N:], C0[:, N:])  # padding columns untouched


def test_sgemm_strided_leading_dims():
    # sub-matrix views: lda/ldb/ldc larger than the logical width
    M, N, K = 96, 80, 72
    Abig, Bbig = ob.frand((M, K + 8), 90), ob.frand((K, N + 12), 91)
    dA, dB = pcl.dev(Abig), pcl.dev(Bbig)
    dC = pcl.dev(np.full((M, N + 4), 5.0, np.float32))
    announce("sgemm strided")
    pcl.check(pcl.lib.pcl_sgemm(N_, N_, M, N, K, dA.ptr, K + 8, dB.ptr, N + 12, None, 0, dC.ptr, N + 4, None))
    pcl.sync()
    C = dC.download((M, N + 4), np.float32)
    assert rel(C[:, :N], ob.gemm_f64(Abig[:, :K], Bbig[:, :N])) <= FP32_TOL
    assert np.all(C[:, N:] == 5.0)  # untouched padding columns


def test_sgemm_host_threads_share_the_null_stream():
    # two host threads call on their default (null) stream at once, with split-K
    # grids of different sizes, so each call's workspace may have to grow while
    # the other thread's call holds the stream's scratch
    import threading
    shapes = [(300, 500, 2000), (200, 260, 4096), (330, 520, 2048), (100, 700, 3000)]
    cases = []
    for i, (M, N, K) in enumerate(shapes):
        A, B = ob.frand((M, K), 6000 + i), ob.frand((K, N), 6100 + i)
        cases.append((A, B, ob.gemm_f64(A, B)))
    errors = []

    def worker(order):
        try:
            for _ in range(5):
                for i in order:
                    A, B, R = cases[i]
                    (M, K), N = A.shape, B.shape[1]
                    err = rel(sgemm(N_, N_, A, B, M, N, K), R)
                    if err > FP32_TOL:
                        errors.append((i, err))
        except Exception as e:  # surfaced by the assert below
            errors.append(repr(e))

    announce("sgemm two host threads")
    threads = [threading.Thread(target=worker, args=(o,)) for o in ([0, 1, 2, 3], [3, 2, 1, 0])]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads)
    assert errors == []


def test_sgemm_deterministic():
    M, N, K = 512, 512, 777
    A, B = _operands(N_, T_, M, N, K, 95)
    announce("sgemm determinism")
    C1 = sgemm(N_, T_, A, B, M, N, K)
    C2 = sgemm(N_, T_, A, B, M, N, K)
    np.testing.assert_array_equal(C1, C2)


# 350M-class shapes (M = 4 x 1024 tokens): forward NN, tied-head NT, and the
# trainer's backward layouts dX = dY.W^T (NT) and dW = X^T.dY (TN).
FULL = [
    ("qkv", N_, N_, 4096, 3072, 1024),
    ("attn_out", N_, N_, 4096, 1024, 1024),
    ("ff1", N_, N_, 4096, 4096, 1024),
    ("ff2", N_, N_, 4096, 1024, 4096),
    ("head", N_, T_, 4096, 50257, 1024),
    ("dX_ff1", N_, T_, 4096, 1024, 4096),
    ("dW_ff1", T_, N_, 1024, 4096, 4096),
]


@pytest.mark.parametrize("name,opA,opB,M,N,K", FULL)
def test_sgemm_350m_sampled(name, opA, opB, M, N, K):
    A = ob.normal((M, K) if opA == N_ else (K, M), 500, 0.0, 1.0)
    B = ob.normal((K, N) if opB == N_ else (N, K), 501, 0.0, 0.02)
    announce("sgemm 350M", name, M, N, K)
    C = sgemm(opA, opB, A, B, M, N, K)
    rows = np.random.default_rng(0).choice(M, 48, replace=False)
    Arows = A if opA == N_ else np.ascontiguousarray(A.T)
    R = sampled_rows_f64(Arows, B, rows, transB=opB == T_)
    assert rel(C[rows], R) <= FP32_TOL
    assert np.isfinite(C).all()


def test_sgemm_grown_prefill_ff1_with_bias():
    # the grown model's FFN up projection at prefill,
    # T = 256 tokens of d_model 512 into d_ff 2048 (transformer.c:150,
    # train.c:524 through matmul_forward, train.c:181-211): activations ~ N(0,1),
    # weights ~ N(0, 0.02), bias added; every output against the f64 truth and
    # the reference-order restatement (i-k-j, tensor.c:34-53) plus the bias
    M, K, N = 256, 512, 2048
    A = ob.normal((M, K), 610, 0.0, 1.0)
    W = ob.normal((K, N), 611, 0.0, 0.02)
    b = ob.normal((N,), 612, 0.0, 0.02)
    announce("sgemm grown FF1 + bias", M, N, K)
    C = sgemm(N_, N_, A, W, M, N, K, bias=b)
    assert rel(C, ob.gemm_f64(A, W, bias=b)) <= FP32_TOL
    assert rel(C, ob.matmul_ikj(A, W) + b) <= FP32_TOL


# The trainer's backward products on the 350M-class shapes (train.c:551-569:
# matmul_backward for the QKV, attention-output and FFN-down weights; d_model
# 1024, d_ff 4096, 4 x 1024 tokens), with upstream gradients ~ N(0, 1e-3)
# accumulated onto existing gradients as
# train.c's += does: dX = dY . W^T (NT), dW = X^T . dY (TN).
BWD = [  # name, layout, M, N, K, operand shapes (A, B)
    ("dX_qkv", N_, T_, 4096, 1024, 3072),
    ("dW_qkv", T_, N_, 1024, 3072, 4096),
    ("dX_attn_out", N_, T_, 4096, 1024, 1024),
    ("dW_attn_out", T_, N_, 1024, 1024, 4096),
    ("dX_ff2", N_, T_, 4096, 4096, 1024),
    ("dW_ff2", T_, N_, 4096, 1024, 4096),
]


@pytest.mark.parametrize("name,opA,opB,M,N,K", BWD)
def test_sgemm_350m_backward_sampled(name, opA, opB, M, N, K):
    if opA == N_:  # dX: A = dY (M x K gradients), B = W stored N x K
        A = ob.normal((M, K), 700, 0.0, 1e-3)
        B = ob.normal((N, K), 701, 0.0, 0.02)
    else:  # dW: A = X (K tokens x M), B = dY (K x N gradients)
        A = ob.normal((K, M), 702, 0.0, 1.0)
        B = ob.normal((K, N), 703, 0.0, 1e-3)
    C0 = ob.normal((M, N), 704, 0.0, 1e-3)
    announce("sgemm 350M backward", name, M, N, K)
    C = sgemm(opA, opB, A, B, M, N, K, C0=C0)
    rows = np.random.default_rng(5).choice(M, 48, replace=False)
    Arows = A if opA == N_ else np.ascontiguousarray(A.T)
    R = sampled_rows_f64(Arows, B, rows, transB=opB == T_) + C0[rows]
    assert rel(C[rows], R) <= FP32_TOL
    # the whole product through its row and column sums (f64): 1^T C and C 1
    Af, Bf = A.astype(np.float64), B.astype(np.float64)
    Aop = Af if opA == N_ else Af.T
    Bop = Bf.T if opB == T_ else Bf
    colsum = Aop.sum(0) @ Bop + C0.astype(np.float64).sum(0)
    rowsum = Aop @ Bop.sum(1) + C0.astype(np.float64).sum(1)
    assert rel(C.astype(np.float64).sum(0), colsum) <= FP32_TOL
    assert rel(C.astype(np.float64).sum(1), rowsum) <= FP32_TOL
