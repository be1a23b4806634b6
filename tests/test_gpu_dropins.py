"""The reference-signature drop-ins on the GPU, against the reference's own
outputs (tests/golden/, written by train.c / model.c / transformer.c /
tensor.c built from source) and the CPU oracle. FP32 bar: 1e-4 normwise.
"""
import hashlib
import os

import numpy as np
import pytest

import binding as ob
import pcl
from gpu_util import FP32_TOL, announce, rel, require_device

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")
p = ob.p
L = pcl.lib


@pytest.fixture(scope="module", autouse=True)
def _device():
    require_device()


def gold(name):
    return np.load(os.path.join(GOLD, name))


def test_matmul_golden():
    g = gold("tensor_matmul_f32.npz")
    for key in [k for k in g.files if k.startswith("C_")]:
        tag = key[2:]
        A, B, Cr = g["A_" + tag], g["B_" + tag], g[key]
        M, K = A.shape
        N = B.shape[1]
        Cm = np.full((M, N), np.nan, np.float32)
        announce("matmul", tag)
        L.matmul(p(A), p(B), p(Cm), M, K, N)
        pcl.check_void()
        assert rel(Cm, Cr) <= FP32_TOL, tag


def test_train_gemms_golden():
    g = gold("train_gemms.npz")
    M, K, N, Mh, D, V = (int(v) for v in g["dims"])
    Y = np.empty((M, N), np.float32)
    announce("matmul_forward")
    L.matmul_forward(p(Y), p(g["X"]), p(g["W"]), p(g["bias"]), M, K, N)
    pcl.check_void()
    assert rel(Y, g["Y"]) <= FP32_TOL
    dX, dW, db = g["dX0"].copy(), g["dW0"].copy(), g["db0"].copy()
    announce("matmul_backward")
    L.matmul_backward(p(g["dY"]), p(g["X"]), p(g["W"]), p(dX), p(dW), p(db), M, K, N)
    pcl.check_void()
    for got, want in ((dX, g["dX"]), (dW, g["dW"]), (db, g["db"])):
        assert rel(got, want) <= FP32_TOL
    pcl.check(L.pcl_set_model_dims(D, V))
    lo = np.empty((Mh, V), np.float32)
    announce("tied_head_forward")
    L.tied_head_forward(p(lo), p(g["lnf"]), p(g["wte"]), Mh)
    pcl.check_void()
    assert rel(lo, g["logits"]) <= FP32_TOL
    dlnf = np.full((Mh, D), 3.0, np.float32)
    dwte = g["dwte0"].copy()
    announce("tied_head_backward")
    L.tied_head_backward(p(dlnf), p(dwte), p(g["dlog"]), p(g["lnf"]), p(g["wte"]), Mh)
    pcl.check_void()
    assert rel(dlnf, g["dlnf"]) <= FP32_TOL
    assert rel(dwte, g["dwte"]) <= FP32_TOL


def test_decode_golden():
    g = gold("decode_gemv.npz")
    K, N, T, D, V = (int(v) for v in g["dims"])
    for fn in (L.proj_token, L.matvec):
        y = np.empty(N, np.float32)
        announce("decode gemv", fn.__name__)
        fn(p(y), p(g["x"]), p(g["W"]), p(g["b"]), K, N)
        pcl.check_void()
        assert rel(y, g["y"]) <= FP32_TOL
    s1, s2 = (int(v) for v in g["head_seeds"])
    xs = ob.normal((T, D), s1)
    wte = ob.normal((V, D), s2, 0.0, 0.02)
    assert hashlib.sha256(xs.tobytes() + wte.tobytes()).digest() == g["head_input_sha256"].tobytes()
    pcl.check(L.pcl_set_model_dims(D, V))
    lo = np.empty((T, V), np.float32)
    announce("lm_head")
    L.lm_head(p(lo), p(xs), p(wte), T)
    pcl.check_void()
    assert rel(lo, g["logits"]) <= FP32_TOL


def test_lm_head_prefill_and_tied_head_shapes():
    # grown model: D=512, V=2048; prefill T=256 (GEMM path) and T=1 (GEMV path)
    D, V = 512, 2048
    pcl.check(L.pcl_set_model_dims(D, V))
    wte = ob.normal((V, D), 60, 0.0, 0.02)
    for T in (256, 1, 8):
        x = ob.normal((T, D), 61 + T)
        lo = np.empty((T, V), np.float32)
        announce("lm_head", T)
        L.lm_head(p(lo), p(x), p(wte), T)
        pcl.check_void()
        ref = np.empty((T, V), np.float32)
        ob.oracle().orc_lm_head(p(ref), p(x), p(wte), T, D, V)
        assert rel(lo, ref) <= FP32_TOL


def test_device_api_head_backward_vocab_50257():
    # The GPU trainer's head backward (train_kaggle.cu:173-174) over a
    # 50257-float logits row: gemm_nn d_lnf = dlogits . wte and gemm_tn
    # dwte += dlogits^T . lnf. The misaligned rows take the realigned path
    # (64-float rows, the aligned core on the LDS-DMA kernel, the 17-wide
    # vocabulary edge on the generic kernel); f64 rows and vocabulary entries
    # on both sides of the edge are compared.
    M, V, D = 1024, 50257, 1024
    dl = ob.normal((M, V), 80, 0.0, 1e-3)
    wte = ob.normal((V, D), 81, 0.0, 0.02)
    lnf = ob.normal((M, D), 82)
    W0 = ob.normal((V, D), 83, 0.0, 1e-3)
    ddl, dwte, dlnf = pcl.dev(dl), pcl.dev(wte), pcl.dev(lnf)
    dout = pcl.empty((M, D), np.float32)
    dW = pcl.dev(W0)
    L.gpu_init()
    announce("gemm_nn head backward", M, V, D)
    L.gemm_nn(ddl.ptr, dwte.ptr, None, dout.ptr, M, V, D)
    pcl.check_void()
    announce("gemm_tn head backward", M, V, D)
    L.gemm_tn(ddl.ptr, dlnf.ptr, dW.ptr, M, V, D)
    pcl.check_void()
    pcl.sync()
    rows = np.unique(np.r_[0, M - 1, np.random.default_rng(5).choice(M, 30, replace=False)])
    R = dl[rows].astype(np.float64) @ wte.astype(np.float64)
    assert rel(dout.download((M, D), np.float32)[rows], R) <= FP32_TOL
    vs = np.unique(np.r_[0, 1, 63, 64, 50239, 50240, 50241, 50256, np.random.default_rng(6).choice(V, 30, replace=False)])
    R = W0[vs].astype(np.float64) + dl[:, vs].T.astype(np.float64) @ lnf.astype(np.float64)
    assert rel(dW.download((V, D), np.float32)[vs], R) <= FP32_TOL


def test_device_api_dropins():
    M, K, N = 300, 200, 260
    A = ob.normal((M, K), 70)
    B = ob.normal((K, N), 71, 0, 0.02)
    bias = ob.normal((N,), 72)
    dA, dB, db = pcl.dev(A), pcl.dev(B), pcl.dev(bias)
    dC = pcl.empty((M, N), np.float32)
    L.gpu_init()
    announce("gemm_nn")
    L.gemm_nn(dA.ptr, dB.ptr, db.ptr, dC.ptr, M, K, N)
    pcl.check_void()
    pcl.sync()
    assert rel(dC.download((M, N), np.float32), ob.gemm_f64(A, B, bias=bias)) <= FP32_TOL
    # gemm_nt: C(M,N) ?= A(M,K) B(N,K)^T
    Bt = np.ascontiguousarray(B.T)
    dBt = pcl.dev(Bt)
    C0 = ob.normal((M, N), 73)
    dC.upload(C0)
    announce("gemm_nt accum")
    L.gemm_nt(dA.ptr, dBt.ptr, dC.ptr, M, K, N, 1)
    pcl.check_void()
    pcl.sync()
    assert rel(dC.download((M, N), np.float32), ob.gemm_f64(A, B, C0=C0)) <= FP32_TOL
    announce("gemm_nt set")
    L.gemm_nt(dA.ptr, dBt.ptr, dC.ptr, M, K, N, 0)
    pcl.check_void()
    pcl.sync()
    assert rel(dC.download((M, N), np.float32), ob.gemm_f64(A, B)) <= FP32_TOL
    # gemm_tn: C(K,N) += A(M,K)^T B(M,N)
    Bm = ob.normal((M, N), 74)
    dBm = pcl.dev(Bm)
    W0 = ob.normal((K, N), 75)
    dW = pcl.dev(W0)
    announce("gemm_tn")
    L.gemm_tn(dA.ptr, dBm.ptr, dW.ptr, M, K, N)
    pcl.check_void()
    pcl.sync()
    R = W0.astype(np.float64) + A.T.astype(np.float64) @ Bm.astype(np.float64)
    assert rel(dW.download((K, N), np.float32), R) <= FP32_TOL
    db0 = ob.normal((N,), 76)
    ddb = pcl.dev(db0)
    announce("bias_bwd drop-in")
    L.bias_bwd(ddb.ptr, dBm.ptr, M, N)
    pcl.check_void()
    pcl.sync()
    assert rel(ddb.download((N,), np.float32), db0.astype(np.float64) + Bm.astype(np.float64).sum(0)) <= FP32_TOL


def test_dropin_errors_are_reported():
    pcl.check(L.pcl_set_model_dims(64, 96))
    L.pcl_clear_error()
    L.matmul(None, None, None, -1, 4, 4)
    assert L.pcl_last_status() == pcl.PCL_ERR_INVALID_ARG
    L.pcl_clear_error()
    assert L.pcl_set_model_dims(0, 5) == pcl.PCL_ERR_INVALID_ARG
