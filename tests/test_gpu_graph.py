"""Graph capture of native calls (decode loops): every replay must equal the
eager result bit for bit, including after eager work that grows the stream's
scratch between replays, and when the scratch first grows inside the capture.

The captured sequence mixes the products of a decode step: split-K GEMVs (two
kernels each: partial sums, then the ordered reduction), the tied-head GEMV,
INT8 GEMV and GEMM with dequantisation, and an FP32 GEMM.
"""
import ctypes as C

import numpy as np
import pytest

import binding as ob
import pcl
from gpu_util import announce, require_device

pytestmark = pytest.mark.gpu
OP_N, OP_T = 0, 1


@pytest.fixture(scope="module", autouse=True)
def _device():
    require_device()


@pytest.fixture()
def stream():
    s = pcl.lib.pcl_stream_create()
    assert s, pcl.last_error()
    pcl.check(pcl.lib.pcl_set_stream(s))
    yield s
    pcl.check(pcl.lib.pcl_stream_destroy(s))
    pcl.check(pcl.lib.pcl_set_stream(None))


def _packed(K, N, seed):
    Bq = ob.s8((K, N), seed)
    dB = pcl.dev(Bq)
    dBp = pcl.DeviceBuffer(pcl.lib.pcl_s8_packed_bytes(K, N))
    pcl.check(pcl.lib.pcl_pack_b_s8(dB.ptr, N, K, N, dBp.ptr, None, None))
    pcl.sync()
    return dBp


class Step:
    """Operands of one decode-like step and the calls that compute it."""

    def __init__(self):
        L = pcl.lib
        self.x = pcl.dev(ob.uniform((4, 2048), 1, -1, 1).astype(np.float32))
        self.W1 = pcl.dev(ob.uniform((2048, 512), 2, -0.02, 0.02).astype(np.float32))   # K x N
        self.Wh = pcl.dev(ob.uniform((2048, 512), 3, -0.02, 0.02).astype(np.float32))   # N x K (head)
        self.xu = pcl.dev(ob.u8((4, 512), 4))
        self.Bp = _packed(512, 1536, 5)
        self.sa = pcl.dev(ob.uniform((256,), 6, 1e-3, 1e-2).astype(np.float32))
        self.sb = pcl.dev(ob.uniform((1536,), 7, 1e-3, 1e-2).astype(np.float32))
        self.Au = pcl.dev(ob.u8((256, 512), 8))
        self.A = pcl.dev(ob.uniform((128, 64), 9, -1, 1).astype(np.float32))
        self.B = pcl.dev(ob.uniform((64, 96), 10, -1, 1).astype(np.float32))
        self.outs = {}
        self.L = L

    def alloc(self):
        return {
            "y1": pcl.empty((1, 512), np.float32),      # split-K GEMV, M=1
            "y4": pcl.empty((4, 512), np.float32),      # split-K GEMV, M=4
            "yh": pcl.empty((2, 2048), np.float32),     # tied head, M=2
            "yi": pcl.empty((4, 1536), np.float32),     # INT8 GEMV dequant
            "ci": pcl.empty((256, 1536), np.float32),   # INT8 GEMM dequant
            "cf": pcl.empty((128, 96), np.float32),     # FP32 GEMM
        }

    def run(self, o):
        L, c = self.L, pcl.check
        c(L.pcl_sgemv(OP_N, 1, 512, 2048, self.x.ptr, 2048, self.W1.ptr, 512, None, 0, o["y1"].ptr, 512, None))
        c(L.pcl_sgemv(OP_N, 4, 512, 2048, self.x.ptr, 2048, self.W1.ptr, 512, None, 0, o["y4"].ptr, 512, None))
        c(L.pcl_sgemv(OP_T, 2, 2048, 512, self.x.ptr, 2048, self.Wh.ptr, 512, None, 0, o["yh"].ptr, 2048, None))
        c(L.pcl_gemv_u8s8_dq(self.xu.ptr, 512, self.Bp.ptr, None, self.sa.ptr, self.sb.ptr, o["yi"].ptr, 1536,
                             4, 1536, 512, None))
        c(L.pcl_gemm_u8s8_dq(self.Au.ptr, 512, self.Bp.ptr, None, self.sa.ptr, self.sb.ptr, o["ci"].ptr, 1536,
                             256, 1536, 512, None))
        c(L.pcl_sgemm(OP_N, OP_N, 128, 96, 64, self.A.ptr, 64, self.B.ptr, 96, None, 0, o["cf"].ptr, 96, None))

    @staticmethod
    def fetch(o):
        pcl.sync()
        shapes = {"y1": (1, 512), "y4": (4, 512), "yh": (2, 2048), "yi": (4, 1536), "ci": (256, 1536),
                  "cf": (128, 96)}
        return {k: o[k].download(shapes[k], np.float32) for k in o}


def _capture(step, outs):
    pcl.check(pcl.lib.pcl_graph_begin())
    step.run(outs)
    g = C.c_void_p()
    pcl.check(pcl.lib.pcl_graph_end(C.byref(g)))
    assert g.value
    return g


@pytest.mark.parametrize("warm", [True, False], ids=["scratch-ready", "scratch-grows-in-capture"])
def test_graph_replays_match_eager(stream, warm):
    announce("graph capture", "warm" if warm else "cold")
    step = Step()
    eager_out = step.alloc()
    if warm:
        step.run(eager_out)
        ref = Step.fetch(eager_out)
    graph_out = step.alloc()
    g = _capture(step, graph_out)
    if not warm:
        step.run(eager_out)  # eager after capture, same stream and scratch
        ref = Step.fetch(eager_out)
    big = pcl.empty((8, 2048), np.float32)
    xb = pcl.dev(ob.uniform((8, 8192), 11, -1, 1).astype(np.float32))
    Wb = pcl.dev(ob.uniform((8192, 2048), 12, -0.01, 0.01).astype(np.float32))
    try:
        for r in range(3):
            for k in graph_out:  # poison the outputs (a synchronous host copy)
                graph_out[k].upload(np.full(graph_out[k].nbytes // 4, np.nan, np.float32))
            if r == 1:
                # eager work that needs a larger split-K workspace: the stream's
                # scratch grows and the buffer the graph recorded must survive
                pcl.check(pcl.lib.pcl_sgemv(OP_N, 8, 2048, 8192, xb.ptr, 8192, Wb.ptr, 2048, None, 0,
                                            big.ptr, 2048, None))
            pcl.check(pcl.lib.pcl_graph_launch(g))
            got = Step.fetch(graph_out)
            for k in ref:
                np.testing.assert_array_equal(got[k], ref[k], err_msg=f"replay {r}: {k}")
    finally:
        pcl.check(pcl.lib.pcl_graph_destroy(g))


def test_graph_needs_a_created_stream():
    pcl.check(pcl.lib.pcl_set_stream(None))
    assert pcl.lib.pcl_graph_begin() == pcl.PCL_ERR_INVALID_ARG


def test_host_dropins_refuse_under_capture(stream):
    # host-pointer drop-ins copy host operands and wait for the stream: while
    # the thread's stream captures they fail before touching it, the capture
    # stays valid, and they run again once it has ended
    announce("graph host drop-in refusal")
    M, K, N = 64, 32, 48
    A = ob.uniform((M, K), 20, -1, 1).astype(np.float32)
    B = ob.uniform((K, N), 21, -1, 1).astype(np.float32)
    Cout = np.full((M, N), np.nan, np.float32)
    dA, dB, dC = pcl.dev(A), pcl.dev(B), pcl.empty((M, N), np.float32)
    pcl.check(pcl.lib.pcl_graph_begin())
    try:
        pcl.lib.matmul(pcl.ptr(A), pcl.ptr(B), pcl.ptr(Cout), M, K, N)
        assert pcl.lib.pcl_last_status() == pcl.PCL_ERR_INVALID_ARG
        assert b"captured" in pcl.lib.pcl_last_error()
        assert np.isnan(Cout).all()
        pcl.check(pcl.lib.pcl_set_model_dims(N, N))
        lg = ob.normal((4, N), 22)
        t = np.arange(4, dtype=np.int32)
        dl = np.full_like(lg, np.nan)
        pcl.lib.cross_entropy(pcl.ptr(lg), pcl.ptr(t), pcl.ptr(dl), 4)
        assert pcl.lib.pcl_last_status() == pcl.PCL_ERR_INVALID_ARG
        # a native call is still recorded into the same capture
        pcl.check(pcl.lib.pcl_sgemm(OP_N, OP_N, M, N, K, dA.ptr, K, dB.ptr, N, None, 0, dC.ptr, N, None))
    finally:
        g = C.c_void_p()
        pcl.check(pcl.lib.pcl_graph_end(C.byref(g)))
    try:
        pcl.check(pcl.lib.pcl_graph_launch(g))
        pcl.sync()
        pcl.lib.matmul(pcl.ptr(A), pcl.ptr(B), pcl.ptr(Cout), M, K, N)
        pcl.check_void()
        np.testing.assert_array_equal(dC.download((M, N), np.float32), Cout)
        assert np.abs(Cout - A.astype(np.float64) @ B).max() <= 1e-4 * np.abs(Cout).max()
    finally:
        pcl.check(pcl.lib.pcl_graph_destroy(g))


def test_release_scratch(stream):
    # split-K GEMV workspace released and grown again: same bits; a stream a
    # graph was captured on keeps its scratch (the graph may use it)
    announce("release scratch")
    x = pcl.dev(ob.uniform((8, 8192), 30, -1, 1).astype(np.float32))
    W = pcl.dev(ob.uniform((8192, 2048), 31, -0.01, 0.01).astype(np.float32))
    y = pcl.empty((8, 2048), np.float32)

    def run():
        pcl.check(pcl.lib.pcl_sgemv(OP_N, 8, 2048, 8192, x.ptr, 8192, W.ptr, 2048, None, 0, y.ptr, 2048, None))
        pcl.sync()
        return y.download((8, 2048), np.float32)

    first = run()
    pcl.check(pcl.lib.pcl_release_scratch(stream))
    np.testing.assert_array_equal(run(), first)
    pcl.check(pcl.lib.pcl_graph_begin())
    pcl.check(pcl.lib.pcl_sgemv(OP_N, 8, 2048, 8192, x.ptr, 8192, W.ptr, 2048, None, 0, y.ptr, 2048, None))
    g = C.c_void_p()
    pcl.check(pcl.lib.pcl_graph_end(C.byref(g)))
    try:
        assert pcl.lib.pcl_release_scratch(stream) == pcl.PCL_ERR_INVALID_ARG
        pcl.check(pcl.lib.pcl_graph_launch(g))
        pcl.sync()
        np.testing.assert_array_equal(y.download((8, 2048), np.float32), first)
    finally:
        pcl.check(pcl.lib.pcl_graph_destroy(g))
