"""Softmax cross-entropy and the tied head fused with it, on the GPU, against
the oracle's restatement of train.c:449-465 (orc_cross_entropy, pinned by
train.c built from source in tests/test_oracle.py) and train.c:531/718/542 in
sequence (orc_head_ce).

Tolerances: against the same computation in float64, dlogits, d_lnf and dwte
max|X-R|/max|R| <= 1e-4 (FP32_TOL) and the mean loss to 1e-5 relative. Against
the oracle the bound is FP32_TOL plus the oracle's own distance from float64:
train.c adds the softmax denominator in one fp32 running sum, which at a 50257
vocabulary drops every term below half an ulp of the sum (about 2e-4 of p on a
row where one logit dominates); the kernel's per-thread sums keep them.
"""
import numpy as np
import pytest

import binding as ob
import pcl
from gpu_util import FP32_TOL, announce, rel, require_device

pytestmark = pytest.mark.gpu
LOSS_RTOL = 1e-5


@pytest.fixture(scope="module", autouse=True)
def _device():
    require_device()


def _inputs(M, V, seed, scale=3.0):
    lg = ob.normal((M, V), seed, 0.0, scale)
    t = (ob.u8((M,), seed + 1).astype(np.int64) * 7919 % V).astype(np.int32)
    t[0] = V - 1
    if M > 1:
        t[1] = 0
    return lg, t


def _ce64(lg, t):
    """float64 softmax cross-entropy: (mean loss, dlogits)."""
    x = lg.astype(np.float64)
    M = x.shape[0]
    mx = np.where(np.isfinite(x.max(1)), x.max(1), 0.0)[:, None]
    e = np.exp(x - mx)
    p = e / e.sum(1, keepdims=True)
    loss = float(np.mean(-np.log(p[np.arange(M), t] + 1e-30)))
    p[np.arange(M), t] -= 1.0
    return loss, p / M


def _check_ce(loss, dl, lg, t):
    want_loss, want_dl = ob.cross_entropy(lg, t)
    loss64, dl64 = _ce64(lg, t)
    assert loss == pytest.approx(loss64, rel=LOSS_RTOL, abs=1e-7)
    assert rel(dl, dl64) <= FP32_TOL
    own = abs(want_loss / loss64 - 1) if loss64 else 0.0  # the oracle's own distance
    assert loss == pytest.approx(want_loss, rel=LOSS_RTOL + own, abs=1e-7)
    assert rel(dl, want_dl) <= FP32_TOL + rel(want_dl, dl64)


def _ce(lg, t, ld=None, inplace=False, loss0=0.0):
    M, V = lg.shape
    ld = ld or V
    host = np.zeros((M, ld), np.float32)
    host[:, :V] = lg
    dlg, dt = pcl.dev(host), pcl.dev(t)
    dloss = pcl.dev(np.array([loss0], np.float32))
    dd = dlg if inplace else pcl.dev(np.full((M, ld), np.nan, np.float32))
    pcl.check(pcl.lib.pcl_cross_entropy(dlg.ptr, ld, dt.ptr, dd.ptr, ld, M, V, dloss.ptr, None))
    pcl.sync()
    return float(dloss.download((1,), np.float32)[0]), dd.download((M, ld), np.float32)[:, :V]


@pytest.mark.parametrize("M,V,ld,inplace", [(1, 96, None, False), (37, 2048, None, True),
                                            (300, 1000, 1024, False), (256, 50257, None, True),
                                            (4096, 2048, None, False), (5, 50257, 50304, True)])
def test_cross_entropy_vs_oracle(M, V, ld, inplace):
    announce("cross_entropy", M, V, ld, inplace)
    lg, t = _inputs(M, V, 1000 + M + V)
    loss, dl = _ce(lg, t, ld, inplace)
    _check_ce(loss, dl, lg, t)


@pytest.mark.parametrize("M,V", [(7, 1), (5, 3), (9, 5)])
def test_cross_entropy_tiny_vocab(M, V):
    # rows shorter than one 16-byte alignment head (V = 1: p = 1, loss 0, dl 0)
    lg, t = _inputs(M, V, 1050 + V)
    loss, dl = _ce(lg, t)
    _check_ce(loss, dl, lg, t)
    if V == 1:
        assert loss == 0.0 and not dl.any()


def test_cross_entropy_mixed_alignment():
    # logits rows of 1001 floats, dlogits rows of 1000: the two rows' 16-byte
    # phases differ, so the element-by-element path runs
    M, V = 40, 997
    lg, t = _inputs(M, V, 1060)
    host = np.zeros((M, 1001), np.float32)
    host[:, :V] = lg
    dlg, dt = pcl.dev(host), pcl.dev(t)
    dd = pcl.dev(np.full((M, 1000), np.nan, np.float32))
    dloss = pcl.dev(np.zeros(1, np.float32))
    pcl.check(pcl.lib.pcl_cross_entropy(dlg.ptr, 1001, dt.ptr, dd.ptr, 1000, M, V, dloss.ptr, None))
    pcl.sync()
    _check_ce(float(dloss.download((1,), np.float32)[0]), dd.download((M, 1000), np.float32)[:, :V], lg, t)


def test_cross_entropy_extreme_rows():
    # a near one-hot row, a row of -inf except two entries, uniform rows
    M, V = 4, 3000
    lg, t = _inputs(M, V, 1100, 1.0)
    lg[0] *= 40.0
    lg[1, :] = -np.inf
    lg[1, [5, 2999]] = [1.0, 2.0]
    t[1] = 5
    lg[2, :] = 7.0
    lg[3, :] = -3.0
    loss, dl = _ce(lg, t)
    assert np.isfinite(loss)
    _check_ce(loss, dl, lg, t)


def test_cross_entropy_loss_accumulates_and_bad_target():
    lg, t = _inputs(16, 500, 1200)
    loss, _ = _ce(lg, t, loss0=1.5)
    assert loss == pytest.approx(1.5 + ob.cross_entropy(lg, t)[0], rel=LOSS_RTOL)
    t[3] = 500
    loss, dl = _ce(lg, t)
    assert np.isnan(loss)
    # rows with valid targets are unaffected
    want = ob.cross_entropy(np.delete(lg, 3, 0), np.delete(t, 3))[1] * (15.0 / 16.0)
    assert rel(np.delete(dl, 3, 0), want) <= FP32_TOL


def test_cross_entropy_argument_errors():
    d = pcl.empty((8, 64), np.float32)
    dt = pcl.dev(np.zeros(8, np.int32))
    dloss = pcl.empty((1,), np.float32)
    off = pcl.lib.pcl_cross_entropy(d.ptr, 64, dt.ptr, d.ptr + 4, 64, 8, 64, dloss.ptr, None)
    assert off == pcl.PCL_ERR_INVALID_ARG
    assert pcl.lib.pcl_cross_entropy(d.ptr, 32, dt.ptr, d.ptr, 32, 8, 64, dloss.ptr, None) == \
        pcl.PCL_ERR_INVALID_ARG
    assert pcl.lib.pcl_cross_entropy(d.ptr, 64, dt.ptr, d.ptr, 64, 0, 64, dloss.ptr, None) == pcl.PCL_OK
    pcl.lib.pcl_clear_error()


def test_ce_dropins():
    # gpu_kernels.h:78-81 (device, M_ROWS = B*T) and train.c:450 (host)
    B, T, V = 2, 64, 777
    lg, t = _inputs(B * T, V, 1300)
    pcl.check(pcl.lib.pcl_set_model_dims(64, V))
    pcl.check(pcl.lib.pcl_set_attn_dims(B, T, 4))
    want_loss, want_dl = _ce64(lg, t)
    dlg, dt = pcl.dev(lg), pcl.dev(t)
    dloss = pcl.dev(np.zeros(1, np.float32))
    dd = pcl.dev(np.full_like(lg, np.nan))
    pcl.lib.ce_fwd_bwd(dlg.ptr, dt.ptr, dd.ptr, dloss.ptr)
    pcl.check_void()
    pcl.sync()
    assert float(dloss.download((1,), np.float32)[0]) == pytest.approx(want_loss, rel=LOSS_RTOL)
    assert rel(dd.download(lg.shape, np.float32), want_dl) <= FP32_TOL
    dl_host = np.full_like(lg, np.nan)
    loss = pcl.lib.cross_entropy(pcl.ptr(lg), pcl.ptr(t), pcl.ptr(dl_host), B * T)
    pcl.check_void()
    assert loss == pytest.approx(want_loss, rel=LOSS_RTOL)
    assert rel(dl_host, want_dl) <= FP32_TOL


def _head64(x, w, t, dw0=None):
    """float64 head + cross-entropy: (loss, d_lnf, dwte accumulated onto dw0)."""
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    loss, dl = _ce64(x64 @ w64.T, t)
    dw = dl.T @ x64
    return loss, dl @ w64, dw if dw0 is None else dw + dw0


def _head(x, w, t, dw0, chunk_bytes=0, want_dx=True, want_dw=True, loss0=0.0):
    M, D = x.shape
    V = w.shape[0]
    dx_, dw_, dt = pcl.dev(x), pcl.dev(w), pcl.dev(t)
    ddx = pcl.dev(np.full((M, D), np.nan, np.float32)) if want_dx else None
    ddw = pcl.dev(dw0) if want_dw else None
    dloss = pcl.dev(np.array([loss0], np.float32))
    pcl.check(pcl.lib.pcl_head_ce(dx_.ptr, dw_.ptr, dt.ptr, M, D, V, dloss.ptr,
                                  ddx.ptr if ddx else None, ddw.ptr if ddw else None, chunk_bytes, None))
    pcl.sync()
    return (float(dloss.download((1,), np.float32)[0]),
            ddx.download((M, D), np.float32) if ddx else None,
            ddw.download((V, D), np.float32) if ddw else None)


# (M, D, V, chunk rows or 0): the grown model, the 350M vocabulary, a ragged
# vocabulary (V % 64 != 0 and V < 64), several chunks with a ragged last one
HEAD_CASES = [(256, 512, 2048, 0), (64, 1024, 50257, 0), (100, 64, 1000, 0), (70, 32, 50, 0),
              (300, 128, 3001, 128), (257, 256, 2048, 1)]


@pytest.mark.parametrize("M,D,V,chunk_rows", HEAD_CASES)
def test_head_ce_vs_oracle(M, D, V, chunk_rows):
    announce("head_ce", M, D, V, chunk_rows)
    seed = 1400 + M + V
    x = ob.normal((M, D), seed, 0.0, 1.0)
    w = ob.normal((V, D), seed + 1, 0.0, 0.1)
    t = (ob.u8((M,), seed + 2).astype(np.int64) * 7919 % V).astype(np.int32)
    t[0] = V - 1
    dw0 = ob.normal((V, D), seed + 3, 0.0, 1e-3)
    ldp = (V + 63) // 64 * 64
    loss, dx, dw = _head(x, w, t, dw0, chunk_rows * ldp * 4, loss0=0.25)
    loss64, dx64, dw64 = _head64(x, w, t, dw0)
    assert loss == pytest.approx(0.25 + loss64, rel=LOSS_RTOL)
    assert rel(dx, dx64) <= FP32_TOL
    assert rel(dw - dw0, dw64 - dw0) <= FP32_TOL
    want_loss, want_dx, want_dw = ob.head_ce(x, w, t, dwte=dw0)
    assert rel(dx, want_dx) <= FP32_TOL + rel(want_dx, dx64)
    assert rel(dw - dw0, want_dw - dw0) <= FP32_TOL + rel(want_dw - dw0, dw64 - dw0)


def test_head_ce_optional_gradients():
    M, D, V = 128, 64, 700
    x = ob.normal((M, D), 1500, 0.0, 1.0)
    w = ob.normal((V, D), 1501, 0.0, 0.1)
    t = (np.arange(M) * 5 % V).astype(np.int32)
    dw0 = np.zeros((V, D), np.float32)
    loss_a, dx_a, dw_a = _head(x, w, t, dw0)
    loss_b, dx_b, _ = _head(x, w, t, dw0, want_dw=False)
    loss_c, _, dw_c = _head(x, w, t, dw0, want_dx=False)
    assert loss_a == loss_b == loss_c
    np.testing.assert_array_equal(dx_a, dx_b)
    np.testing.assert_array_equal(dw_a, dw_c)


def test_head_ce_350m_full_size():
    # 4096 x 1024 tokens x 50257 vocabulary (one 824 MB chunk): rows of d_lnf
    # depend on their own logits only, so sampled rows are checked against the
    # oracle run on those rows alone (rescaled from 1/4 to 1/M); the sum of dwte
    # over the vocabulary is sum_m (sum_v dl[m,v]) lnf[m] = 0; a run in chunks of
    # 1024 rows gives the same loss and gradients
    M, D, V = 4096, 1024, 50257
    announce("head_ce 350M", M, D, V)
    x = ob.normal((M, D), 1600, 0.0, 1.0)
    w = ob.normal((V, D), 1601, 0.0, 0.05)
    t = (ob.u8((M,), 1602).astype(np.int64) * 7919 % V).astype(np.int32)
    dw0 = np.zeros((V, D), np.float32)
    loss, dx, dw = _head(x, w, t, dw0)
    rows = np.array([0, 1, 2047, 4095])
    _, sub_dx, _ = _head64(x[rows], w, t[rows])
    assert rel(dx[rows], sub_dx * (len(rows) / M)) <= FP32_TOL
    colsum = dw.astype(np.float64).sum(0)
    assert np.abs(colsum).max() <= 1e-4 * np.abs(dw).max() * np.sqrt(V)
    loss_c, dx_c, dw_c = _head(x, w, t, dw0, 1024 * ((V + 63) // 64 * 64) * 4)
    assert loss_c == pytest.approx(loss, rel=LOSS_RTOL)
    assert rel(dx_c, dx) <= FP32_TOL
    assert rel(dw_c, dw) <= FP32_TOL
    assert np.log(V) * 0.5 < loss < np.log(V) * 2


def test_head_ce_realigned_operands():
    # D % 4 != 0 (rows not 16-byte aligned) and chunk products of >= 2^30
    # multiply-adds: the logits, d_lnf and dwte products copy their misaligned
    # operands into the stream's realign buffer while the logits chunk and the
    # row losses stay in the head's own scratch; two chunks of 256 rows
    M, D, V = 512, 1022, 8192
    announce("head_ce realigned", M, D, V)
    x = ob.normal((M, D), 1700, 0.0, 1.0)
    w = ob.normal((V, D), 1701, 0.0, 0.05)
    t = (ob.u8((M,), 1702).astype(np.int64) * 7919 % V).astype(np.int32)
    dw0 = ob.normal((V, D), 1703, 0.0, 1e-3)
    loss, dx, dw = _head(x, w, t, dw0, 256 * V * 4)
    loss64, dx64, dw64 = _head64(x, w, t, dw0)
    assert loss == pytest.approx(loss64, rel=LOSS_RTOL)
    assert rel(dx, dx64) <= FP32_TOL
    assert rel(dw - dw0, dw64 - dw0) <= FP32_TOL
