"""Causal attention parity on the GPU: pcl_attn_fwd (f32 MFMA, one fused launch)
against the CPU oracle (train.c:339-370 restated, pinned by the reference
built from source in tests/test_oracle.py).

Tolerance: max|X-R|/max|R| <= 1e-4 for att and for the stored probabilities,
the north-star fp32 bar. At the full 350M-class shape (B=4, T=1024, 16 heads of
64) sampled query rows are checked against f64 numpy, and every probability row
against the sizes-independent facts: each row sums to one and is zero above
the diagonal.
"""
import numpy as np
import pytest

import binding as ob
import pcl
from gpu_util import FP32_TOL, announce, rel, require_device

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    require_device()


def _qkv(B, T, ld, seed, std=1.0):
    return tuple(ob.normal((B * T, ld), seed + i, 0.0, std) for i in range(3))


def attn(q, k, v, B, T, H, dh, ld=None, probs=True, cols=(0, 0, 0)):
    """pcl_attn_fwd on device copies; q/k/v may share one buffer (cols = column
    offsets of Q, K, V inside it). Returns (att, probs or None)."""
    ld = q.shape[1] if ld is None else ld
    bufs = {}
    ptrs = []
    for a, c in zip((q, k, v), cols):
        key = id(a)
        if key not in bufs:
            bufs[key] = pcl.dev(a)
        ptrs.append(bufs[key].ptr + 4 * c)
    datt = pcl.dev(np.full((B * T, H * dh), np.nan, np.float32))
    dp = pcl.dev(np.full((B * H, T, T), np.nan, np.float32)) if probs else None
    pcl.check(pcl.lib.pcl_attn_fwd(ptrs[0], ptrs[1], ptrs[2], ld, datt.ptr, H * dh,
                                   dp.ptr if dp else None, B, T, H, dh, None))
    pcl.sync()
    att = datt.download((B * T, H * dh), np.float32)
    return att, (dp.download((B * H, T, T), np.float32) if dp else None)


# T = 96 and 160 end on a stage of two 32-key blocks whose second block lies past T;
# 130 has rows that are not a multiple of four floats (no 16-byte probability stores)
SHAPES = [(1, 1, 1, 32), (2, 33, 2, 32), (1, 128, 1, 64), (2, 200, 2, 64), (1, 129, 3, 128),
          (3, 256, 2, 128), (1, 300, 4, 32), (1, 96, 2, 64), (2, 160, 1, 32), (1, 130, 2, 64)]


@pytest.mark.parametrize("B,T,H,dh", SHAPES)
def test_attn_fwd_vs_oracle(B, T, H, dh):
    announce("attn_fwd", B, T, H, dh)
    q, k, v = _qkv(B, T, H * dh, 300 + T + dh)
    att, pr = attn(q, k, v, B, T, H, dh)
    att_r, pr_r = ob.attention_forward(q, k, v, B, T, H, dh)
    assert rel(att, att_r) <= FP32_TOL
    assert rel(pr, pr_r) <= FP32_TOL
    assert np.all(np.triu(pr, 1) == 0.0)


def attn_lse(q, k, v, B, T, H, dh):
    """pcl_attn_fwd_lse: (att, lse (B*H) x T)."""
    dq, dk, dv = pcl.dev(q), pcl.dev(k), pcl.dev(v)
    datt = pcl.dev(np.full((B * T, H * dh), np.nan, np.float32))
    dl = pcl.dev(np.full((B * H, T), np.nan, np.float32))
    pcl.check(pcl.lib.pcl_attn_fwd_lse(dq.ptr, dk.ptr, dv.ptr, q.shape[1], datt.ptr, H * dh, dl.ptr,
                                       B, T, H, dh, None))
    pcl.sync()
    return datt.download((B * T, H * dh), np.float32), dl.download((B * H, T), np.float32)


def probs_from_lse(q, k, lse, B, T, H, dh):
    """p_ij = exp(s_ij - lse_i) for j <= i, s = q.k / sqrtf(dh) in f64."""
    scale = np.float64(1.0 / np.sqrt(np.float32(dh)))
    P = np.zeros((B * H, T, T))
    for b in range(B):
        for h in range(H):
            c = slice(h * dh, (h + 1) * dh)
            S = q[b * T:(b + 1) * T, c].astype(np.float64) @ k[b * T:(b + 1) * T, c].astype(np.float64).T
            P[b * H + h] = np.tril(np.exp(S * scale - lse[b * H + h][:, None]))
    return P


@pytest.mark.parametrize("B,T,H,dh", SHAPES)
def test_attn_fwd_one_pass_and_lse_vs_oracle(B, T, H, dh):
    # the one-pass kernel (no probabilities): att against the oracle, and the
    # row log-sum-exp reproduces the oracle's probabilities exp(s - lse)
    announce("attn_fwd one pass", B, T, H, dh)
    q, k, v = _qkv(B, T, H * dh, 300 + T + dh)
    att, lse = attn_lse(q, k, v, B, T, H, dh)
    att_r, pr_r = ob.attention_forward(q, k, v, B, T, H, dh)
    assert rel(att, att_r) <= FP32_TOL
    assert rel(probs_from_lse(q, k, lse, B, T, H, dh), pr_r) <= FP32_TOL
    # pcl_attn_fwd without probabilities is the same kernel
    a2, _ = attn(q, k, v, B, T, H, dh, probs=False)
    np.testing.assert_array_equal(att, a2)


def test_attn_fwd_without_probs_agrees():
    B, T, H, dh = 2, 160, 2, 64
    announce("attn_fwd probs=NULL", B, T, H, dh)
    q, k, v = _qkv(B, T, H * dh, 410)
    a1, _ = attn(q, k, v, B, T, H, dh)
    a2, _ = attn(q, k, v, B, T, H, dh, probs=False)
    assert rel(a2, a1) <= FP32_TOL


def test_attn_fwd_fused_qkv_buffer():
    # Q, K, V as column slices of one (B*T) x 3D buffer (the fused QKV GEMM output)
    B, T, H, dh = 2, 96, 4, 32
    D = H * dh
    announce("attn_fwd fused qkv", B, T, H, dh)
    qkv = ob.normal((B * T, 3 * D), 420)
    att, pr = attn(qkv, qkv, qkv, B, T, H, dh, ld=3 * D, cols=(0, D, 2 * D))
    q, k, v = (np.ascontiguousarray(qkv[:, i * D:(i + 1) * D]) for i in range(3))
    att_r, pr_r = ob.attention_forward(q, k, v, B, T, H, dh)
    assert rel(att, att_r) <= FP32_TOL
    assert rel(pr, pr_r) <= FP32_TOL


def test_attn_fwd_large_scores():
    # scores of magnitude ~100 (no overflow: the row max is subtracted first)
    B, T, H, dh = 1, 64, 1, 64
    announce("attn_fwd large scores")
    q, k, v = _qkv(B, T, H * dh, 430, std=3.5)
    att, pr = attn(q, k, v, B, T, H, dh)
    att_r, pr_r = ob.attention_forward(q, k, v, B, T, H, dh)
    assert np.isfinite(att).all()
    assert rel(att, att_r) <= FP32_TOL
    assert rel(pr, pr_r) <= FP32_TOL
    # the one-pass kernel rescales as the running maximum grows
    att1, lse = attn_lse(q, k, v, B, T, H, dh)
    assert np.isfinite(att1).all() and np.isfinite(lse).all()
    assert rel(att1, att_r) <= FP32_TOL
    assert rel(probs_from_lse(q, k, lse, B, T, H, dh), pr_r) <= FP32_TOL


@pytest.mark.parametrize("B,T,H,dh", [(4, 1024, 16, 64), (4, 1024, 12, 128), (1, 256, 16, 32)])
def test_attn_fwd_full_size_properties(B, T, H, dh):
    # 350M-class (16 heads of 64, B=4, T=1024), the reference GPU trainer's heads
    # (12 of 128) and the grown model (16 of 32, T=256)
    announce("attn_fwd full", B, T, H, dh)
    q, k, v = _qkv(B, T, H * dh, 440 + dh)
    att, pr = attn(q, k, v, B, T, H, dh)
    np.testing.assert_allclose(pr.sum(axis=2, dtype=np.float64), 1.0, rtol=0, atol=2e-5)
    assert np.all(np.triu(pr, 1) == 0.0)
    rng = np.random.default_rng(7)
    scale = 1.0 / np.sqrt(np.float32(dh))
    worst = 0.0
    for _ in range(24):
        b, h, i = int(rng.integers(B)), int(rng.integers(H)), int(rng.integers(T))
        rows = slice(b * T, b * T + i + 1)
        cols = slice(h * dh, (h + 1) * dh)
        s = (k[rows, cols].astype(np.float64) @ q[b * T + i, cols].astype(np.float64)) * np.float64(scale)
        p = np.exp(s - s.max())
        p /= p.sum()
        o = p @ v[rows, cols].astype(np.float64)
        worst = max(worst, rel(att[b * T + i, cols], o), rel(pr[b * H + h, i, : i + 1], p))
    assert worst <= FP32_TOL
    # the one-pass kernel at the same size: sampled rows and their log-sum-exp
    att1, lse = attn_lse(q, k, v, B, T, H, dh)
    worst = 0.0
    for _ in range(24):
        b, h, i = int(rng.integers(B)), int(rng.integers(H)), int(rng.integers(T))
        rows = slice(b * T, b * T + i + 1)
        cols = slice(h * dh, (h + 1) * dh)
        s = (k[rows, cols].astype(np.float64) @ q[b * T + i, cols].astype(np.float64)) * np.float64(scale)
        ls = s.max() + np.log(np.exp(s - s.max()).sum())
        o = np.exp(s - ls) @ v[rows, cols].astype(np.float64)
        worst = max(worst, rel(att1[b * T + i, cols], o))
        assert abs(lse[b * H + h, i] - ls) <= 1e-5 * max(1.0, abs(ls))
    assert worst <= FP32_TOL


def test_attention_dropins():
    # train.c attention_forward (host pointers) and gpu_kernels.h attn_fwd
    # (device pointers), dims from pcl_set_model_dims / pcl_set_attn_dims
    B, T, H, dh = 2, 64, 4, 32
    D = H * dh
    announce("attention drop-ins", B, T, H, dh)
    pcl.check(pcl.lib.pcl_set_model_dims(D, 96))
    pcl.check(pcl.lib.pcl_set_attn_dims(B, T, H))
    q, k, v = _qkv(B, T, D, 450)
    att = np.zeros((B * T, D), np.float32)
    pr = np.zeros((B * H, T, T), np.float32)
    pcl.lib.attention_forward(pcl.ptr(q), pcl.ptr(k), pcl.ptr(v), pcl.ptr(att), pcl.ptr(pr), B, T)
    pcl.check_void()
    att_r, pr_r = ob.attention_forward(q, k, v, B, T, H, dh)
    assert rel(att, att_r) <= FP32_TOL and rel(pr, pr_r) <= FP32_TOL
    dq, dk, dv = pcl.dev(q), pcl.dev(k), pcl.dev(v)
    datt, dp = pcl.empty((B * T, D), np.float32), pcl.empty((B * H, T, T), np.float32)
    pcl.lib.attn_fwd(dq.ptr, dk.ptr, dv.ptr, datt.ptr, dp.ptr)
    pcl.check_void()
    pcl.sync()
    np.testing.assert_array_equal(datt.download((B * T, D), np.float32), att)
    np.testing.assert_array_equal(dp.download((B * H, T, T), np.float32), pr)


def test_attn_fwd_argument_errors():
    q = pcl.empty((64, 64), np.float32)
    for args in [(q.ptr, q.ptr, q.ptr, 64, q.ptr, 64, None, 1, 64, 1, 48, None),   # head size
                 (q.ptr, q.ptr, q.ptr, 30, q.ptr, 64, None, 1, 64, 1, 32, None),   # ld < H*dh
                 (q.ptr + 4, q.ptr, q.ptr, 64, q.ptr, 64, None, 1, 16, 1, 32, None)]:  # alignment
        assert pcl.lib.pcl_attn_fwd(*args) == pcl.PCL_ERR_INVALID_ARG
        assert pcl.lib.pcl_attn_fwd_lse(*args) == pcl.PCL_ERR_INVALID_ARG
        pcl.lib.pcl_clear_error()
    # lse may not overlap att
    a = pcl.empty((64, 64), np.float32)
    assert pcl.lib.pcl_attn_fwd_lse(q.ptr, q.ptr, q.ptr, 64, a.ptr, 64, a.ptr + 4 * 64, 1, 64, 2, 32,
                                    None) == pcl.PCL_ERR_INVALID_ARG
    pcl.lib.pcl_clear_error()


# ------------------------------------------------------------- backward ----
def attn_bwd(d_att, q, k, v, probs, B, T, H, dh, grads0=None, accumulate=False, scratch=False, att=None):
    """pcl_attn_bwd (pcl_attn_bwd_ex when the forward's output att is given)
    on device copies; returns (dq, dk, dv[, dS])."""
    D = H * dh
    bufs = [pcl.dev(x) for x in (d_att, q, k, v, probs)]
    g = grads0 if grads0 is not None else [np.full((B * T, D), np.nan, np.float32)] * 3
    dg = [pcl.dev(x) for x in g]
    ds = pcl.dev(np.zeros((B * H, T, T), np.float32)) if scratch else None
    if att is None:
        pcl.check(pcl.lib.pcl_attn_bwd(dg[0].ptr, dg[1].ptr, dg[2].ptr, D, ds.ptr if ds else None,
                                       bufs[0].ptr, D, bufs[1].ptr, bufs[2].ptr, bufs[3].ptr, D, bufs[4].ptr,
                                       B, T, H, dh, int(accumulate), None))
    else:
        da = pcl.dev(att)
        pcl.check(pcl.lib.pcl_attn_bwd_ex(dg[0].ptr, dg[1].ptr, dg[2].ptr, D, ds.ptr if ds else None,
                                          bufs[0].ptr, D, bufs[1].ptr, bufs[2].ptr, bufs[3].ptr, D,
                                          bufs[4].ptr, da.ptr, att.shape[1], B, T, H, dh, int(accumulate), None))
    pcl.sync()
    out = [x.download((B * T, D), np.float32) for x in dg]
    if scratch:
        out.append(ds.download((B * H, T, T), np.float32))
    return out


# 96 / 160: a last block inside T and its stage partner past it; 130: rows not a multiple of
# four floats (no 16-byte P and dS access) with heads of 64
@pytest.mark.parametrize("B,T,H,dh", [(1, 1, 1, 32), (2, 33, 2, 32), (1, 128, 1, 64), (2, 200, 2, 64),
                                      (1, 129, 3, 128), (2, 256, 2, 128), (1, 300, 4, 32), (1, 96, 2, 64),
                                      (2, 160, 1, 32), (1, 130, 2, 64)])
def test_attn_bwd_vs_oracle(B, T, H, dh):
    announce("attn_bwd", B, T, H, dh)
    D = H * dh
    q, k, v = _qkv(B, T, D, 500 + T + dh)
    d_att = ob.normal((B * T, D), 510 + T)
    _, pr = attn(q, k, v, B, T, H, dh)
    g0 = [ob.normal((B * T, D), 520 + i, 0.0, 0.1) for i in range(3)]
    got = attn_bwd(d_att, q, k, v, pr, B, T, H, dh, grads0=g0, accumulate=True)
    want = ob.attention_backward(d_att, q, k, v, pr, B, T, H, dh, *g0)
    for name, a, r in zip("qkv", got, want):
        assert rel(a, r) <= FP32_TOL, name
    # set mode equals accumulating onto zeros
    got0 = attn_bwd(d_att, q, k, v, pr, B, T, H, dh)
    want0 = ob.attention_backward(d_att, q, k, v, pr, B, T, H, dh)
    for name, a, r in zip("qkv", got0, want0):
        assert rel(a, r) <= FP32_TOL, name
    # given the forward's output, D_i = dAtt_i . att_i: the same gradients
    att, _ = attn(q, k, v, B, T, H, dh)
    got_ex = attn_bwd(d_att, q, k, v, pr, B, T, H, dh, grads0=g0, accumulate=True, att=att)
    for name, a, r in zip("qkv", got_ex, want):
        assert rel(a, r) <= FP32_TOL, name


@pytest.mark.parametrize("B,T,H,dh", [(4, 1024, 16, 64), (4, 1024, 12, 128)])
def test_attn_bwd_full_size_identities(B, T, H, dh):
    # With rows of P summing to one: sum_j dS_ij = 0 (so sum_j dK_j = 0 per
    # head) and sum_j dV_j = sum_i dAtt_i; sampled dQ rows against f64 numpy
    announce("attn_bwd full", B, T, H, dh)
    D = H * dh
    q, k, v = _qkv(B, T, D, 540 + dh)
    d_att = ob.normal((B * T, D), 545)
    _, pr = attn(q, k, v, B, T, H, dh)
    dq, dk, dv, ds = attn_bwd(d_att, q, k, v, pr, B, T, H, dh, scratch=True)
    scale = np.float64(1.0 / np.sqrt(np.float32(dh)))
    rs = np.tril(ds.astype(np.float64)).sum(axis=2)
    assert np.max(np.abs(rs)) <= 1e-4 * max(1.0, np.max(np.abs(ds)))
    for b in range(B):
        rows = slice(b * T, (b + 1) * T)
        sv = dv[rows].astype(np.float64).sum(axis=0)
        so = d_att[rows].astype(np.float64).sum(axis=0)
        assert np.max(np.abs(sv - so)) <= 1e-4 * np.max(np.abs(so)) * 4
        sk = dk[rows].astype(np.float64).sum(axis=0)
        assert np.max(np.abs(sk)) <= 1e-4 * max(1.0, np.max(np.abs(dk[rows])))
    rng = np.random.default_rng(11)
    worst = 0.0
    for _ in range(16):
        b, h, i = int(rng.integers(B)), int(rng.integers(H)), int(rng.integers(T))
        cols = slice(h * dh, (h + 1) * dh)
        keys = slice(b * T, b * T + i + 1)
        p = pr[b * H + h, i, : i + 1].astype(np.float64)
        dp = v[keys, cols].astype(np.float64) @ d_att[b * T + i, cols].astype(np.float64)
        dsr = p * (dp - np.dot(p, dp)) * scale
        worst = max(worst, rel(dq[b * T + i, cols], dsr @ k[keys, cols].astype(np.float64)),
                    rel(ds[b * H + h, i, : i + 1], dsr))
    assert worst <= FP32_TOL
    # with the forward's output: the same dS and gradients within the fp32 bar
    att, _ = attn(q, k, v, B, T, H, dh, probs=False)
    dq2, dk2, dv2, ds2 = attn_bwd(d_att, q, k, v, pr, B, T, H, dh, scratch=True, att=att)
    for a, r in ((dq2, dq), (dk2, dk), (dv2, dv), (np.tril(ds2), np.tril(ds))):
        assert rel(a, r) <= FP32_TOL


def test_attn_bwd_ex_argument_errors():
    q = pcl.empty((64, 64), np.float32)
    base = [q.ptr, q.ptr, q.ptr, 64, None, q.ptr, 64, q.ptr, q.ptr, q.ptr, 64, q.ptr]
    for att, ld_o in ((None, 64), (q.ptr, 30), (q.ptr, 62), (q.ptr + 4, 64)):
        assert pcl.lib.pcl_attn_bwd_ex(*base, att, ld_o, 1, 64, 2, 32, 0, None) == pcl.PCL_ERR_INVALID_ARG
        pcl.lib.pcl_clear_error()


def test_attention_backward_dropins():
    B, T, H, dh = 2, 64, 4, 32
    D = H * dh
    announce("attention backward drop-ins", B, T, H, dh)
    pcl.check(pcl.lib.pcl_set_model_dims(D, 96))
    pcl.check(pcl.lib.pcl_set_attn_dims(B, T, H))
    q, k, v = _qkv(B, T, D, 560)
    d_att = ob.normal((B * T, D), 565)
    _, pr = ob.attention_forward(q, k, v, B, T, H, dh)
    g = [np.ones((B * T, D), np.float32) for _ in range(3)]
    pcl.lib.attention_backward(*[pcl.ptr(x) for x in g], pcl.ptr(d_att), pcl.ptr(q), pcl.ptr(k),
                               pcl.ptr(v), pcl.ptr(pr), B, T)
    pcl.check_void()
    want = ob.attention_backward(d_att, q, k, v, pr, B, T, H, dh,
                                 *[np.ones((B * T, D), np.float32) for _ in range(3)])
    for a, r in zip(g, want):
        assert rel(a, r) <= FP32_TOL
    bufs = [pcl.dev(x) for x in (d_att, q, k, v, pr)]
    dg = [pcl.dev(np.full((B * T, D), 7.0, np.float32)) for _ in range(3)]
    scr = pcl.empty((B * H, T, T), np.float32)
    pcl.lib.attn_bwd(dg[0].ptr, dg[1].ptr, dg[2].ptr, scr.ptr, *[x.ptr for x in bufs])
    pcl.check_void()
    pcl.sync()
    want0 = ob.attention_backward(d_att, q, k, v, pr, B, T, H, dh)  # gpu_kernels.cu: beta = 0
    for x, r in zip(dg, want0):
        assert rel(x.download((B * T, D), np.float32), r) <= FP32_TOL
