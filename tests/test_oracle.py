"""Pin the CPU oracle (oracle/pcl_oracle.c) before trusting it.

Each restated function is checked by something other than its own formula:
the reference's known-answer test, closed forms and invariants, numpy's f64
matmul as a library routine, the golden fixtures written by the reference's
own code (tests/golden/), and -- where this container built it -- the
reference compiled from source (oracle/_ref). A planted mistake (dropped
term, transposed operand, wrong offset) fails at least one of these.
"""
import hashlib
import os

import numpy as np
import pytest

import binding as ob

p = ob.p
O = ob.oracle
# The reference is built with -ffast-math (reassociated, vectorised fp32 sums),
# so reference-vs-restatement fp32 agreement is ~1e-6; 1e-5 is the bar here,
# ten times tighter than the GPU's 1e-4 and far below any dropped-term error.
REF_TOL = 1e-5
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def gold(name):
    return np.load(os.path.join(GOLD, name))


# ------------------------------------------------------------------ PRNG ----
def _xorshift_py(s, n):
    out = []
    for _ in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out.append(s)
    return out


def test_xorshift_matches_recurrence():
    # train.c:73-78 recurrence, restated independently in Python
    import ctypes

    st = ctypes.c_uint32(12345)
    got = [O().orc_xorshift32(ctypes.byref(st)) for _ in range(10)]
    assert got == _xorshift_py(12345, 10)


def test_frand_formula():
    a = ob.frand((8,), 1234, 0.02)
    want = [((x & 0xFFFFFF) / 16777216.0 * 2.0 - 1.0) * 0.02 for x in _xorshift_py(1234, 8)]
    np.testing.assert_allclose(a, np.float32(want), rtol=0, atol=1e-9)


def test_int_fills_cover_range():
    u = ob.u8((1 << 16,), 7)
    s = ob.s8((1 << 16,), 8)
    assert u.min() == 0 and u.max() == 255
    assert s.min() == -128 and s.max() == 127
    assert abs(u.astype(float).mean() - 127.5) < 2 and abs(s.astype(float).mean() + 0.5) < 2


def test_normal_moments():
    z = ob.normal((200000,), 99, 0.0, 1.0)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01


# ------------------------------------------------------------ FP32 KATs ----
def _kat_closed_form(M, K, N):
    i = np.arange(M)[:, None]
    k = np.arange(K)[None, :]
    a = ((i * K + k) % 13 - 6).astype(np.int64)  # A[i,k] = 0.1*a
    kk = np.arange(K)[:, None]
    j = np.arange(N)[None, :]
    b = ((kk * N + j) % 7 - 3).astype(np.int64)
    return (a @ b).astype(np.float64) * 0.01


def test_tensor_selftest_kat_c00():
    # tensor.c:204-205 inputs, tensor.c:237-241 check: C[0,0] = 0.07000
    M = K = N = 1024
    A = np.empty(M * K, np.float32)
    B = np.empty(K * N, np.float32)
    O().orc_fill_kat_tensor(p(A), A.size, p(B), B.size)
    Cm = ob.matmul_ikj(A.reshape(M, K), B.reshape(K, N))
    assert abs(float(Cm[0, 0]) - 0.07) < 5e-5
    ref = _kat_closed_form(M, K, N)
    assert abs(ref[0, 0] - 0.07) < 1e-12
    assert ob.normwise_rel_err(Cm, ref) < 1e-5


def test_closed_form_full_matrix_small():
    M, K, N = 37, 90, 53  # K coprime to 7 and 13: non-degenerate sums
    A = np.empty(M * K, np.float32)
    B = np.empty(K * N, np.float32)
    O().orc_fill_kat_tensor(p(A), A.size, p(B), B.size)
    A, B = A.reshape(M, K), B.reshape(K, N)
    want = _kat_closed_form(M, K, N)
    for got in (ob.matmul_ikj(A, B), ob.gemm_f64(A, B)):
        assert ob.normwise_rel_err(got, want) < 1e-6


def test_identity_ones_and_empty_k():
    B = ob.frand((64, 48), 3)
    I = np.eye(64, dtype=np.float32)
    np.testing.assert_array_equal(ob.matmul_ikj(I, B), B)
    np.testing.assert_array_equal(ob.gemm_f64(I, B), B)
    ones = np.ones((5, 64), np.float32)
    np.testing.assert_allclose(ob.gemm_f64(ones, B), np.repeat(B.astype(np.float64).sum(0, keepdims=True), 5, 0),
                               rtol=1e-6)
    z = ob.gemm_f64(np.zeros((4, 0), np.float32), np.zeros((0, 6), np.float32),
                    bias=np.arange(6, dtype=np.float32))
    np.testing.assert_array_equal(z, np.tile(np.arange(6, dtype=np.float32), (4, 1)))


@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (7, 13, 5), (64, 100, 33)])
def test_gemm_layouts_against_numpy(M, K, N):
    A = ob.frand((M, K), 11)
    B = ob.frand((K, N), 12)
    want = A.astype(np.float64) @ B.astype(np.float64)
    Cnn = np.empty((M, N), np.float32)
    O().orc_gemm_nn(p(A), p(B), None, p(Cnn), M, K, N)
    assert ob.normwise_rel_err(Cnn, want) < 1e-7
    Bt = np.ascontiguousarray(B.T)  # (N,K)
    Cnt = np.full((M, N), 0.5, np.float32)
    O().orc_gemm_nt(p(A), p(Bt), p(Cnt), M, K, N, 1)  # accumulate onto 0.5
    assert ob.normwise_rel_err(Cnt - 0.5, want) < 1e-6
    # TN: C(K,N) += A(M,K)^T B(M,N) -- use A as the (M,K) operand, A2 as (M,N)
    A2 = ob.frand((M, N), 13)
    Ctn = np.zeros((K, N), np.float32)
    O().orc_gemm_tn(p(A), p(A2), p(Ctn), M, K, N)
    assert ob.normwise_rel_err(Ctn, A.T.astype(np.float64) @ A2.astype(np.float64)) < 1e-7


def test_transpose_identity_links_layouts():
    # (A.B)^T = B^T A^T: nn(A,B) equals nt(A, B^T) and tn(A^T stored, B)
    A = ob.frand((19, 23), 21)
    B = ob.frand((23, 29), 22)
    nn = ob.gemm_f64(A, B)
    nt = ob.gemm_f64(A, np.ascontiguousarray(B.T), transB=True)
    tn = ob.gemm_f64(np.ascontiguousarray(A.T), B, transA=True)
    np.testing.assert_array_equal(nn, nt)
    np.testing.assert_array_equal(nn, tn)


def test_matvec_bias_init_and_order():
    M, K, N = 3, 50, 70
    x = ob.normal((M, K), 31)
    W = ob.normal((K, N), 32, 0, 0.02)
    b = ob.normal((N,), 33)
    y = np.empty((M, N), np.float32)
    O().orc_matvec(p(y), p(x), p(W), p(b), M, K, N)
    assert ob.normwise_rel_err(y, x.astype(np.float64) @ W + b) < 1e-6
    O().orc_matvec(p(y), p(x), p(W), None, M, K, N)
    assert ob.normwise_rel_err(y, x.astype(np.float64) @ W) < 1e-6


# ---------------------------------------------- golden (reference output) ----
def test_golden_tensor_matmul():
    g = gold("tensor_matmul_f32.npz")
    for key in [k for k in g.files if k.startswith("C_")]:
        tag = key[2:]
        A, B, Cr = g["A_" + tag], g["B_" + tag], g[key]
        assert ob.normwise_rel_err(ob.matmul_ikj(A, B), Cr) < REF_TOL, tag


def test_golden_train_gemms():
    g = gold("train_gemms.npz")
    M, K, N, Mh, D, V = (int(v) for v in g["dims"])
    Y = np.empty((M, N), np.float32)
    O().orc_matmul_forward(p(Y), p(g["X"]), p(g["W"]), p(g["bias"]), M, K, N)
    assert ob.normwise_rel_err(Y, g["Y"]) < REF_TOL
    dX, dW, db = g["dX0"].copy(), g["dW0"].copy(), g["db0"].copy()
    O().orc_matmul_backward(p(g["dY"]), p(g["X"]), p(g["W"]), p(dX), p(dW), p(db), M, K, N)
    for got, want in ((dX, g["dX"]), (dW, g["dW"]), (db, g["db"])):
        assert ob.normwise_rel_err(got, want) < REF_TOL
    lo = np.empty((Mh, V), np.float32)
    O().orc_tied_head_forward(p(lo), p(g["lnf"]), p(g["wte"]), Mh, D, V)
    assert ob.normwise_rel_err(lo, g["logits"]) < REF_TOL
    dlnf = np.full((Mh, D), 3.0, np.float32)
    dwte = g["dwte0"].copy()
    O().orc_tied_head_backward(p(dlnf), p(dwte), p(g["dlog"]), p(g["lnf"]), p(g["wte"]), Mh, D, V)
    assert ob.normwise_rel_err(dlnf, g["dlnf"]) < REF_TOL
    assert ob.normwise_rel_err(dwte, g["dwte"]) < REF_TOL


def test_golden_decode():
    g = gold("decode_gemv.npz")
    K, N, T, D, V = (int(v) for v in g["dims"])
    y = np.empty((1, N), np.float32)
    O().orc_matvec(p(y), p(g["x"]), p(g["W"]), p(g["b"]), 1, K, N)
    assert ob.normwise_rel_err(y[0], g["y"]) < REF_TOL
    s1, s2 = (int(v) for v in g["head_seeds"])
    xs = ob.normal((T, D), s1)
    wte = ob.normal((V, D), s2, 0.0, 0.02)
    assert hashlib.sha256(xs.tobytes() + wte.tobytes()).digest() == g["head_input_sha256"].tobytes()
    lo = np.empty((T, V), np.float32)
    O().orc_lm_head(p(lo), p(xs), p(wte), T, D, V)
    assert ob.normwise_rel_err(lo, g["logits"]) < REF_TOL


def test_golden_gemm_bench_int8():
    g = gold("gemm_bench_int8.npz")
    M, K, N, Kpad = (int(v) for v in g["dims"])
    Au = np.empty((M, Kpad), np.uint8)
    scale = O().orc_quantize_A(p(g["A"]), p(Au), M, K, Kpad)
    assert np.float32(scale) == g["scale"]
    np.testing.assert_array_equal(Au, g["Au"])
    Bp = np.empty_like(g["Bp"])
    bscale = np.empty(N, np.float32)
    colsum = np.empty(N, np.int32)
    O().orc_quantize_B_pack(p(g["B"]), p(Bp), p(bscale), p(colsum), K, N, Kpad)
    np.testing.assert_array_equal(Bp, g["Bp"])
    np.testing.assert_array_equal(bscale, g["bscale"])
    np.testing.assert_array_equal(colsum, g["colsum"])
    Cq = np.empty((M, N), np.float32)
    O().orc_gemm_int8_kernel(p(g["Au"]), Kpad, p(g["Bp"]), p(g["corr"]), p(g["dq"]), p(Cq), M, N)
    np.testing.assert_array_equal(Cq, g["C_int8"])  # bit-exact, reference op order
    # the offset identity: v = sum Au*Bq - 128*colsum = sum (Au-128)*Bq
    Bq = np.empty((Kpad, N), np.int8)
    O().orc_unpack_vnni(p(g["Bp"]), p(Bq), Kpad, N, Kpad)
    V = ob.gemm_u8s8_i32(g["Au"], Bq)
    np.testing.assert_array_equal(ob.dequant(V, None, g["dq"]), g["C_int8"])
    # INT8 vs FP32 of the same inputs: README.md:31 reports 0.56% RMS relative
    assert O().orc_rms_rel(p(Cq), p(g["C_f32"]), Cq.size) < 0.02


# -------------------------------------------------------- INT8 identities ----
def test_vnni_offset_identity_and_special_cases():
    M, K, N = 16, 96, 32
    Au = ob.u8((M, K), 41)
    Bq = ob.s8((K, N), 42)
    raw = np.empty((M, N), np.int32)
    O().orc_gemm_u8s8_raw_i32(p(Au), K, p(Bq), N, p(raw), N, M, N, K)
    v = ob.gemm_u8s8_i32(Au, Bq)
    colsum = Bq.astype(np.int64).sum(0)
    np.testing.assert_array_equal(raw.astype(np.int64) - 128 * colsum, v)
    np.testing.assert_array_equal(v, (Au.astype(np.int64) - 128) @ Bq.astype(np.int64))
    # Au == 128 everywhere -> exactly zero; Bq == 1 -> row sums of (Au - 128)
    assert not ob.gemm_u8s8_i32(np.full((M, K), 128, np.uint8), Bq).any()
    rs = (Au.astype(np.int64) - 128).sum(1)
    np.testing.assert_array_equal(ob.gemm_u8s8_i32(Au, np.ones((K, N), np.int8)), np.repeat(rs[:, None], N, 1))


def test_int8_extreme_values_fit_int32():
    # |sum| <= K*128*128: all -128 activations against all -128 weights
    K = 4096
    v = ob.gemm_u8s8_i32(np.zeros((1, K), np.uint8), np.full((K, 2), -128, np.int8))
    assert int(v[0, 0]) == K * 128 * 128


def test_quantizer_rules():
    # round half away from zero, clamp to +-127, 128 padding
    A = np.array([[0.5, -0.5, 1.5, -2.5, 127.0, -127.0, 0.0]], np.float32)
    Au = np.empty((1, 8), np.uint8)
    s = O().orc_quantize_A(p(A), p(Au), 1, 7, 8)
    assert s == np.float32(127.0) * np.float32(np.float32(1) / np.float32(127))
    np.testing.assert_array_equal(Au[0].astype(int) - 128, [1, -1, 2, -3, 127, -127, 0, 0])
    sa = np.empty(2, np.float32)
    A2 = np.array([[1.0, -2.0], [0.0, 0.0]], np.float32)
    Au2 = np.empty((2, 2), np.uint8)
    O().orc_quantize_A_rows(p(A2), p(Au2), p(sa), 2, 2, 2)
    R = np.float32(np.float32(1) / np.float32(127))
    assert sa[0] == np.float32(2.0) * R and sa[1] == np.float32(1e-8) * R
    np.testing.assert_array_equal(Au2[1], [128, 128])


def test_rms_rel_kat():
    # README.md:31: per-tensor A / per-column B INT8 vs FP32 = 0.56% RMS rel.
    M = K = N = 1024
    A = ob.frand((M, K), 51)
    B = ob.frand((K, N), 52)
    Au = np.empty((M, K), np.uint8)
    sa = O().orc_quantize_A(p(A), p(Au), M, K, K)
    Bq = np.empty((K, N), np.int8)
    bs = np.empty(N, np.float32)
    O().orc_quantize_B_cols(p(B), p(Bq), p(bs), K, N)
    V = ob.gemm_u8s8_i32(Au, Bq)
    Cq = ob.dequant(V, None, (np.float32(sa) * bs).astype(np.float32))
    Cf = ob.gemm_f64(A, B)
    rel = O().orc_rms_rel(p(Cq), p(Cf), Cq.size)
    assert 4.5e-3 < rel < 7e-3


# -------------------------------------- the reference built from source ----
def _ref_or_skip(name):
    lib = ob.ref(name)
    if lib is None:
        pytest.skip(f"oracle/_ref/{name} not built (reference tree absent at build time)")
    return lib


def test_oracle_vs_ref_gemm_bench_rungs():
    gb = _ref_or_skip("libref_gemm_bench.so")
    if not gb.pcl_ref_cpu_ok():
        pytest.skip("host CPU lacks AVX-512 VNNI")
    M, K, N = 128, 256, 512  # gemm_bench's v3 block divisibility (gemm_bench.c:341)
    A = ob.frand((M, K), 61)
    B = ob.frand((K, N), 62)
    mine = ob.matmul_ikj(A, B)
    for name in ("pcl_ref_gemm_ikj", "pcl_ref_gemm_naive", "pcl_ref_gemm_micro", "pcl_ref_gemm_packed",
                 "pcl_ref_gemm_packed_mt"):
        Cr = np.empty((M, N), np.float32)
        getattr(gb, name)(p(A), p(B), p(Cr), M, K, N)
        assert ob.normwise_rel_err(mine, Cr) < REF_TOL, name


def test_oracle_vs_ref_int8_random():
    gb = _ref_or_skip("libref_gemm_bench.so")
    if not gb.pcl_ref_cpu_ok():
        pytest.skip("host CPU lacks AVX-512 VNNI")
    M, K, N = 40, 333, 48
    Kpad = (K + 3) & ~3
    A = ob.normal((M, K), 71)
    B = ob.normal((K, N), 72, 0, 0.02)
    Au_r, Au_o = np.empty((M, Kpad), np.uint8), np.empty((M, Kpad), np.uint8)
    s_r = gb.pcl_ref_quantize_A(p(A), p(Au_r), M, K, Kpad)
    s_o = O().orc_quantize_A(p(A), p(Au_o), M, K, Kpad)
    assert np.float32(s_r) == np.float32(s_o)
    np.testing.assert_array_equal(Au_r, Au_o)
    nbp = (N // 16) * (Kpad // 4) * 64
    outs = []
    for fn in (gb.pcl_ref_quantize_B_pack, O().orc_quantize_B_pack):
        Bp, bs, cs = np.empty(nbp, np.int8), np.empty(N, np.float32), np.empty(N, np.int32)
        fn(p(B), p(Bp), p(bs), p(cs), K, N, Kpad)
        outs.append((Bp, bs, cs))
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)
    Bp, bs, cs = outs[0]
    corr = (128 * cs).astype(np.int32)
    dq = (np.float32(s_r) * bs).astype(np.float32)
    Cr, Co = np.empty((M, N), np.float32), np.empty((M, N), np.float32)
    gb.pcl_ref_gemm_int8_kernel(p(Au_r), Kpad, p(Bp), p(corr), p(dq), p(Cr), M - M % 8, N)
    O().orc_gemm_int8_kernel(p(Au_r), Kpad, p(Bp), p(corr), p(dq), p(Co), M, N)
    np.testing.assert_array_equal(Cr[: M - M % 8], Co[: M - M % 8])


def test_oracle_vs_ref_train_and_model():
    tr = _ref_or_skip("libref_train.so")
    md = _ref_or_skip("libref_model.so")
    M, K, N = 33, 17, 48
    dY = ob.normal((M, N), 81)
    X = ob.normal((M, K), 82)
    W = ob.normal((K, N), 83)
    res = []
    for fn in (tr.pcl_ref_matmul_backward, O().orc_matmul_backward):
        dX, dW, db = np.ones((M, K), np.float32), np.ones((K, N), np.float32), np.ones(N, np.float32)
        fn(p(dY), p(X), p(W), p(dX), p(dW), p(db), M, K, N)
        res.append((dX, dW, db))
    for a, b in zip(*res):
        assert ob.normwise_rel_err(a, b) < REF_TOL
    x = ob.normal((130,), 84)
    Wp = ob.normal((130, 77), 85)
    y_r, y_o = np.empty(77, np.float32), np.empty(77, np.float32)
    md.pcl_ref_proj_token(p(y_r), p(x), p(Wp), None, 130, 77)
    O().orc_matvec(p(y_o), p(x), p(Wp), None, 1, 130, 77)
    assert ob.normwise_rel_err(y_o, y_r) < REF_TOL


# ------------------------------------------------------------ attention ----
def _qkv(B, T, D, seed, std=1.0):
    return (ob.normal((B * T, D), seed, 0.0, std), ob.normal((B * T, D), seed + 1, 0.0, std),
            ob.normal((B * T, D), seed + 2, 0.0, std))


@pytest.mark.parametrize("lib", ["libref_train.so", "libref_train_h64.so"])
def test_attention_oracle_vs_ref_train(lib):
    # train.c:339-407 compiled from source at d_head 16 (D=64, 4 heads, T<=16)
    # and d_head 64 (D=128, 2 heads, T<=64); forward and accumulating backward
    tr = _ref_or_skip(lib)
    D, H, Tmax = tr.pcl_ref_train_d_model(), tr.pcl_ref_train_n_heads(), tr.pcl_ref_train_t_size()
    dh = D // H
    B, T = 3, Tmax - 3
    q, k, v = _qkv(B, T, D, 91)
    att_r = np.zeros((B * T, D), np.float32)
    pr_r = np.zeros((B * H, T, T), np.float32)
    tr.pcl_ref_attention_forward(p(q), p(k), p(v), p(att_r), p(pr_r), B, T)
    att_o, pr_o = ob.attention_forward(q, k, v, B, T, H, dh)
    assert ob.normwise_rel_err(att_o, att_r) < REF_TOL
    assert ob.normwise_rel_err(pr_o, pr_r) < REF_TOL
    d_att = ob.normal((B * T, D), 95)
    grads_r = [np.ones((B * T, D), np.float32) for _ in range(3)]
    tr.pcl_ref_attention_backward(p(grads_r[0]), p(grads_r[1]), p(grads_r[2]), p(d_att), p(q), p(k),
                                  p(v), p(pr_r), B, T)
    grads_o = ob.attention_backward(d_att, q, k, v, pr_o, B, T, H, dh,
                                    *[np.ones((B * T, D), np.float32) for _ in range(3)])
    for a, b in zip(grads_o, grads_r):
        assert ob.normwise_rel_err(a, b) < REF_TOL


def test_attention_oracle_closed_forms():
    B, T, H, dh = 2, 9, 2, 32
    D = H * dh
    q, k, v = _qkv(B, T, D, 101)
    # T = 1: the single probability is 1 and att = v
    att, pr = ob.attention_forward(q[:1], k[:1], v[:1], 1, 1, H, dh)
    np.testing.assert_array_equal(att, v[:1])
    assert np.all(pr == 1.0)
    # equal keys: uniform probabilities 1/(i+1), att_i = running mean of v
    kc = np.repeat(k[:1], B * T, axis=0)
    att, pr = ob.attention_forward(q, kc, v, B, T, H, dh)
    for b in range(B):
        for i in range(T):
            want = v[b * T: b * T + i + 1].astype(np.float64).mean(axis=0)
            np.testing.assert_allclose(att[b * T + i], want, rtol=0, atol=1e-5)
            np.testing.assert_allclose(pr[b * H, i, : i + 1], 1.0 / (i + 1), rtol=1e-6)
    # rows of p sum to one, zero above the diagonal
    att, pr = ob.attention_forward(q, k, v, B, T, H, dh)
    np.testing.assert_allclose(pr.sum(axis=2), 1.0, rtol=0, atol=1e-6)
    assert np.all(np.triu(pr, 1) == 0.0)


@pytest.mark.parametrize("dh", [32, 64, 128])
def test_attention_oracle_vs_f64(dh):
    B, T, H = 2, 40, 2
    q, k, v = _qkv(B, T, H * dh, 111)
    a32, p32 = ob.attention_forward(q, k, v, B, T, H, dh)
    a64, p64 = ob.attention_forward(q, k, v, B, T, H, dh, f64=True)
    assert ob.normwise_rel_err(a32, a64) < 1e-5
    assert ob.normwise_rel_err(p32, p64) < 1e-5


def test_attention_backward_vs_central_differences():
    # L = sum(G * att) with the f64 forward; dL/dx by central differences at
    # sampled entries of q, k, v against the accumulating backward
    B, T, H, dh = 1, 7, 2, 32
    D = H * dh
    q, k, v = _qkv(B, T, D, 121, std=0.5)
    G = ob.normal((B * T, D), 125)
    _, pr = ob.attention_forward(q, k, v, B, T, H, dh)
    dq, dk, dv = ob.attention_backward(G, q, k, v, pr, B, T, H, dh)
    rng = np.random.default_rng(5)

    def loss(qq, kk, vv):
        a, _ = ob.attention_forward(qq, kk, vv, B, T, H, dh, f64=True)
        return float(np.sum(G.astype(np.float64) * a))

    eps = 1e-2
    for which, grad in ((0, dq), (1, dk), (2, dv)):
        for _ in range(6):
            r, c = int(rng.integers(B * T)), int(rng.integers(D))
            xs = [q.copy(), k.copy(), v.copy()]
            xs[which][r, c] += eps
            lp = loss(*xs)
            xs[which][r, c] -= 2 * eps
            lm = loss(*xs)
            num = (lp - lm) / (2 * eps)
            assert abs(num - grad[r, c]) < 2e-3 * max(1.0, abs(num)), (which, r, c, num, grad[r, c])


# ----------------------------------------------------------------- GELU ----
def test_gelu_oracle_vs_ref_train():
    tr = _ref_or_skip("libref_train.so")
    x = ob.normal((5000,), 131, 0.0, 2.0)
    g = ob.normal((5000,), 132)
    y_r, d_r = np.empty_like(x), np.empty_like(x)
    tr.pcl_ref_gelu_forward(p(y_r), p(x), x.size)
    tr.pcl_ref_gelu_backward(p(d_r), p(g), p(x), x.size)
    # -ffast-math reassociates the cubic and vectorises tanhf: in the tails
    # (x << 0, where 1 - t^2 cancels) single values differ by a few 1e-6
    # absolute; the normwise bar is the REF_TOL used for every other function
    assert ob.normwise_rel_err(ob.gelu(x), y_r) < REF_TOL
    assert ob.normwise_rel_err(ob.gelu_backward(g, x), d_r) < REF_TOL


def test_gelu_oracle_math():
    # the tanh form approximates x*Phi(x) (exact GELU) to ~1e-3; its derivative
    # matches central differences of the forward (in double)
    from math import erf, sqrt
    x = np.linspace(-6, 6, 1201).astype(np.float32)
    exact = np.array([0.5 * v * (1 + erf(v / sqrt(2))) for v in x.astype(np.float64)])
    assert np.max(np.abs(ob.gelu(x) - exact)) < 2e-3
    assert ob.gelu(np.zeros(3, np.float32)).tolist() == [0.0, 0.0, 0.0]
    k = 0.7978845608028654

    def g64(v):
        return 0.5 * v * (1 + np.tanh(k * (v + 0.044715 * v ** 3)))
    h = 1e-4
    num = (g64(x.astype(np.float64) + h) - g64(x.astype(np.float64) - h)) / (2 * h)
    np.testing.assert_allclose(ob.gelu_backward(np.ones_like(x), x), num, rtol=0, atol=2e-5)


# -------------------------------------------------------- CKP1 decode ----
@pytest.mark.parametrize("dims", [(32, 64, 4, 256, 2, 96), (24, 128, 4, 512, 3, 160)])
def test_decode_oracle_vs_ref_generate(tmp_path, dims):
    # generate.c (+ tokenizer.c) built from source reads the same checkpoint;
    # logits of a token sequence fed at positions 0.. must agree
    gen = _ref_or_skip("libref_generate.so")
    blk, d, h, df, nl, v = dims
    path = str(tmp_path / "m.ckp1")
    ob.write_ckp1(path, blk, d, h, df, nl, v, seed=3)
    assert gen.pcl_ref_gen_load(path.encode()) == v
    om = ob.OracleModel(path)
    assert om.hdr[:7] == [0x434B5031, blk, d, h, df, nl, v]
    toks = [int(t) % v for t in ob.u8((blk,), 5)]
    ref = np.empty(v, np.float32)
    for pos in range(blk):
        got = om.forward(toks[pos], pos)
        gen.pcl_ref_gen_forward(toks[pos], pos, p(ref))
        assert ob.normwise_rel_err(got, ref) < REF_TOL, pos
    om.close()


def test_decode_oracle_first_token_closed_form(tmp_path):
    # at position 0 the attention output is v itself: with identity-free random
    # weights the logits must equal a direct numpy evaluation of the block
    blk, d, h, df, nl, v = 4, 64, 4, 128, 1, 32
    path = str(tmp_path / "m.ckp1")
    ob.write_ckp1(path, blk, d, h, df, nl, v, seed=9)
    raw = np.fromfile(path, dtype="<f4")[8:].astype(np.float64)
    at = 0

    def take(n, shape=None):
        nonlocal at
        a = raw[at: at + n]
        at += n
        return a.reshape(shape) if shape else a
    wte, wpe = take(v * d, (v, d)), take(blk * d, (blk, d))
    g1, b1 = take(d), take(d)
    Wq, bq, Wk, bk, Wv, bv = take(d * d, (d, d)), take(d), take(d * d, (d, d)), take(d), take(d * d, (d, d)), take(d)
    Wo, bo, g2, b2 = take(d * d, (d, d)), take(d), take(d), take(d)
    W1, bf1, W2, bf2 = take(d * df, (d, df)), take(df), take(df * d, (df, d)), take(d)
    gf, bfin = take(d), take(d)

    def ln(x, g, b):
        mu = x.mean()
        return (x - mu) / np.sqrt(((x - mu) ** 2).mean() + 1e-5) * g + b
    tok = 7
    x = wte[tok] + wpe[0]
    att = ln(x, g1, b1) @ Wv + bv  # softmax over one key is 1
    x = x + att @ Wo + bo
    u = ln(x, g2, b2) @ W1 + bf1
    x = x + (0.5 * u * (1 + np.tanh(0.7978845608028654 * (u + 0.044715 * u ** 3)))) @ W2 + bf2
    want = wte @ ln(x, gf, bfin)
    om = ob.OracleModel(path)
    assert ob.normwise_rel_err(om.forward(tok, 0), want) < 1e-5
    om.close()


@pytest.mark.parametrize("dims", [(32, 64, 4, 256, 2, 96), (24, 128, 4, 512, 3, 160)])
def test_decode_oracle_int8_near_ref_generate(tmp_path, dims):
    # the INT8-product step differs from generate.c (built from source) by the
    # quantisation error only: per-column weight and per-token activation
    # scales of amax/127 keep the logits within a few per cent normwise (1.5-3.2%
    # measured here); a dropped bias or a wrong scale is far outside that
    gen = _ref_or_skip("libref_generate.so")
    blk, d, h, df, nl, v = dims
    path = str(tmp_path / "m.ckp1")
    ob.write_ckp1(path, blk, d, h, df, nl, v, seed=4, wstd=0.05)
    assert gen.pcl_ref_gen_load(path.encode()) == v
    om = ob.OracleModel(path, int8=True)
    toks = [int(t) % v for t in ob.u8((blk,), 6)]
    ref = np.empty(v, np.float32)
    errs = []
    for pos in range(blk):
        got = om.forward(toks[pos], pos)
        gen.pcl_ref_gen_forward(toks[pos], pos, p(ref))
        errs.append(ob.normwise_rel_err(got, ref))
    om.close()
    assert 1e-3 < max(errs) < 5e-2, errs


# the small model, the grown model (16 layers, d 512, d_ff 2048, vocab 2048),
# 8448-wide d_ff rows
INT8_WALK_DIMS = [((32, 64, 4, 256, 2, 96), 12), ((256, 512, 16, 2048, 16, 2048), 3),
                  ((16, 64, 4, 8448, 2, 96), 4)]


@pytest.mark.parametrize("dims,npos", INT8_WALK_DIMS)
def test_int8_step_walk_is_the_oracle_step(tmp_path, dims, npos):
    # the op-by-op walk that checks the GPU's INT8 step, run on its own values,
    # gives orc_model_forward_int8's logits bit for bit at every position: the
    # same QKV column join, bias placement, residual order, cached attention,
    # GELU input and head
    from int8_steps import Int8StepChecker
    blk, d, h, df, nl, v = dims
    path = str(tmp_path / "m.ckp1")
    ob.write_ckp1(path, blk, d, h, df, nl, v, seed=51, wstd=0.05)
    chk = Int8StepChecker(path)
    om = ob.OracleModel(path, int8=True)
    toks = [int(t) % v for t in ob.u8((npos,), 53)]
    try:
        for pos in range(npos):
            np.testing.assert_array_equal(chk.step(toks[pos], pos), om.forward(toks[pos], pos))
    finally:
        chk.close()
        om.close()


def test_int8_step_walk_catches_planted_mistakes(tmp_path):
    # the walk's own record, fed back as the source, passes with no byte
    # difference; each planted mistake in it (a bias dropped from a residual,
    # an attention value off by 1e-4 relative, a quantised byte off by one away
    # from any rounding boundary, a scale off by 1e-4, a product off by one
    # ulp, a d_ff row not the FF1 output) fails
    from int8_steps import Int8StepChecker
    blk, d, h, df, nl, v = 8, 64, 4, 256, 2, 96
    path = str(tmp_path / "m.ckp1")
    ob.write_ckp1(path, blk, d, h, df, nl, v, seed=57, wstd=0.05)
    src = Int8StepChecker(path)
    src.step(5, 0)
    rec = src.record
    src.close()

    def run(plant=None):
        r = {k: [np.array(a, copy=True) for a in vals] for k, vals in rec.items()}
        if plant:
            plant(r)
        chk = Int8StepChecker(path)
        try:
            chk.step(5, 0, source=lambda l, pr: tuple(r[(l, pr)]))
            return chk.flips
        finally:
            chk.close()

    assert run() == 0
    lw = ob.read_ckp1(path)["layers"]

    def drop_bias(r):
        r[(1, 0)][0] -= lw[0]["bff2"]

    def att_off(r):
        a = r[(1, 1)][0]
        a[np.argmax(np.abs(a))] *= np.float32(1 + 1e-4)

    def byte_off(r):
        xf = r[(0, 1)][0]
        q, sa = ob.quantize_row(xf, 256)
        t = np.abs(xf / sa[0])
        k = int(np.flatnonzero(np.abs(t - np.round(t)) < 0.25)[0])  # far from a boundary
        r[(0, 1)][1][k] = np.uint8(int(r[(0, 1)][1][k]) + (1 if r[(0, 1)][1][k] < 255 else -1))

    def scale_off(r):
        r[(1, 2)][2] *= np.float32(1 + 1e-4)

    def ulp_off(r):
        y = r[(0, 3)][3]
        y[7] = np.nextafter(y[7], np.float32(np.inf))

    def ff_row(r):
        r[(1, 3)][0][0] += np.float32(1e-3)

    for plant in (drop_bias, att_off, byte_off, scale_off, ulp_off, ff_row):
        with pytest.raises(AssertionError):
            run(plant)



# -------------------------------------------------- cross-entropy ----
def _ce_inputs(M, V, seed, scale=3.0):
    lg = ob.normal((M, V), seed, 0.0, scale)
    t = (ob.u8((M,), seed + 1).astype(np.int64) * 7919 % V).astype(np.int32)
    return lg, t


def test_cross_entropy_vs_ref_train():
    tr = _ref_or_skip("libref_train.so")
    V = tr.pcl_ref_train_vocab()
    for M, seed in ((1, 900), (37, 901), (128, 902)):
        lg, t = _ce_inputs(M, V, seed)
        t[0] = V - 1
        dl_ref = np.empty_like(lg)
        loss_ref = tr.pcl_ref_cross_entropy(p(lg), p(t), p(dl_ref), M)
        loss, dl = ob.cross_entropy(lg, t)
        assert loss == pytest.approx(loss_ref, rel=1e-6)
        assert ob.normwise_rel_err(dl, dl_ref) < REF_TOL


def test_cross_entropy_closed_forms():
    M, V = 5, 1000
    t = np.array([0, 999, 3, 500, 3], np.int32)
    # uniform logits: loss log V, dl = (1/V - onehot)/M
    loss, dl = ob.cross_entropy(np.full((M, V), 2.5, np.float32), t)
    assert loss == pytest.approx(np.log(V), rel=1e-6)
    want = np.full((M, V), 1.0 / V, np.float64)
    want[np.arange(M), t] -= 1.0
    np.testing.assert_allclose(dl, want / M, rtol=0, atol=1e-8)
    # random rows: loss against an f64 log-sum-exp, rows of dl sum to zero, a
    # constant added to a row changes nothing
    lg, t = _ce_inputs(64, 4096, 910, 4.0)
    loss, dl = ob.cross_entropy(lg, t)
    x = lg.astype(np.float64)
    lse = np.log(np.exp(x - x.max(1, keepdims=True)).sum(1)) + x.max(1)
    assert loss == pytest.approx(np.mean(lse - x[np.arange(64), t]), rel=1e-5)
    assert np.abs(dl.astype(np.float64).sum(1)).max() < 1e-6  # vs entries of 1/M = 1.6e-2
    p64 = np.exp(x - lse[:, None])
    p64[np.arange(64), t] -= 1.0
    assert ob.normwise_rel_err(dl, p64 / 64) < 1e-5
    loss2, dl2 = ob.cross_entropy(lg + np.float32(8.0), t)
    assert loss2 == pytest.approx(loss, rel=1e-5)
    assert ob.normwise_rel_err(dl2, dl) < 1e-5


def test_head_ce_central_differences():
    # d_lnf and dwte are the gradients of the mean loss: compare with central
    # differences of an f64 restatement on a tiny problem
    M, D, V = 3, 8, 11
    x = ob.normal((M, D), 920, 0.0, 1.0)
    w = ob.normal((V, D), 921, 0.0, 0.5)
    t = np.array([2, 10, 0], np.int32)

    def f64_loss(xx, ww):
        lg = xx @ ww.T
        mx = lg.max(1, keepdims=True)
        lse = np.log(np.exp(lg - mx).sum(1)) + mx[:, 0]
        return np.mean(lse - lg[np.arange(M), t])
    loss, dx, dw = ob.head_ce(x, w, t)
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    assert loss == pytest.approx(f64_loss(x64, w64), rel=1e-6)
    h = 1e-5
    num_dx = np.zeros((M, D))
    for i in range(M):
        for j in range(D):
            a, b = x64.copy(), x64.copy()
            a[i, j] += h
            b[i, j] -= h
            num_dx[i, j] = (f64_loss(a, w64) - f64_loss(b, w64)) / (2 * h)
    num_dw = np.zeros((V, D))
    for i in range(V):
        for j in range(D):
            a, b = w64.copy(), w64.copy()
            a[i, j] += h
            b[i, j] -= h
            num_dw[i, j] = (f64_loss(x64, a) - f64_loss(x64, b)) / (2 * h)
    # the tied weight's gradient through the head only (the embedding path is
    # outside this function)
    np.testing.assert_allclose(dx, num_dx, rtol=0, atol=2e-6)
    np.testing.assert_allclose(dw, num_dw, rtol=0, atol=2e-6)
    # dwte accumulates
    _, _, dw2 = ob.head_ce(x, w, t, dwte=dw)
    np.testing.assert_allclose(dw2, 2 * dw, rtol=1e-6, atol=1e-9)
