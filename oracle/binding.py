"""ctypes binding of the CPU checker libraries. TEST INFRASTRUCTURE ONLY.

Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg:
  oracle/liboracle.so          this repository's C restatement (pcl_oracle.h)
  oracle/_ref/libref_*.so      the reference's own sources built in place by
                               oracle/Makefile (optional: absent when the
                               reference tree was not available at build time)
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_PATH = os.path.join(HERE, "liboracle.so")
REF_DIR = os.path.join(HERE, "_ref")

_vp, _i, _f, _d, _l, _u32 = C.c_void_p, C.c_int, C.c_float, C.c_double, C.c_long, C.c_uint32
_sz = C.c_size_t

_ORACLE_PROTOS = {
    "orc_xorshift32": (_u32, [C.POINTER(_u32)]),
    "orc_fill_frand": (None, [_vp, _sz, _u32, _f]),
    "orc_fill_uniform": (None, [_vp, _sz, _u32, _f, _f]),
    "orc_fill_normal": (None, [_vp, _sz, _u32, _f, _f]),
    "orc_fill_u8": (None, [_vp, _sz, _u32]),
    "orc_fill_s8": (None, [_vp, _sz, _u32]),
    "orc_fill_kat_tensor": (None, [_vp, _sz, _vp, _sz]),
    "orc_matmul_ikj": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "orc_matmul_naive": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "orc_gemm_f64": (None, [_vp, _l, _l, _vp, _l, _l, _vp, _vp, _l, _i, _i, _i, _i]),
    "orc_gemm_nn": (None, [_vp, _vp, _vp, _vp, _i, _i, _i]),
    "orc_gemm_nt": (None, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "orc_gemm_tn": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "orc_bias_bwd": (None, [_vp, _vp, _i, _i]),
    "orc_matmul_forward": (None, [_vp, _vp, _vp, _vp, _i, _i, _i]),
    "orc_matmul_backward": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i]),
    "orc_tied_head_forward": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "orc_tied_head_backward": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i]),
    "orc_lm_head": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "orc_matvec": (None, [_vp, _vp, _vp, _vp, _i, _i, _i]),
    "orc_quantize_A": (_f, [_vp, _vp, _i, _i, _i]),
    "orc_quantize_A_rows": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "orc_quantize_B_pack": (None, [_vp, _vp, _vp, _vp, _i, _i, _i]),
    "orc_quantize_B_cols": (None, [_vp, _vp, _vp, _i, _i]),
    "orc_unpack_vnni": (None, [_vp, _vp, _i, _i, _i]),
    "orc_gemm_u8s8_i32": (_l, [_vp, _i, _vp, _i, _vp, _i, _i, _i, _i]),
    "orc_gemm_u8s8_raw_i32": (_l, [_vp, _i, _vp, _i, _vp, _i, _i, _i, _i]),
    "orc_gemm_int8_kernel": (None, [_vp, _i, _vp, _vp, _vp, _vp, _i, _i]),
    "orc_dequant": (None, [_vp, _i, _vp, _vp, _vp, _i, _i, _i]),
    "orc_gelu_forward": (None, [_vp, _vp, _l]),
    "orc_gelu_backward": (None, [_vp, _vp, _vp, _l]),
    "orc_attention_forward": (None, [_vp, _vp, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i]),
    "orc_attention_backward": (None, [_vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i]),
    "orc_attention_forward_f64": (None, [_vp, _vp, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i]),
    "orc_cross_entropy": (_f, [_vp, _i, _vp, _vp, _i, _i, _i]),
    "orc_head_ce": (_f, [_vp, _vp, _vp, _i, _i, _i, _vp, _vp]),
    "orc_model_load": (_vp, [C.c_char_p]),
    "orc_model_header": (None, [_vp, _vp]),
    "orc_model_forward": (None, [_vp, _i, _i, _vp]),
    "orc_model_forward_int8": (None, [_vp, _i, _i, _vp]),
    "orc_model_free": (None, [_vp]),
    "orc_layernorm_row": (None, [_vp, _vp, _vp, _vp, _i]),
    "orc_decode_attention": (None, [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp]),
    "orc_model_int8_weights": (_i, [_vp, _i, _i, _vp, _vp]),
    "orc_rms_rel": (_d, [_vp, _vp, _l]),
    "orc_max_abs_diff": (_d, [_vp, _vp, _l]),
}

_REF_PROTOS = {
    "libref_gemm_bench.so": {
        "pcl_ref_cpu_ok": (_i, []),
        "pcl_ref_set_threads": (None, [_i]),
        "pcl_ref_max_threads": (_i, []),
        "pcl_ref_gemm_naive": (None, [_vp, _vp, _vp, _i, _i, _i]),
        "pcl_ref_gemm_ikj": (None, [_vp, _vp, _vp, _i, _i, _i]),
        "pcl_ref_gemm_micro": (None, [_vp, _vp, _vp, _i, _i, _i]),
        "pcl_ref_gemm_packed": (None, [_vp, _vp, _vp, _i, _i, _i]),
        "pcl_ref_gemm_packed_mt": (None, [_vp, _vp, _vp, _i, _i, _i]),
        "pcl_ref_quantize_A": (_f, [_vp, _vp, _i, _i, _i]),
        "pcl_ref_quantize_B_pack": (None, [_vp, _vp, _vp, _vp, _i, _i, _i]),
        "pcl_ref_gemm_int8_kernel": (None, [_vp, _i, _vp, _vp, _vp, _vp, _i, _i]),
        "pcl_ref_gemm_int8_mt": (None, [_i, _vp, _i, _vp, _vp, _vp, _vp, _i, _i]),
        "pcl_ref_peak_gflops": (_d, []),
        "pcl_ref_peak_int8_gops": (_d, []),
        "pcl_ref_bandwidth_gbs": (_d, []),
        "pcl_ref_rms_rel": (_d, [_vp, _vp, _l]),
        "pcl_ref_max_abs_diff": (_d, [_vp, _vp, _l]),
        "pcl_ref_srand": (None, [C.c_uint]),
        "pcl_ref_fill_rand": (None, [_vp, _l]),
    },
    "libref_train.so": {
        "pcl_ref_train_d_model": (_i, []),
        "pcl_ref_train_vocab": (_i, []),
        "pcl_ref_matmul_forward": (None, [_vp, _vp, _vp, _vp, _i, _i, _i]),
        "pcl_ref_matmul_backward": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i]),
        "pcl_ref_tied_head_forward": (None, [_vp, _vp, _vp, _i]),
        "pcl_ref_tied_head_backward": (None, [_vp, _vp, _vp, _vp, _vp, _i]),
        "pcl_ref_train_n_heads": (_i, []),
        "pcl_ref_cross_entropy": (_f, [_vp, _vp, _vp, _i]),
        "pcl_ref_train_t_size": (_i, []),
        "pcl_ref_attention_forward": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
        "pcl_ref_attention_backward": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i]),
        "pcl_ref_gelu_forward": (None, [_vp, _vp, _i]),
        "pcl_ref_gelu_backward": (None, [_vp, _vp, _vp, _i]),
    },
    "libref_train_h64.so": {
        "pcl_ref_train_d_model": (_i, []),
        "pcl_ref_train_n_heads": (_i, []),
        "pcl_ref_train_t_size": (_i, []),
        "pcl_ref_attention_forward": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
        "pcl_ref_attention_backward": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i]),
    },
    "libref_generate.so": {
        "pcl_ref_gen_load": (_i, [C.c_char_p]),
        "pcl_ref_gen_forward": (None, [_i, _i, _vp]),
    },
    "libref_model.so": {
        "pcl_ref_model_d_model": (_i, []),
        "pcl_ref_proj_token": (None, [_vp, _vp, _vp, _vp, _i, _i]),
        "lm_head": (None, [_vp, _vp, _vp, _i]),
        "matmul": (None, [_vp, _vp, _vp, _i, _i, _i]),
    },
}


def _declare(lib, protos):
    for name, (res, args) in protos.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_oracle = None


def oracle():
    """liboracle.so; raises if it has not been built."""
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_PATH):
            raise ImportError(f"{ORACLE_PATH} not built (make -C oracle)")
        _oracle = _declare(C.CDLL(ORACLE_PATH), _ORACLE_PROTOS)
    return _oracle


_refs: dict = {}


def ref(name: str):
    """oracle/_ref/<name> (the reference built from source), or None."""
    if name not in _refs:
        path = os.path.join(REF_DIR, name)
        _refs[name] = _declare(C.CDLL(path), _REF_PROTOS[name]) if os.path.exists(path) else None
    return _refs[name]


def p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ------------------------------------------------------------- inputs ----
def frand(shape, seed, scale=1.0):
    a = np.empty(shape, np.float32)
    oracle().orc_fill_frand(p(a), a.size, seed, scale)
    return a


def uniform(shape, seed, lo, hi):
    a = np.empty(shape, np.float32)
    oracle().orc_fill_uniform(p(a), a.size, seed, lo, hi)
    return a


def normal(shape, seed, mean=0.0, std=1.0):
    a = np.empty(shape, np.float32)
    oracle().orc_fill_normal(p(a), a.size, seed, mean, std)
    return a


def u8(shape, seed):
    a = np.empty(shape, np.uint8)
    oracle().orc_fill_u8(p(a), a.size, seed)
    return a


def s8(shape, seed):
    a = np.empty(shape, np.int8)
    oracle().orc_fill_s8(p(a), a.size, seed)
    return a


# ------------------------------------------------------------ wrappers ----
def matmul_ikj(A, B):
    M, K = A.shape
    N = B.shape[1]
    Cm = np.empty((M, N), np.float32)
    oracle().orc_matmul_ikj(p(A), p(B), p(Cm), M, K, N)
    return Cm


def gemm_f64(A, B, transA=False, transB=False, bias=None, C0=None):
    """(C0 or 0) + op(A).op(B) + bias, double accumulation, one rounding."""
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    if transA:
        K, M = A.shape
        sam, sak = 1, M
    else:
        M, K = A.shape
        sam, sak = K, 1
    if transB:
        N = B.shape[0]
        sbk, sbn = 1, K
    else:
        N = B.shape[1]
        sbk, sbn = N, 1
    Cm = np.zeros((M, N), np.float32) if C0 is None else np.array(C0, np.float32, copy=True)
    oracle().orc_gemm_f64(p(A), sam, sak, p(B), sbk, sbn, p(bias), p(Cm), N, M, N, K,
                          0 if C0 is None else 1)
    return Cm


def gemm_u8s8_i32(Au, Bq):
    """exact sum_k (Au-128)*Bq; Bq is K x N row-major."""
    Au = np.ascontiguousarray(Au)
    Bq = np.ascontiguousarray(Bq)
    M, K = Au.shape
    N = Bq.shape[1]
    Cm = np.empty((M, N), np.int32)
    bad = oracle().orc_gemm_u8s8_i32(p(Au), K, p(Bq), N, p(Cm), N, M, N, K)
    assert bad == 0, "int32 overflow in the oracle"
    return Cm


def dequant(V, sa, sb):
    M, N = V.shape
    out = np.empty((M, N), np.float32)
    oracle().orc_dequant(p(np.ascontiguousarray(V)), N, p(sa), p(sb), p(out), N, M, N)
    return out


def cross_entropy(logits, targets):
    """orc_cross_entropy (train.c:449-465): (mean loss, dlogits)."""
    lg = np.ascontiguousarray(logits, np.float32)
    t = np.ascontiguousarray(targets, np.int32)
    M, V = lg.shape
    dl = np.empty_like(lg)
    loss = oracle().orc_cross_entropy(p(lg), V, p(t), p(dl), V, M, V)
    return float(loss), dl


def head_ce(lnf, wte, targets, dwte=None):
    """orc_head_ce: (mean loss, d_lnf, dwte after accumulation into a copy of
    dwte, zeros when None)."""
    x = np.ascontiguousarray(lnf, np.float32)
    w = np.ascontiguousarray(wte, np.float32)
    t = np.ascontiguousarray(targets, np.int32)
    M, D = x.shape
    V = w.shape[0]
    dx = np.empty((M, D), np.float32)
    dw = np.zeros((V, D), np.float32) if dwte is None else np.array(dwte, np.float32, copy=True)
    loss = oracle().orc_head_ce(p(x), p(w), p(t), M, D, V, p(dx), p(dw))
    return float(loss), dx, dw


def gelu(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    oracle().orc_gelu_forward(p(out), p(x), x.size)
    return out


def gelu_backward(dout, x):
    x = np.ascontiguousarray(x, np.float32)
    dout = np.ascontiguousarray(dout, np.float32)
    din = np.empty_like(x)
    oracle().orc_gelu_backward(p(din), p(dout), p(x), x.size)
    return din


def layernorm_row(x, g, b):
    """orc_layernorm_row (generate.c:109-117) of one row."""
    x, g, b = (np.ascontiguousarray(a, np.float32) for a in (x, g, b))
    y = np.empty_like(x)
    oracle().orc_layernorm_row(p(x), p(g), p(b), p(y), x.size)
    return y


def quantize_row(x, Kp):
    """orc_quantize_A_rows over one row: (u8 bytes padded with 128 to Kp, scale)."""
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(Kp, np.uint8)
    sa = np.empty(1, np.float32)
    oracle().orc_quantize_A_rows(p(x), p(q), p(sa), 1, x.size, Kp)
    return q, sa


def decode_attention(q, kc, vc, H, dh):
    """orc_decode_attention (generate.c:130-152): one query row against cache
    rows 0..len(kc)-1."""
    q, kc, vc = (np.ascontiguousarray(a, np.float32) for a in (q, kc, vc))
    n, ld = kc.shape
    att = np.empty(ld, np.float32)
    sc = np.empty(n, np.float32)
    oracle().orc_decode_attention(p(q), p(kc), p(vc), ld, n - 1, H, dh, p(att), p(sc))
    return att


def read_ckp1(path):
    """The tensors of a CKP1 file (train.c:633-648 order) as float32 arrays:
    {"hdr", "wte", "wpe", "layers": [{g1 b1 Wq bq Wk bk Wv bv Wo bo g2 b2 W1
    bff1 W2 bff2}], "gf", "bf"}; matrices K x N as stored."""
    raw = np.fromfile(path, dtype="<f4")
    hdr = raw[:8].view("<i4").tolist()
    blk, d, _, df, nl, v = hdr[1:7]
    at = [8]

    def take(*shape):
        n = int(np.prod(shape))
        a = raw[at[0]:at[0] + n].reshape(shape).astype(np.float32)
        at[0] += n
        return a
    out = {"hdr": hdr, "wte": take(v, d), "wpe": take(blk, d), "layers": []}
    shapes = [("g1", (d,)), ("b1", (d,)), ("Wq", (d, d)), ("bq", (d,)), ("Wk", (d, d)), ("bk", (d,)),
              ("Wv", (d, d)), ("bv", (d,)), ("Wo", (d, d)), ("bo", (d,)), ("g2", (d,)), ("b2", (d,)),
              ("W1", (d, df)), ("bff1", (df,)), ("W2", (df, d)), ("bff2", (d,))]
    for _ in range(nl):
        out["layers"].append({k: take(*sh) for k, sh in shapes})
    out["gf"], out["bf"] = take(d), take(d)
    assert at[0] == raw.size, "CKP1 size does not match its header"
    return out


def attention_forward(q, k, v, B, T, H, dh, f64=False):
    """(att, probs) of the causal attention restatement; q/k/v (B*T) x ld."""
    q, k, v = (np.ascontiguousarray(x, np.float32) for x in (q, k, v))
    ld = q.shape[1]
    att = np.zeros((B * T, ld), np.float32)
    probs = np.empty((B * H, T, T), np.float32)
    fn = oracle().orc_attention_forward_f64 if f64 else oracle().orc_attention_forward
    fn(p(q), p(k), p(v), ld, p(att), ld, p(probs), B, T, H, dh)
    return att, probs


def attention_backward(d_att, q, k, v, probs, B, T, H, dh, dq=None, dk=None, dv=None):
    """(dq, dk, dv) accumulated onto the given arrays (zeros if None)."""
    q, k, v, d_att = (np.ascontiguousarray(x, np.float32) for x in (q, k, v, d_att))
    ld = q.shape[1]
    dq, dk, dv = (np.zeros_like(q) if a is None else np.array(a, np.float32, copy=True)
                  for a in (dq, dk, dv))
    oracle().orc_attention_backward(p(dq), p(dk), p(dv), p(d_att), d_att.shape[1], p(q), p(k),
                                    p(v), ld, p(np.ascontiguousarray(probs, np.float32)), B, T,
                                    H, dh)
    return dq, dk, dv


def write_ckp1(path, blk, d, h, df, nl, v, seed, step=0, wstd=0.02):
    """A CKP1 checkpoint (train.c:633-648 layout) with synthetic parameters:
    gains 1 + N(0, 0.1), biases N(0, 0.02), matrices N(0, wstd), embeddings N(0, 0.1)."""
    import struct
    sizes = []
    sizes.append(("emb", v * d))
    sizes.append(("emb", blk * d))
    for _ in range(nl):
        sizes += [("g", d), ("b", d), ("w", d * d), ("b", d), ("w", d * d), ("b", d), ("w", d * d), ("b", d),
                  ("w", d * d), ("b", d), ("g", d), ("b", d), ("w", d * df), ("b", df), ("w", df * d), ("b", d)]
    sizes += [("g", d), ("b", d)]
    with open(path, "wb") as f:
        f.write(struct.pack("<8i", 0x434B5031, blk, d, h, df, nl, v, step))
        for i, (kind, n) in enumerate(sizes):
            s = seed * 1000 + i + 1
            if kind == "g":
                a = normal((n,), s, 1.0, 0.1)
            elif kind == "b":
                a = normal((n,), s, 0.0, 0.02)
            elif kind == "w":
                a = normal((n,), s, 0.0, wstd)
            else:
                a = normal((n,), s, 0.0, 0.1)
            f.write(a.astype("<f4").tobytes())


class OracleModel:
    """orc_model_* (generate.c restated) over a CKP1 file; int8 selects the
    INT8-product step (orc_model_forward_int8)."""

    def __init__(self, path, int8=False):
        self.int8 = int8
        self.m = oracle().orc_model_load(path.encode())
        if not self.m:
            raise ValueError(f"{path}: not a CKP1 checkpoint")
        hdr = np.empty(8, np.int32)
        oracle().orc_model_header(self.m, p(hdr))
        self.hdr = hdr.tolist()

    def forward(self, tok, pos):
        out = np.empty(self.hdr[6], np.float32)
        fn = oracle().orc_model_forward_int8 if self.int8 else oracle().orc_model_forward
        fn(self.m, tok, pos, p(out))
        return out

    def int8_weights(self, layer, which):
        """The INT8 step's quantised operand (K x N int8) and per-column
        scales: which 0..5 = Wq Wk Wv Wo W1 W2; layer n_layers = the head."""
        d, df, v, nl = self.hdr[2], self.hdr[4], self.hdr[6], self.hdr[5]
        K, N = (d, v) if layer == nl else ((df, d) if which == 5 else (d, df if which == 4 else d))
        Bq = np.empty((K, N), np.int8)
        sb = np.empty(N, np.float32)
        got = oracle().orc_model_int8_weights(self.m, layer, which, p(Bq), p(sb))
        assert got == K * N, (layer, which)
        return Bq, sb

    def close(self):
        if self.m:
            oracle().orc_model_free(self.m)
            self.m = None


def normwise_rel_err(X, R):
    """max|X-R| / max|R| -- the FP32 parity metric (tolerance 1e-4)."""
    X = np.asarray(X, np.float64)
    R = np.asarray(R, np.float64)
    den = np.max(np.abs(R)) if R.size else 0.0
    num = np.max(np.abs(X - R)) if R.size else 0.0
    return 0.0 if num == 0 else num / max(den, 1e-30)
