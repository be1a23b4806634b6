"""Op-by-op check of one INT8 decode step (imported by test_gpu_model.py and
test_oracle.py).

Int8StepChecker walks generate.c's forward (:118-183) with INT8 products as
the oracle's INT8 step does (orc_model_forward_int8): per layer LayerNorm ->
QKV product (+ bq|bk|bv) -> cached attention -> O product (+ bo) added to x ->
LayerNorm -> FF1 product (+ bff1) -> GELU -> FF2 product (+ bff2) added to x;
final LayerNorm and the tied-head product. Every value comes from the oracle's
own functions (layernorm_row, quantize_row, gemm_u8s8_i32, dequant, gelu,
decode_attention) and its quantised weights.

With a capture source (the GPU's tap: per product the input row, quantised
row, scale and dequantised output it used), each op is checked against the
oracle's op applied to the GPU's own inputs, so no error carries over from one
op to the next:
  - the input row equals the oracle's value of it (the embedding exactly; a
    residual add to within two roundings of its terms; the attention row to
    ATT_TOL normwise; the d_ff row exactly, being the FF1 output);
  - the quantised row equals the oracle's quantisation of the oracle transform
    (LayerNorm / bias + GELU) of the GPU's input, except bytes one step apart
    whose value lies within BOUNDARY of a rounding boundary (the two
    transforms differ only by fp32 rounding); the scale to SCALE_TOL;
  - the product equals, bit for bit, the oracle's exact integer GEMV of the
    GPU's quantised row times the oracle's quantised weights, dequantised with
    the GPU's scale (float(v) * (sa * sb[n])).
Without a source (source=None) the checker's own values are used at every op
(and kept in .record in the source's form) and the step returns the oracle's
INT8 logits; that mode is held bit-exact to orc_model_forward_int8 on the CPU,
which pins the walk itself.
"""
import numpy as np

import binding as ob

ATT_TOL = 1e-5      # normwise, fp32 softmax and sums in another order
SCALE_TOL = 1e-5    # relative, the row maximum after another rounding of its transform
BOUNDARY = 2e-3     # quantiser units from a .5 boundary for a one-step byte difference
EPS32 = 2.0 ** -23


def kpad256(k):
    return (k + 255) // 256 * 256


class Int8StepChecker:
    def __init__(self, path):
        self.P = ob.read_ckp1(path)
        hdr = self.P["hdr"]
        self.blk, self.D, self.H, self.F, self.L, self.V = hdr[1:7]
        self.om = ob.OracleModel(path, int8=True)
        self.W = []
        for l in range(self.L):
            q = [self.om.int8_weights(l, i) for i in range(6)]
            qkv = (np.ascontiguousarray(np.concatenate([q[0][0], q[1][0], q[2][0]], axis=1)),
                   np.concatenate([q[0][1], q[1][1], q[2][1]]))
            self.W.append([qkv, q[3], q[4], q[5]])
        self.head = self.om.int8_weights(self.L, 0)
        self.kc = np.zeros((self.L, self.blk, self.D), np.float32)
        self.vc = np.zeros((self.L, self.blk, self.D), np.float32)
        self.flips = 0       # one-step byte differences at a rounding boundary
        self.values = 0      # quantised values compared
        self.att_err = 0.0   # worst attention-row error seen
        self._cap = None
        self._source = None
        self.record = {}

    def close(self):
        self.om.close()

    # ------------------------------------------------------------------
    def _input(self, l, prod, want, mode, mag=None):
        """The product's input row: the GPU's (checked against want) or want."""
        if self._source is None:
            self.record[(l, prod)] = [want]
            return want
        self._cap = self._source(l, prod)
        got = self._cap[0]
        where = f"layer {l} product {prod}"
        if mode == "exact":
            np.testing.assert_array_equal(got, want, err_msg=where)
        elif mode == "att":
            e = ob.normwise_rel_err(got, want)
            self.att_err = max(self.att_err, e)
            assert e <= ATT_TOL, (where, e)
        else:  # residual add: two roundings of terms of size mag
            bad = np.abs(got.astype(np.float64) - want) > 2 * EPS32 * mag
            assert not bad.any(), (where, np.flatnonzero(bad)[:8])
        return got

    def _product(self, l, prod, xf, Bq, sb):
        """Quantise the transformed row xf, multiply: the GPU's product,
        checked, or the oracle's."""
        K = xf.size
        Kp = kpad256(K)
        q_want, sa_want = ob.quantize_row(xf, Kp)
        if self._source is None:
            xq, sa = q_want, sa_want
        else:
            _, xq, sa, y_got = self._cap
            where = f"layer {l} product {prod}"
            assert abs(float(sa[0]) / float(sa_want[0]) - 1.0) <= SCALE_TOL, (where, sa, sa_want)
            d = xq.astype(np.int32) - q_want.astype(np.int32)
            assert (xq[K:] == 128).all(), where
            assert np.abs(d).max() <= 1, (where, np.abs(d).max())
            k = np.flatnonzero(d)
            if k.size:
                t = np.abs(xf[k].astype(np.float64) / float(sa_want[0]))
                off = np.abs(t - np.floor(t) - 0.5)
                assert (off <= BOUNDARY).all(), (where, k[off > BOUNDARY][:8], off.max())
            self.flips += int(k.size)
            self.values += K
        v = ob.gemm_u8s8_i32(xq[None, :K], Bq)
        y = ob.dequant(v, np.asarray(sa, np.float32), sb)[0]
        if self._source is not None:
            np.testing.assert_array_equal(y_got, y, err_msg=f"layer {l} product {prod}")
        else:
            self.record[(l, prod)] += [xq, sa, y]
        return y

    # ------------------------------------------------------------------
    def step(self, tok, pos, source=None):
        """One position; source(l, prod) -> (xin, xq, sa, y) of the GPU, or
        None for the oracle's own values. Returns the head product (logits)."""
        self._source = source
        self.record = {}
        P, D, H = self.P, self.D, self.H
        x_want = P["wte"][tok] + P["wpe"][pos]
        x = self._input(0, 0, x_want, "exact")
        for l in range(self.L):
            lw, W = P["layers"][l], self.W[l]
            if l > 0:
                x = self._input(l, 0, x_want, "resid", mag)
            y = self._product(l, 0, ob.layernorm_row(x, lw["g1"], lw["b1"]), *W[0])
            qkv = y + np.concatenate([lw["bq"], lw["bk"], lw["bv"]])
            self.kc[l, pos], self.vc[l, pos] = qkv[D:2 * D], qkv[2 * D:]
            att = ob.decode_attention(qkv[:D], self.kc[l, :pos + 1], self.vc[l, :pos + 1], H, D // H)
            att = self._input(l, 1, att, "att")
            y = self._product(l, 1, att, *W[1])
            x_want = x + (y + lw["bo"])
            mag = np.abs(x) + np.abs(y) + np.abs(lw["bo"])
            x = self._input(l, 2, x_want, "resid", mag)
            h = self._product(l, 2, ob.layernorm_row(x, lw["g2"], lw["b2"]), *W[2])
            h = self._input(l, 3, h, "exact")
            y = self._product(l, 3, ob.gelu(h + lw["bff1"]), *W[3])
            x_want = x + (y + lw["bff2"])
            mag = np.abs(x) + np.abs(y) + np.abs(lw["bff2"])
        x = self._input(self.L, 0, x_want, "resid", mag)
        logits = self._product(self.L, 0, ob.layernorm_row(x, P["gf"], P["bf"]), *self.head)
        self._source = None
        return logits
