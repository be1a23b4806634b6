"""INT8 parity on the GPU: u8 x s8 -> int32 must be bit-exact.

Checked against the exact int64 oracle, against golden outputs written by the
reference's own gemm_bench.c (tests/golden/gemm_bench_int8.npz), and at full
config sizes by exact integer checksums (column sums of C equal
colsum(A-128).B; row sums equal (A-128).rowsum(B)) plus exact sampled rows.
"""
import os

import numpy as np
import pytest

import binding as ob
import pcl
from gpu_util import announce, require_device

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")
p = ob.p


@pytest.fixture(scope="module", autouse=True)
def _device():
    require_device()


def pack(Bq):
    """Bq (K x N row-major s8) -> device packed buffer + colsum."""
    K, N = Bq.shape
    dB = pcl.dev(Bq)
    dBp = pcl.DeviceBuffer(pcl.lib.pcl_s8_packed_bytes(K, N))
    dcs = pcl.empty((N,), np.int32)
    pcl.check(pcl.lib.pcl_pack_b_s8(dB.ptr, N, K, N, dBp.ptr, dcs.ptr, None))
    pcl.sync()
    return dBp, dcs.download((N,), np.int32)


def igemm_i32(Au, Bq, gemv=False):
    M, K = Au.shape
    N = Bq.shape[1]
    dBp, _ = pack(Bq)
    dA = pcl.dev(Au)
    dC = pcl.empty((M, N), np.int32)
    fn = pcl.lib.pcl_gemv_u8s8_i32 if gemv else pcl.lib.pcl_gemm_u8s8_i32
    pcl.check(fn(dA.ptr, K, dBp.ptr, dC.ptr, N, M, N, K, None))
    pcl.sync()
    return dC.download((M, N), np.int32)


def exact(Au, Bq):
    return (Au.astype(np.int64) - 128) @ Bq.astype(np.int64)


def test_pack_layout_and_colsum():
    K, N = 200, 96
    Bq = ob.s8((K, N), 11)
    announce("pack_b_s8", K, N)
    dBp, cs = pack(Bq)
    Kp = pcl.lib.pcl_s8_kpad(K)
    got = dBp.download((N, Kp), np.int8)
    np.testing.assert_array_equal(got[:, :K], Bq.T)
    assert not got[:, K:].any()  # zero padding beyond K
    np.testing.assert_array_equal(cs, Bq.astype(np.int64).sum(0))


@pytest.mark.parametrize("M,N,K", [(17, 33, 80), (64, 64, 64), (256, 512, 256), (129, 257, 1000),
                                   (300, 200, 48), (9, 16, 4096), (1024, 1024, 1024)])
def test_igemm_i32_exact(M, N, K):
    Au = ob.u8((M, K), 20 + M)
    Bq = ob.s8((K, N), 21 + N)
    announce("igemm i32", M, N, K)
    np.testing.assert_array_equal(igemm_i32(Au, Bq), ob.gemm_u8s8_i32(Au, Bq))


def test_igemm_extremes():
    # all -128 x all -128 and 255 x 127: the largest magnitudes of the range
    M, N, K = 64, 64, 4096
    announce("igemm extremes")
    C = igemm_i32(np.zeros((M, K), np.uint8), np.full((K, N), -128, np.int8))
    assert (C == K * 128 * 128).all()
    C = igemm_i32(np.full((M, K), 255, np.uint8), np.full((K, N), 127, np.int8))
    assert (C == K * 127 * 127).all()
    C = igemm_i32(np.full((M, K), 128, np.uint8), ob.s8((K, N), 5))
    assert not C.any()


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
def test_igemv_i32_exact(M):
    for N, K in ((1536, 512), (512, 2048), (2048, 512), (100, 77), (64, 8192)):
        Au = ob.u8((M, K), 30 + M)
        Bq = ob.s8((K, N), 31 + N)
        announce("igemv i32", M, N, K)
        np.testing.assert_array_equal(igemm_i32(Au, Bq, gemv=True), ob.gemm_u8s8_i32(Au, Bq))


@pytest.mark.parametrize("M", [3, 4, 5, 8])
def test_igemv_wide_exact(M):
    # several activation rows against a wide N: the 350M head, a K that is a
    # multiple of 16 but not of 32, and a short K
    for N, K in ((50257, 1024), (9000, 1040), (8192, 256)):
        Au = ob.u8((M, K), 130 + M)
        Bq = ob.s8((K, N), 131 + N)
        announce("igemv wide i32", M, N, K)
        np.testing.assert_array_equal(igemm_i32(Au, Bq, gemv=True), ob.gemm_u8s8_i32(Au, Bq))


@pytest.mark.parametrize("M,N", [(8, 9000), (8, 9001), (3, 9001)])
def test_igemv_wide_dequant_bit_exact(M, N):
    # the matrix-core GEMV stores a lane's four adjacent outputs with one 16-byte
    # store; an odd N leaves every output row but the first misaligned
    K = 1024
    Au = ob.u8((M, K), 140)
    Bq = ob.s8((K, N), 141)
    sa = ob.uniform((M,), 142, 1e-3, 1e-2)
    sb = ob.uniform((N,), 143, 1e-3, 1e-2)
    off = ob.s8((N,), 144).astype(np.int32) * 1000
    V = exact(Au, Bq).astype(np.int32)
    announce("igemv wide dq", M, N, K)
    np.testing.assert_array_equal(_dq_run(Au, Bq, sa, sb), ob.dequant(V, sa, sb))
    np.testing.assert_array_equal(_dq_run(Au, Bq, None, sb), ob.dequant(V, None, sb))
    np.testing.assert_array_equal(_dq_run(Au, Bq, None, sb, off),
                                  ob.dequant((V + off).astype(np.int32), None, sb))


# (K, N) for one or two activation rows: rows of 1 to 33 packed segments of
# 256 bytes (K from 7 to 9000, whole and partial segments) against short,
# ragged N, every output form, column offsets
DOT_SHAPES = ((7, 129), (300, 63), (700, 33), (1000, 95), (1040, 17), (2048, 31), (2100, 9),
              (4096, 23), (4200, 5), (8192, 7), (9000, 70))


@pytest.mark.parametrize("M", [1, 2])
def test_igemv_dot_geometry(M):
    for K, N in DOT_SHAPES:
        Au = ob.u8((M, K), 150 + K)
        Bq = ob.s8((K, N), 151 + N)
        sa = ob.uniform((M,), 152, 1e-3, 1e-2)
        sb = ob.uniform((N,), 153, 1e-3, 1e-2)
        off = ob.s8((N,), 154).astype(np.int32) * 1000
        V = exact(Au, Bq).astype(np.int32)
        announce("igemv dot geometry", M, N, K)
        np.testing.assert_array_equal(igemm_i32(Au, Bq, gemv=True), V)
        np.testing.assert_array_equal(_dq_run(Au, Bq, sa, sb, off),
                                      ob.dequant((V + off).astype(np.int32), sa, sb))
        np.testing.assert_array_equal(_dq_run(Au, Bq, None, sb), ob.dequant(V, None, sb))


@pytest.mark.parametrize("M,K,ldx", [(3, 130, 144), (8, 2050, 2064), (5, 61, 64)])
def test_igemv_padded_rows(M, K, ldx):
    # 16-byte aligned activation rows whose K is not a multiple of 16: the
    # staging's vector loads stop at K (re-centred bytes past K stay zero)
    N = 100
    Ap = ob.u8((M, ldx), 35 + K)
    Bq = ob.s8((K, N), 36)
    dBp, _ = pack(Bq)
    dA, dC = pcl.dev(Ap), pcl.empty((M, N), np.int32)
    announce("igemv padded rows", M, K, ldx)
    pcl.check(pcl.lib.pcl_gemv_u8s8_i32(dA.ptr, ldx, dBp.ptr, dC.ptr, N, M, N, K, None))
    pcl.sync()
    np.testing.assert_array_equal(dC.download((M, N), np.int32), exact(Ap[:, :K], Bq).astype(np.int32))


def _dq_run(Au, Bq, sa, sb, col_off=None):
    M, K = Au.shape
    N = Bq.shape[1]
    dBp, _ = pack(Bq)
    dA = pcl.dev(Au)
    dsa = pcl.dev(sa) if sa is not None else None
    dsb = pcl.dev(sb)
    doff = pcl.dev(col_off) if col_off is not None else None
    dC = pcl.empty((M, N), np.float32)
    pcl.check(pcl.lib.pcl_gemm_u8s8_dq(dA.ptr, K, dBp.ptr, doff.ptr if doff else None,
                                       dsa.ptr if dsa else None, dsb.ptr, dC.ptr, N, M, N, K, None))
    pcl.sync()
    return dC.download((M, N), np.float32)


@pytest.mark.parametrize("M,N,K", [(2048, 2048, 2048), (4096, 3072, 1024), (4, 1536, 512), (200, 300, 96)])
def test_igemm_dequant_bit_exact(M, N, K):
    # gemm_bench INT8 config: per-row x per-column scales ~ U[1e-3, 1e-2]
    Au = ob.u8((M, K), 40)
    Bq = ob.s8((K, N), 41)
    sa = ob.uniform((M,), 42, 1e-3, 1e-2)
    sb = ob.uniform((N,), 43, 1e-3, 1e-2)
    rows = np.unique(np.r_[0, M - 1, np.random.default_rng(1).choice(M, min(M, 64), replace=False)])
    V = exact(Au[rows], Bq).astype(np.int32)
    announce("igemm dq rowcol", M, N, K)
    C = _dq_run(Au, Bq, sa, sb)
    np.testing.assert_array_equal(C[rows], ob.dequant(V, sa[rows], sb))
    announce("igemm dq col", M, N, K)
    C = _dq_run(Au, Bq, None, sb)
    np.testing.assert_array_equal(C[rows], ob.dequant(V, None, sb))
    off = ob.s8((N,), 44).astype(np.int32) * 1000
    announce("igemm dq col_off", M, N, K)
    C = _dq_run(Au, Bq, None, sb, off)
    np.testing.assert_array_equal(C[rows], ob.dequant((V + off).astype(np.int32), None, sb))


# BASELINE.json configs[2], INT8: the grown model's prefill GEMMs at T = 256
# (d_model 512, d_ff 2048): QKV, attention output, FFN up, FFN down, with
# per-token u8 activations and per-channel s8 weights, dequantised by
# sa[m] * sb[n] (transformer.c:123-158; gemm_bench.c:272-275). Every output
# is compared, int32 and dequantised, against the exact integer oracle.
GROWN_PREFILL = [("qkv", 256, 1536, 512), ("attn_out", 256, 512, 512), ("ffn_up", 256, 2048, 512),
                 ("ffn_down", 256, 512, 2048)]


@pytest.mark.parametrize("name,M,N,K", GROWN_PREFILL)
def test_igemm_grown_prefill_bit_exact(name, M, N, K):
    Au = ob.u8((M, K), 90 + K)
    Bq = ob.s8((K, N), 91 + N)
    sa = ob.uniform((M,), 92, 1e-3, 1e-2)
    sb = ob.uniform((N,), 93, 1e-3, 1e-2)
    V = ob.gemm_u8s8_i32(Au, Bq)
    announce("igemm grown prefill", name, M, N, K)
    np.testing.assert_array_equal(igemm_i32(Au, Bq), V)
    np.testing.assert_array_equal(_dq_run(Au, Bq, sa, sb), ob.dequant(V, sa, sb))


@pytest.mark.parametrize("M", [3, 40])
def test_int8_k0(M):
    # K == 0 reads no activation (NULL A): v = 0, so C = float(col_off) * dq
    N = 70
    sa = ob.uniform((M,), 45, 1e-3, 1e-2)
    sb = ob.uniform((N,), 46, 1e-3, 1e-2)
    off = ob.s8((N,), 47).astype(np.int32) * 1000
    dBp = pcl.DeviceBuffer(256)  # no packed bytes at K = 0
    dsa, dsb, doff = pcl.dev(sa), pcl.dev(sb), pcl.dev(off)
    dC = pcl.empty((M, N), np.float32)
    announce("int8 K=0", M)
    fn = pcl.lib.pcl_gemv_u8s8_dq if M <= 8 else pcl.lib.pcl_gemm_u8s8_dq
    pcl.check(fn(None, 0, dBp.ptr, doff.ptr, dsa.ptr, dsb.ptr, dC.ptr, N, M, N, 0, None))
    pcl.sync()
    want = ob.dequant(np.broadcast_to(off, (M, N)).astype(np.int32), sa, sb)
    np.testing.assert_array_equal(dC.download((M, N), np.float32), want)
    dI = pcl.empty((M, N), np.int32)
    fn = pcl.lib.pcl_gemv_u8s8_i32 if M <= 8 else pcl.lib.pcl_gemm_u8s8_i32
    pcl.check(fn(None, 0, dBp.ptr, dI.ptr, N, M, N, 0, None))
    pcl.sync()
    np.testing.assert_array_equal(dI.download((M, N), np.int32), np.zeros((M, N), np.int32))


@pytest.mark.parametrize("M,N,K", [(2048, 2048, 2048), (4096, 3072, 1024), (4096, 1024, 1024),
                                   (4096, 4096, 1024), (4096, 1024, 4096), (4096, 50257, 1024)])
def test_igemm_full_size_checksums(M, N, K):
    # size-independent exact properties at the configs' full sizes
    Au = ob.u8((M, K), 60 + K)
    Bq = ob.s8((K, N), 61 + N)
    announce("igemm full", M, N, K)
    C = igemm_i32(Au, Bq).astype(np.int64)
    A8 = Au.astype(np.int64) - 128
    B8 = Bq.astype(np.int64)
    np.testing.assert_array_equal(C.sum(0), A8.sum(0) @ B8)  # column checksums
    np.testing.assert_array_equal(C.sum(1), A8 @ B8.sum(1))  # row checksums
    rows = np.random.default_rng(2).choice(M, 8, replace=False)
    np.testing.assert_array_equal(C[rows], A8[rows] @ B8)


@pytest.mark.parametrize("M,N,K", [(2100, 4100, 256), (2100, 4100, 768), (4096, 2200, 1024)])
def test_igemm_persistent_multi_tile(M, N, K):
    # 128x128 grids of more tiles than CUs: each workgroup of the
    # producer/consumer kernel loops over several output tiles (the K-tile
    # stream crosses tile boundaries; K = 256 gives fewer K tiles per
    # workgroup than ring stages on the last round); ragged edges, per-row and
    # per-column scales and column offsets, int32 and dequantised outputs
    Au = ob.u8((M, K), 80 + K)
    Bq = ob.s8((K, N), 81)
    sa = ob.uniform((M,), 82, 1e-3, 1e-2)
    sb = ob.uniform((N,), 83, 1e-3, 1e-2)
    off = ob.s8((N,), 84).astype(np.int32) * 1000
    rows = np.unique(np.r_[0, 127, 128, M - 1, np.random.default_rng(4).choice(M, 24, replace=False)])
    V = exact(Au[rows], Bq).astype(np.int32)
    announce("igemm persistent", M, N, K)
    C = igemm_i32(Au, Bq)
    np.testing.assert_array_equal(C[rows], V)
    A8 = Au.astype(np.int64) - 128
    np.testing.assert_array_equal(C.astype(np.int64).sum(0), A8.sum(0) @ Bq.astype(np.int64))
    C = _dq_run(Au, Bq, sa, sb, off)
    np.testing.assert_array_equal(C[rows], ob.dequant((V + off).astype(np.int32), sa[rows], sb))


@pytest.mark.parametrize("N", [16400, 16384])
def test_igemm_dequant_output_beyond_256mib(N):
    # outputs past 256 MiB take the persistent producer/consumer kernels:
    # 128x128 row-class tiles at a pitch off 128-byte lines (16400 floats: two
    # classes), 256x128 tiles at a line-multiple pitch; every dequant operand
    # (per-row, per-column scales and column offsets) is staged through LDS
    M, K = 4096, 256
    Au = ob.u8((M, K), 70)
    Bq = ob.s8((K, N), 71)
    sa = ob.uniform((M,), 72, 1e-3, 1e-2)
    sb = ob.uniform((N,), 73, 1e-3, 1e-2)
    off = ob.s8((N,), 74).astype(np.int32) * 1000
    rows = np.unique(np.r_[0, 255, 256, M - 1, np.random.default_rng(3).choice(M, 24, replace=False)])
    V = exact(Au[rows], Bq).astype(np.int32)
    announce("igemm dq > 256 MiB", M, N, K)
    C = _dq_run(Au, Bq, sa, sb, off)
    np.testing.assert_array_equal(C[rows], ob.dequant((V + off).astype(np.int32), sa[rows], sb))
    del C
    C = _dq_run(Au, Bq, None, sb)
    np.testing.assert_array_equal(C[rows], ob.dequant(V, None, sb))


@pytest.mark.parametrize("M,N,K", [(2100, 2070, 1040), (4100, 3100, 528), (4000, 3000, 528), (2056, 2048, 2064)])
def test_igemm_ragged_large_tiles(M, N, K):
    # ragged M, N and K (K % 128 != 0) on the 128x128 (two K groups),
    # 256x256 and 256x192 (4000 x 3000) tile paths; float64 products of these integers are exact
    # (every partial sum stays far below 2**53)
    Au = ob.u8((M, K), 80 + M)
    Bq = ob.s8((K, N), 81 + N)
    announce("igemm ragged large", M, N, K)
    C = igemm_i32(Au, Bq)
    ref = (Au.astype(np.float64) - 128) @ Bq.astype(np.float64)
    np.testing.assert_array_equal(C, ref.astype(np.int64))


def _exact_f64(Au, Bq):
    # float64 products of these integers are exact (every partial sum stays
    # far below 2**53), so BLAS gives the whole int32 result
    return ((Au.astype(np.float64) - 128) @ Bq.astype(np.float64)).astype(np.int64)


def test_igemm_headline_full_compare():
    # BASELINE.json configs[1] (gemm_bench INT8, M = N = K = 2048): every
    # output compared, int32 and dequantised (per-row x per-column scales ~
    # U[1e-3, 1e-2], gemm_bench.c:272-275), not only sampled rows
    M = N = K = 2048
    Au = ob.u8((M, K), 100)
    Bq = ob.s8((K, N), 101)
    sa = ob.uniform((M,), 102, 1e-3, 1e-2)
    sb = ob.uniform((N,), 103, 1e-3, 1e-2)
    announce("igemm headline full", M, N, K)
    V = _exact_f64(Au, Bq)
    np.testing.assert_array_equal(igemm_i32(Au, Bq), V)
    np.testing.assert_array_equal(_dq_run(Au, Bq, sa, sb), ob.dequant(V.astype(np.int32), sa, sb))


# One round of 128x128 tiles (256 tiles on 256 CUs) runs the K-grouped
# 16x16x64 kernel: one K group below K = 4096, two from there on. Exact and
# ragged extents in M, N and K (K padded to 256 by the host entry point),
# every output compared, int32 and dequantised with per-row and per-column
# scales and column offsets.
@pytest.mark.parametrize("M,N,K", [(4096, 1024, 1024), (2000, 2040, 2064), (4096, 1024, 4096),
                                   (4000, 1000, 4100), (2040, 1985, 8192)])
def test_igemm_one_round_tiles_full_compare(M, N, K):
    Au = ob.u8((M, K), 110 + K % 97)
    Bq = ob.s8((K, N), 111 + N % 89)
    sa = ob.uniform((M,), 112, 1e-3, 1e-2)
    sb = ob.uniform((N,), 113, 1e-3, 1e-2)
    off = ob.s8((N,), 114).astype(np.int32) * 1000
    announce("igemm one round", M, N, K)
    V = _exact_f64(Au, Bq)
    np.testing.assert_array_equal(igemm_i32(Au, Bq), V)
    V32 = V.astype(np.int32)
    np.testing.assert_array_equal(_dq_run(Au, Bq, sa, sb, off), ob.dequant((V32 + off).astype(np.int32), sa, sb))
    np.testing.assert_array_equal(_dq_run(Au, Bq, None, sb), ob.dequant(V32, None, sb))


def _run_pitched(Au, Bq, ldc, shift, sa=None, sb=None, col_off=None):
    """C (M x N) written at pitch ldc, starting `shift` elements into its
    buffer; int32 when sb is None, else dequantised. Returns the M x N view."""
    M, K = Au.shape
    N = Bq.shape[1]
    dBp, _ = pack(Bq)
    dA = pcl.dev(Au)
    total = (M - 1) * ldc + N + shift
    dC = pcl.DeviceBuffer(4 * total)
    pcl.check(pcl.lib.pcl_memset(dC.ptr, 0xFF, 4 * total))
    cptr = dC.ptr + 4 * shift
    if sb is None:
        pcl.check(pcl.lib.pcl_gemm_u8s8_i32(dA.ptr, K, dBp.ptr, cptr, ldc, M, N, K, None))
        dt = np.int32
    else:
        dsa = pcl.dev(sa) if sa is not None else None
        dsb = pcl.dev(sb)
        doff = pcl.dev(col_off) if col_off is not None else None
        pcl.check(pcl.lib.pcl_gemm_u8s8_dq(dA.ptr, K, dBp.ptr, doff.ptr if doff else None,
                                           dsa.ptr if dsa else None, dsb.ptr, cptr, ldc, M, N, K, None))
        dt = np.float32
    pcl.sync()
    flat = dC.download((total,), dt)
    out = np.lib.stride_tricks.as_strided(flat[shift:], (M, N), (4 * ldc, 4)).copy()
    # nothing written between the rows
    gaps = np.lib.stride_tricks.as_strided(flat[shift + N:], (M - 1, ldc - N), (4 * ldc, 4)) if ldc > N else None
    if gaps is not None:
        assert (gaps.view(np.uint32) == 0xFFFFFFFF).all()
    return out


# Outputs whose rows start off 128-byte lines (odd pitch: 32 row classes;
# pitch = 2 mod 4: 16; a line-multiple pitch from a base 4 bytes into a
# line: one shifted class) take row-class tiles on the producer/consumer
# kernel: every output compared, int32 and dequantised, and the padding
# between rows left untouched.
@pytest.mark.parametrize("M,N,K,ldc,shift", [(4096, 1281, 512, 1281, 0), (4096, 1282, 768, 1282, 0),
                                             (4096, 1280, 512, 1280, 1), (4000, 1300, 520, 1301, 3),
                                             (4096, 2200, 256, 2203, 0)])
def test_igemm_row_class_tiles_full_compare(M, N, K, ldc, shift):
    Au = ob.u8((M, K), 120 + N % 91)
    Bq = ob.s8((K, N), 121 + K % 83)
    sa = ob.uniform((M,), 122, 1e-3, 1e-2)
    sb = ob.uniform((N,), 123, 1e-3, 1e-2)
    off = ob.s8((N,), 124).astype(np.int32) * 1000
    announce("igemm row classes", M, N, K, ldc, shift)
    V = _exact_f64(Au, Bq)
    np.testing.assert_array_equal(_run_pitched(Au, Bq, ldc, shift), V)
    V32 = V.astype(np.int32)
    np.testing.assert_array_equal(_run_pitched(Au, Bq, ldc, shift, sa, sb, off),
                                  ob.dequant((V32 + off).astype(np.int32), sa, sb))
    np.testing.assert_array_equal(_run_pitched(Au, Bq, ldc, shift, None, sb),
                                  ob.dequant(V32, None, sb))


@pytest.mark.parametrize("K", [256, 768])
def test_igemm_row_class_tiles_beyond_256mib(K):
    # the head's route (outputs past 256 MiB) with an odd pitch: 32 row
    # classes of 128 rows on the persistent kernel, tiles in fixed slots
    # (K = 256: two K tiles per tile) or handed out from the stream's per-XCD
    # counters (K = 768), three calls in a row (the counters must be back at
    # zero after each); every output compared in row blocks
    M, N = 4096, 16401
    Au = ob.u8((M, K), 130)
    Bq = ob.s8((K, N), 131)
    sa = ob.uniform((M,), 132, 1e-3, 1e-2)
    sb = ob.uniform((N,), 133, 1e-3, 1e-2)
    off = ob.s8((N,), 134).astype(np.int32) * 1000
    announce("igemm row classes > 256 MiB", M, N, K)
    C = _run_pitched(Au, Bq, N, 0)
    for r in range(0, M, 512):
        np.testing.assert_array_equal(C[r:r + 512], _exact_f64(Au[r:r + 512], Bq))
    del C
    C = _run_pitched(Au, Bq, N, 0, sa, sb, off)
    for r in range(0, M, 512):
        V = _exact_f64(Au[r:r + 512], Bq).astype(np.int32)
        np.testing.assert_array_equal(C[r:r + 512], ob.dequant((V + off).astype(np.int32), sa[r:r + 512], sb))
    del C
    C = _run_pitched(Au, Bq, N, 0, None, sb)
    for r in range(0, M, 1024):
        V = _exact_f64(Au[r:r + 1024], Bq).astype(np.int32)
        np.testing.assert_array_equal(C[r:r + 1024], ob.dequant(V, None, sb))


def test_quantizers_byte_exact():
    M, K, N = 96, 250, 80
    A = ob.normal((M, K), 70)
    B = ob.normal((K, N), 71, 0, 0.02)
    Kpad = 256
    dA, dB = pcl.dev(A), pcl.dev(B)
    # per-tensor (quantize_A rule)
    dAu, ds = pcl.empty((M, Kpad), np.uint8), pcl.empty((1,), np.float32)
    announce("quantize_a_tensor")
    pcl.check(pcl.lib.pcl_quantize_a_tensor(dA.ptr, M, K, dAu.ptr, Kpad, ds.ptr, None))
    pcl.sync()
    Au_ref = np.empty((M, Kpad), np.uint8)
    s_ref = ob.oracle().orc_quantize_A(p(A), p(Au_ref), M, K, Kpad)
    assert ds.download((1,), np.float32)[0] == np.float32(s_ref)
    np.testing.assert_array_equal(dAu.download((M, Kpad), np.uint8), Au_ref)
    # per-row
    dsa = pcl.empty((M,), np.float32)
    announce("quantize_a_rows")
    pcl.check(pcl.lib.pcl_quantize_a_rows(dA.ptr, M, K, dAu.ptr, Kpad, dsa.ptr, None))
    pcl.sync()
    sa_ref = np.empty(M, np.float32)
    ob.oracle().orc_quantize_A_rows(p(A), p(Au_ref), p(sa_ref), M, K, Kpad)
    np.testing.assert_array_equal(dsa.download((M,), np.float32), sa_ref)
    np.testing.assert_array_equal(dAu.download((M, Kpad), np.uint8), Au_ref)
    # per-column weights, native layout
    Kp = pcl.lib.pcl_s8_kpad(K)
    dBp = pcl.DeviceBuffer(pcl.lib.pcl_s8_packed_bytes(K, N))
    dbs, dcs = pcl.empty((N,), np.float32), pcl.empty((N,), np.int32)
    announce("quantize_b_cols")
    pcl.check(pcl.lib.pcl_quantize_b_cols(dB.ptr, K, N, dBp.ptr, dbs.ptr, dcs.ptr, None))
    pcl.sync()
    Bq_ref = np.empty((K, N), np.int8)
    bs_ref = np.empty(N, np.float32)
    ob.oracle().orc_quantize_B_cols(p(B), p(Bq_ref), p(bs_ref), K, N)
    got = dBp.download((N, Kp), np.int8)
    np.testing.assert_array_equal(got[:, :K], Bq_ref.T)
    assert not got[:, K:].any()
    np.testing.assert_array_equal(dbs.download((N,), np.float32), bs_ref)
    np.testing.assert_array_equal(dcs.download((N,), np.int32), Bq_ref.astype(np.int64).sum(0))
    # reference VNNI layout
    Kv = (K + 3) & ~3
    nbp = (N // 16) * (Kv // 4) * 64
    dBv = pcl.empty((nbp,), np.int8)
    announce("quantize_b_vnni")
    pcl.check(pcl.lib.pcl_quantize_b_vnni(dB.ptr, K, N, Kv, dBv.ptr, dbs.ptr, dcs.ptr, None))
    pcl.sync()
    Bp_ref, bs2, cs2 = np.empty(nbp, np.int8), np.empty(N, np.float32), np.empty(N, np.int32)
    ob.oracle().orc_quantize_B_pack(p(B), p(Bp_ref), p(bs2), p(cs2), K, N, Kv)
    np.testing.assert_array_equal(dBv.download((nbp,), np.int8), Bp_ref)
    np.testing.assert_array_equal(dcs.download((N,), np.int32), cs2)


def test_vnni_repack_matches_native_pack():
    K, N, Kpad = 300, 64, 300
    Bq = ob.s8((K, N), 80)
    Bp = np.zeros((N // 16) * (Kpad // 4) * 64, np.int8)
    for n in range(N):  # write the VNNI layout of gemm_bench.c:254 directly
        pp, i = divmod(n, 16)
        for k in range(K):
            Bp[pp * (Kpad // 4) * 64 + (k // 4) * 64 + i * 4 + k % 4] = Bq[k, n]
    dBp = pcl.dev(Bp)
    dout = pcl.DeviceBuffer(pcl.lib.pcl_s8_packed_bytes(K, N))
    dcs = pcl.empty((N,), np.int32)
    announce("pack_b_vnni")
    pcl.check(pcl.lib.pcl_pack_b_vnni(dBp.ptr, K, Kpad, N, dout.ptr, dcs.ptr, None))
    pcl.sync()
    ref_pk, ref_cs = pack(Bq)
    Kp = pcl.lib.pcl_s8_kpad(K)
    np.testing.assert_array_equal(dout.download((N, Kp), np.int8), ref_pk.download((N, Kp), np.int8))
    np.testing.assert_array_equal(dcs.download((N,), np.int32), ref_cs)


def test_dropins_vs_reference_golden():
    """quantize_A / quantize_B_pack / gemm_int8_kernel host drop-ins against
    the bytes and floats the reference's gemm_bench.c produced."""
    g = np.load(os.path.join(GOLD, "gemm_bench_int8.npz"))
    M, K, N, Kpad = (int(v) for v in g["dims"])
    L = pcl.lib
    Au = np.empty((M, Kpad), np.uint8)
    announce("drop-in quantize_A")
    scale = L.quantize_A(p(g["A"]), p(Au), M, K, Kpad)
    pcl.check_void()
    assert np.float32(scale) == g["scale"]
    np.testing.assert_array_equal(Au, g["Au"])
    Bp = np.empty_like(g["Bp"])
    bs, cs = np.empty(N, np.float32), np.empty(N, np.int32)
    announce("drop-in quantize_B_pack")
    L.quantize_B_pack(p(g["B"]), p(Bp), p(bs), p(cs), K, N, Kpad)
    pcl.check_void()
    np.testing.assert_array_equal(Bp, g["Bp"])
    np.testing.assert_array_equal(bs, g["bscale"])
    np.testing.assert_array_equal(cs, g["colsum"])
    C = np.empty((M, N), np.float32)
    announce("drop-in gemm_int8_kernel")
    L.gemm_int8_kernel(p(g["Au"]), Kpad, p(g["Bp"]), p(g["corr"]), p(g["dq"]), p(C), M, N)
    pcl.check_void()
    np.testing.assert_array_equal(C, g["C_int8"])
    # a caller-supplied corr that is not 128*colsum is honoured too
    corr2 = (g["corr"] + 7).astype(np.int32)
    announce("drop-in gemm_int8_kernel corr+7")
    L.gemm_int8_kernel(p(g["Au"]), Kpad, p(g["Bp"]), p(corr2), p(g["dq"]), p(C), M, N)
    pcl.check_void()
    C_ref = np.empty((M, N), np.float32)
    ob.oracle().orc_gemm_int8_kernel(p(g["Au"]), Kpad, p(g["Bp"]), p(corr2), p(g["dq"]), p(C_ref), M, N)
    np.testing.assert_array_equal(C, C_ref)


def test_int8_arg_errors():
    L = pcl.lib
    assert L.pcl_gemm_u8s8_i32(None, 16, None, None, 16, 4, 16, 16, None) == pcl.PCL_ERR_INVALID_ARG
    assert L.pcl_gemm_u8s8_i32(None, 200000, None, None, 16, 4, 16, 200000, None) == pcl.PCL_ERR_RANGE
    buf = pcl.empty((64,), np.int8)
    # packed weights must be 16-byte aligned
    st = L.pcl_gemm_u8s8_i32(buf.ptr, 16, buf.ptr + 1, buf.ptr, 16, 1, 1, 16, None)
    assert st == pcl.PCL_ERR_INVALID_ARG
