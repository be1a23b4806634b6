"""Grouped decode GEMV (pcl_gemv_group_*) on the GPU: many independent products
in one launch, each held to its single call's bar.

FP32 products (W K x N as generate.c:95-107 matvec, W N x K as the tied head
model.c:64-77) against the reference-order oracle (orc_matvec / orc_lm_head)
and the f64 truth, <= 1e-4; INT8 products (u8 x packed s8) bit-exact against
the exact integer oracle, int32 and dequantised (gemm_bench.c:272-275 order).
The groups cover the grown-model decode sweep (16 layers of
QKV 512x1536, O 512x512, FF1 512x2048, FF2 2048x512 and the 2048-vocab head)
at M = 1, 4, 8, mixed kinds in one launch, ragged N and K, and repeated runs.
"""
import ctypes as C

import numpy as np
import pytest

import binding as ob
import pcl
from gpu_util import FP32_TOL, announce, rel, require_device

pytestmark = pytest.mark.gpu
p = ob.p


@pytest.fixture(scope="module", autouse=True)
def _device():
    require_device()


def pack(Bq):
    K, N = Bq.shape
    dB = pcl.dev(Bq)
    dBp = pcl.DeviceBuffer(pcl.lib.pcl_s8_packed_bytes(K, N))
    pcl.check(pcl.lib.pcl_pack_b_s8(dB.ptr, N, K, N, dBp.ptr, None, None))
    pcl.sync()
    return dBp


class Product:
    """One product's host data, device buffers and descriptor."""

    def __init__(self, kind, M, K, N, seed, bias=False, accumulate=False, mode=2, col_off=False):
        self.kind, self.M, self.K, self.N = kind, M, K, N
        self.keep = []
        if kind == pcl.GEMV_U8S8:
            self.X = ob.u8((M, K), seed)
            self.Bq = ob.s8((K, N), seed + 1)
            self.sa = ob.uniform((M,), seed + 2, 1e-3, 1e-2) if mode == 2 else None
            self.sb = ob.uniform((N,), seed + 3, 1e-3, 1e-2) if mode >= 1 else None
            self.off = (ob.s8((N,), seed + 4).astype(np.int32) * 1000) if col_off else None
            dW = pack(self.Bq)
            ldw = pcl.lib.pcl_s8_kpad(K)
            ydt = np.int32 if mode == 0 else np.float32
        else:
            self.X = ob.normal((M, K), seed)
            self.W = ob.normal((K, N) if kind == pcl.GEMV_F32_N else (N, K), seed + 1, 0.0, 0.02)
            dW = pcl.dev(self.W)
            ldw = self.W.shape[1]
            ydt = np.float32
        self.b = ob.normal((N,), seed + 5) if bias else None
        self.Y0 = ob.normal((M, N), seed + 6) if accumulate else None
        self.ydt = ydt
        dX = pcl.dev(self.X)
        dY = pcl.dev(self.Y0) if accumulate else pcl.empty((M, N), ydt)
        db = pcl.dev(self.b) if bias else None
        dsa = pcl.dev(self.sa) if kind == pcl.GEMV_U8S8 and self.sa is not None else None
        dsb = pcl.dev(self.sb) if kind == pcl.GEMV_U8S8 and self.sb is not None else None
        doff = pcl.dev(self.off) if kind == pcl.GEMV_U8S8 and self.off is not None else None
        self.keep += [dX, dW, dY, db, dsa, dsb, doff]
        self.dY = dY
        self.desc = pcl.GemvDesc(kind=kind, M=M, N=N, K=K, X=dX.ptr, ldx=K, W=dW.ptr, ldw=ldw,
                                 bias=db.ptr if db else None, accumulate=int(accumulate),
                                 col_off=doff.ptr if doff else None, sa=dsa.ptr if dsa else None,
                                 sb=dsb.ptr if dsb else None, Y=dY.ptr, ldy=N)

    def result(self):
        return self.dY.download((self.M, self.N), self.ydt)

    def check(self):
        got = self.result()
        M, K, N = self.M, self.K, self.N
        if self.kind == pcl.GEMV_U8S8:
            V = ob.gemm_u8s8_i32(self.X, self.Bq)
            if self.off is not None:
                V = (V.astype(np.int64) + self.off).astype(np.int32)
            want = V if self.sb is None else ob.dequant(V, self.sa, self.sb)
            np.testing.assert_array_equal(got, want)
            return
        Rr = np.empty((M, N), np.float32)
        if self.kind == pcl.GEMV_F32_N:
            ob.oracle().orc_matvec(p(Rr), p(self.X), p(self.W), p(self.b) if self.b is not None else None,
                                   M, K, N)
            truth = ob.gemm_f64(self.X, self.W, bias=self.b, C0=self.Y0)
        else:
            ob.oracle().orc_lm_head(p(Rr), p(self.X), p(self.W), M, K, N)
            if self.b is not None:
                Rr = Rr + self.b
            truth = ob.gemm_f64(self.X, self.W, transB=True, bias=self.b, C0=self.Y0)
        if self.Y0 is not None:
            Rr = Rr + self.Y0
        assert rel(got, Rr) <= FP32_TOL
        assert rel(got, truth) <= FP32_TOL


LAYER = [(512, 1536), (512, 512), (512, 2048), (2048, 512)]


def run_group(prods, repeat=1):
    g = pcl.GemvGroup([q.desc for q in prods])
    for _ in range(repeat):
        g.run()
    pcl.sync()
    g.close()


@pytest.mark.parametrize("M", [1, 4, 8])
def test_group_grown_sweep_fp32(M):
    # 4 of the 16 layers (the shapes repeat) and the tied head, one launch
    prods = [Product(pcl.GEMV_F32_N, M, K, N, 1000 + 10 * i) for i, (K, N) in enumerate(LAYER * 4)]
    prods.append(Product(pcl.GEMV_F32_T, M, 512, 2048, 1900))
    announce("gemv group fp32 sweep", M, len(prods))
    run_group(prods)
    for q in prods:
        q.check()


@pytest.mark.parametrize("M", [1, 4, 8])
def test_group_grown_sweep_int8(M):
    prods = [Product(pcl.GEMV_U8S8, M, K, N, 2000 + 10 * i) for i, (K, N) in enumerate(LAYER * 4)]
    prods.append(Product(pcl.GEMV_U8S8, M, 512, 2048, 2900))
    announce("gemv group int8 sweep", M, len(prods))
    run_group(prods)
    for q in prods:
        q.check()


def test_group_mixed_kinds_ragged():
    # every kind in one launch; N not a multiple of the strip, K not of 16 or
    # 64, bias, accumulate, each INT8 output form, different M per product
    prods = [
        Product(pcl.GEMV_F32_N, 3, 100, 68, 3000, bias=True),
        Product(pcl.GEMV_F32_N, 8, 2048, 516, 3010, bias=True, accumulate=True),
        Product(pcl.GEMV_F32_N, 1, 7, 4, 3020),
        Product(pcl.GEMV_F32_T, 5, 132, 77, 3030, bias=True, accumulate=True),
        Product(pcl.GEMV_F32_T, 2, 1024, 1000, 3040),
        Product(pcl.GEMV_U8S8, 8, 1040, 300, 3050, mode=2, col_off=True),
        Product(pcl.GEMV_U8S8, 4, 100, 33, 3060, mode=1),
        Product(pcl.GEMV_U8S8, 1, 2048, 512, 3070, mode=0),
        Product(pcl.GEMV_U8S8, 6, 16, 1, 3080, mode=0, col_off=True),
    ]
    announce("gemv group mixed", len(prods))
    run_group(prods)
    for q in prods:
        q.check()


def test_group_repeated_runs_identical():
    # a group replayed gives identical bits (fixed summation order); with
    # accumulate each run adds the product again
    prods = [Product(pcl.GEMV_F32_N, 4, 2048, 512, 4000), Product(pcl.GEMV_F32_T, 4, 1024, 4096, 4010),
             Product(pcl.GEMV_U8S8, 4, 1024, 4096, 4020)]
    g = pcl.GemvGroup([q.desc for q in prods])
    announce("gemv group replay")
    g.run()
    pcl.sync()
    first = [q.result() for q in prods]
    for _ in range(3):
        g.run()
    pcl.sync()
    for q, f in zip(prods, first):
        np.testing.assert_array_equal(q.result(), f)
    g.close()
    prods[0].check()
    prods[2].check()


def test_group_head_350m_int8():
    # the 350M tied head (V 50257 x D 1024), INT8, 8 rows, in one group with a
    # small product
    prods = [Product(pcl.GEMV_U8S8, 8, 1024, 50257, 5000, mode=2),
             Product(pcl.GEMV_F32_N, 8, 1024, 1024, 5010, bias=True)]
    announce("gemv group 350M head")
    run_group(prods)
    for q in prods:
        q.check()


def test_group_staging_beyond_64kb():
    # staged activations above 64 KB of LDS (the limit is 112 KB per block):
    # fp32 N x K weights with 8 rows of K = 3072 stage 96 KB; INT8 8 rows of
    # K = 8192 stage 8 * (8192 + 16) bytes plus the 16 KB operand regions
    prods = [Product(pcl.GEMV_F32_T, 8, 3072, 1000, 6000, bias=True),
             Product(pcl.GEMV_F32_T, 7, 3000, 333, 6010, accumulate=True)]
    announce("gemv group 96 KB staging")
    run_group(prods)
    for q in prods:
        q.check()
    prods = [Product(pcl.GEMV_U8S8, 8, 8192, 700, 6020, mode=2, col_off=True)]
    announce("gemv group int8 82 KB staging")
    run_group(prods)
    for q in prods:
        q.check()


def test_group_staging_limit_is_reported():
    # beyond 112 KB per block: PCL_ERR_RANGE at creation, before any launch
    q = Product(pcl.GEMV_F32_T, 8, 4096, 16, 6030)
    grp = C.c_void_p()
    arr = (pcl.GemvDesc * 1)(q.desc)
    st = pcl.lib.pcl_gemv_group_create(arr, 1, C.byref(grp))
    assert st == pcl.PCL_ERR_RANGE, st
    assert b"LDS" in pcl.lib.pcl_last_error()


@pytest.mark.parametrize("M", [1, 2])
def test_group_int8_dot_geometry(M):
    # an all-INT8 group of one or two rows over rows of 1 to 32 packed
    # segments of 256 bytes in one launch (short, ragged N; every output
    # form; column offsets), then a group with a row of 9000 bytes
    shapes = ((7, 129), (300, 63), (700, 33), (1000, 95), (1040, 17), (2048, 31), (2100, 9),
              (4096, 23), (4200, 5), (8192, 7))
    prods = [Product(pcl.GEMV_U8S8, M, K, N, 7100 + 10 * i, mode=i % 3, col_off=i % 2 == 1)
             for i, (K, N) in enumerate(shapes)]
    announce("gemv group int8 dot geometry", M)
    run_group(prods, repeat=2)
    for q in prods:
        q.check()
    prods = [Product(pcl.GEMV_U8S8, M, 9000, 70, 7300, mode=2, col_off=True),
             Product(pcl.GEMV_U8S8, M, 512, 100, 7310, mode=1)]
    announce("gemv group int8 past the dot path", M)
    run_group(prods, repeat=2)
    for q in prods:
        q.check()


@pytest.mark.parametrize("M", [3, 4, 8])
def test_group_int8_matrix_core_slice_counts(M):
    # an all-INT8 group of three to eight rows runs the matrix-core path with
    # two 256-byte weight slices in flight per wave: rows of 1, 2, 3, 4, 5, 8
    # and 9 slices (the pair loop's odd tails included), ragged N, every
    # output form, column offsets; run twice
    shapes = ((100, 70), (512, 64), (700, 130), (1024, 33), (1040, 200), (2048, 65), (2100, 9))
    prods = [Product(pcl.GEMV_U8S8, M, K, N, 7400 + 10 * i, mode=i % 3, col_off=i % 2 == 0)
             for i, (K, N) in enumerate(shapes)]
    announce("gemv group int8 matrix-core slice counts", M)
    run_group(prods, repeat=2)
    for q in prods:
        q.check()


@pytest.mark.parametrize("M", [1, 2])
def test_group_int8_dot_path_ragged(M):
    # an all-INT8 group of one or two rows runs the dot-product path: ragged
    # N (not a multiple of the 64-row strip), K not a multiple of 16 or of
    # 256, long K, every output form, column offsets
    prods = [Product(pcl.GEMV_U8S8, M, 100, 33, 7000, mode=1),
             Product(pcl.GEMV_U8S8, M, 1040, 300, 7010, mode=2, col_off=True),
             Product(pcl.GEMV_U8S8, M, 2048, 512, 7020, mode=0),
             Product(pcl.GEMV_U8S8, M, 7, 70, 7030, mode=0, col_off=True),
             Product(pcl.GEMV_U8S8, M, 8192, 129, 7040, mode=2)]
    announce("gemv group int8 dot path", M)
    run_group(prods, repeat=2)
    for q in prods:
        q.check()
