"""Measured roofs on the GPU (pcl_measure_peak_mfma, pcl_measure_bandwidth,
pcl_measure_lds_feed):
gemm_bench's own roof measurements (gemm_bench.c:195-210, 287-325) restated
for the matrix cores and HBM. A roof can only be checked against physics: it
must be positive, below the part's datasheet peak (a rate above it would
mean miscounted work), and the i8 rate on zeros must not be below the rate on
random bytes (less switching, the clock stays at least as high)."""
import ctypes as C

import pytest

import pcl
from gpu_util import announce, require_device

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    require_device()


def _mfma(data):
    r = C.c_double(0)
    pcl.check(pcl.lib.pcl_measure_peak_mfma(data, C.byref(r)))
    return r.value


def test_mfma_roofs_below_datasheet_peak():
    announce("roofs: mfma")
    i8_random, i8_zero, f32 = _mfma(0), _mfma(1), _mfma(2)
    assert 500.0 < i8_random <= 5033.0 * 1.001
    assert i8_random <= i8_zero * 1.03 and i8_zero <= 5033.0 * 1.001
    assert 10.0 < f32 <= 157.3 * 1.001


def test_hbm_roof_below_datasheet_peak():
    announce("roofs: hbm")
    g = (C.c_double * 4)()
    pcl.check(pcl.lib.pcl_measure_bandwidth(512 << 20, g))
    for v in g:  # triad, copy, read, write
        assert 1000.0 < v <= 8000.0


def test_int8_tile_feed_roof():
    # the L2 -> LDS operand feed of the 128x128-tile INT8 grids: positive and
    # below what 256 CUs can take in at 64 bytes per clock at 2.4 GHz (a rate
    # above it would mean miscounted bytes); argument errors before any work
    announce("roofs: int8 tile feed")
    r = C.c_double(0)
    for m, n, k in ((2048, 2048, 2048), (4096, 1024, 4096)):
        pcl.check(pcl.lib.pcl_measure_lds_feed(m, n, k, C.byref(r)))
        assert 1000.0 < r.value <= 256 * 64 * 2.4
        pcl.check(pcl.lib.pcl_measure_tile_read(m, n, k, C.byref(r)))  # the same stream into registers
        assert 1000.0 < r.value <= 256 * 64 * 2.4
    assert pcl.lib.pcl_measure_lds_feed(2000, 2048, 2048, C.byref(r)) == pcl.PCL_ERR_INVALID_ARG
    assert pcl.lib.pcl_measure_tile_read(2048, 2048, 2000, C.byref(r)) == pcl.PCL_ERR_INVALID_ARG
