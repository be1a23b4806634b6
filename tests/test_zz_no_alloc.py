"""pcl_sgemv_noalloc: the allocation-free form of pcl_sgemv, its split-K partial
sums in a static device array instead of a per-stream workspace.

It runs the same plan and kernels as pcl_sgemv, so its results must be
bit-identical to pcl_sgemv's (and within the FP32 bar of the matvec oracle,
generate.c:95-107). Two calls in a row, the second on a smaller input, check
that the shared static scratch carries nothing over from one call to the next;
a shape needing more scratch than the array holds is refused before any
launch.
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


def run(fn, opW, X, W, bias, Y0):
    M, K = X.shape
    N = W.shape[1] if opW == pcl.OP_N else W.shape[0]
    dX, dW, db = pcl.dev(X), pcl.dev(W), pcl.dev(bias)
    dY = pcl.dev(Y0)
    pcl.check(fn(opW, M, N, K, dX.ptr, K, dW.ptr, W.shape[1], db.ptr, 1, dY.ptr, N, None))
    pcl.sync()
    return dY.download((M, N), np.float32)


# (opW, M, K, N): long-K shapes, so the plan splits K and the partial sums go
# to the static scratch; the second case of each pair is smaller than the first
PAIRS = [
    ((pcl.OP_N, 8, 4096, 1536), (pcl.OP_N, 3, 2048, 512)),
    ((pcl.OP_T, 4, 8192, 96), (pcl.OP_T, 1, 4096, 40)),
]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_sgemv_twice(first, second):
    for i, (opW, M, K, N) in enumerate((first, second)):
        announce("sgemv_noalloc", opW, M, K, N)
        X = ob.normal((M, K), 900 + i + K)
        W = ob.normal((K, N) if opW == pcl.OP_N else (N, K), 910 + i + N, 0.0, 0.02)
        b = ob.normal((N,), 920 + i)
        Y0 = ob.normal((M, N), 930 + i)  # accumulate: Y += X.W + b
        got = run(pcl.lib.pcl_sgemv_noalloc, opW, X, W, b, Y0)
        want = run(pcl.lib.pcl_sgemv, opW, X, W, b, Y0)
        np.testing.assert_array_equal(got, want)
        Wn = W if opW == pcl.OP_N else np.ascontiguousarray(W.T)
        assert rel(got, ob.gemm_f64(X, Wn, bias=b) + Y0) <= FP32_TOL


def test_noalloc_refuses_oversized_scratch():
    # M = 8 over a very deep K splits into thousands of chunks: 16 MiB of
    # partial sums, beyond the 4 MiB array; refused before any launch (the
    # operand pointers are never used)
    M, N, K = 8, 256, 1 << 20
    Y = pcl.empty((M, N), np.float32)
    fake = 1 << 20
    pcl.lib.pcl_clear_error()
    st = pcl.lib.pcl_sgemv_noalloc(pcl.OP_N, M, N, K, fake, K, fake, N, None, 0, Y.ptr, N, None)
    assert st == pcl.PCL_ERR_RANGE
    assert b"static" in pcl.lib.pcl_last_error()
    pcl.lib.pcl_clear_error()
