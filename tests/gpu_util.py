"""Helpers shared by the GPU parity tests (imported by tests/test_gpu_*.py)."""
import sys

import numpy as np

import binding as ob
import pcl

FP32_TOL = 1e-4  # max|C-R| / max|R| against the CPU oracle


def require_device():
    st = pcl.lib.pcl_init()
    if st != pcl.PCL_OK:
        raise pcl.PclError(st, pcl.last_error())


def announce(*parts):
    """Name the case on stdout before a GPU step (flushed: survives a crash)."""
    print("[gpu-case]", *parts, flush=True)
    sys.stdout.flush()


def sgemm(opA, opB, A, B, M, N, K, bias=None, C0=None):
    """Run pcl_sgemm on device copies; returns C as numpy."""
    dA, dB = pcl.dev(A), pcl.dev(B)
    dbias = pcl.dev(bias) if bias is not None else None
    if C0 is None:
        dC = pcl.empty((M, N), np.float32)
    else:
        dC = pcl.dev(C0)
    lda = A.shape[1] if A.ndim == 2 else 0
    ldb = B.shape[1] if B.ndim == 2 else 0
    pcl.check(pcl.lib.pcl_sgemm(opA, opB, M, N, K, dA.ptr, max(lda, 1), dB.ptr, max(ldb, 1),
                                dbias.ptr if dbias else None, 0 if C0 is None else 1, dC.ptr, N, None))
    pcl.sync()
    return dC.download((M, N), np.float32)


def sampled_rows_f64(A, B, rows, transB=False):
    """Exact-enough reference for selected rows: f64 numpy (a library routine)."""
    Bf = B.astype(np.float64)
    if transB:
        Bf = Bf.T
    return A[rows].astype(np.float64) @ Bf


def rel(X, R):
    return ob.normwise_rel_err(X, R)
