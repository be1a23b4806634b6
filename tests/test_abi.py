"""The C-ABI boundary on any host (no GPU calls are made to compute).

- libpcl_hip.so loads and exports every function include/pcl_hip.h declares;
- the header keeps the reference's exact drop-in prototypes;
- argument errors are reported as statuses before any device work, and on a
  host without a gfx950 GPU compute calls fail loudly (no CPU fallback);
- the C drivers compile and link against the library.
"""
import os
import re
import subprocess

import pytest

import pcl

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_function():
    names = pcl.header_functions()
    assert len(names) >= 50
    missing = [n for n in names if not hasattr(pcl.lib, n)]
    assert not missing, missing


# reference prototypes (argument types and order) the drop-ins must keep
REFERENCE_PROTOTYPES = {
    # tensor.h:40
    "matmul": "void matmul(const float *A, const float *B, float *C, int M, int K, int N)",
    # train.c:181
    "matmul_forward": "void matmul_forward(float *out, const float *in, const float *Wt, const float *bias, int M, int K, int N)",
    # train.c:219
    "matmul_backward": "void matmul_backward(const float *dY, const float *X, const float *Wt, float *dX, float *dW, float *db, int M, int K, int N)",
    # train.c:412, 424
    "tied_head_forward": "void tied_head_forward(float *logits, const float *lnf, const float *wte, int M)",
    "tied_head_backward": "void tied_head_backward(float *d_lnf, float *dwte, const float *d_logits, const float *lnf, const float *wte, int M)",
    # model.h:56
    "lm_head": "void lm_head(float *logits, const float *x, const float *wte, int num_tokens)",
    # transformer.c:174, generate.c:95
    "proj_token": "void proj_token(float *out, const float *in, const float *W, const float *bias, int K, int N)",
    "matvec": "void matvec(float *out, const float *x, const float *W, const float *b, int K, int N)",
    # gemm_bench.c:225, 238, 278
    "quantize_A": "float quantize_A(const float *A, uint8_t *Au, int M, int K, int Kpad)",
    "quantize_B_pack": "void quantize_B_pack(const float *B, int8_t *Bp, float *bscale, int32_t *colsum, int K, int N, int Kpad)",
    "gemm_int8_kernel": "void gemm_int8_kernel(const uint8_t *Au, int Kpad, const int8_t *Bp, const int32_t *corr, const float *dq, float *C, int M, int N)",
    # gpu_kernels.h:39, 48-51
    "gpu_init": "void gpu_init(void)",
    "gemm_nn": "void gemm_nn(const float *A, const float *B, const float *bias, float *C, int M, int K, int N)",
    "gemm_nt": "void gemm_nt(const float *A, const float *B, float *C, int M, int K, int N, int accum)",
    "gemm_tn": "void gemm_tn(const float *A, const float *B, float *C, int M, int K, int N)",
    "bias_bwd": "void bias_bwd(float *db, const float *dY, int M, int N)",
}


def _norm(s):
    return re.sub(r"\s+", " ", s).replace("( ", "(").replace(" )", ")").strip()


def test_header_keeps_reference_prototypes():
    text = open(pcl.HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {m.group(1): _norm(m.group(0).rstrip(";"))
             for m in re.finditer(r"^[a-z][\w\s\*]*?\b(\w+)\s*\([^;]*?\)\s*;", text, flags=re.M)}
    for name, proto in REFERENCE_PROTOTYPES.items():
        assert decls.get(name) == _norm(proto), (name, decls.get(name))


def test_argument_errors_before_device_work():
    L = pcl.lib
    assert L.pcl_sgemm(0, 0, -1, 4, 4, None, 4, None, 4, None, 0, None, 4, None) == pcl.PCL_ERR_INVALID_ARG
    assert L.pcl_sgemm(2, 0, 4, 4, 4, None, 4, None, 4, None, 0, None, 4, None) == pcl.PCL_ERR_INVALID_ARG
    assert L.pcl_sgemm(0, 0, 4, 4, 4, None, 4, None, 4, None, 0, None, 4, None) == pcl.PCL_ERR_INVALID_ARG
    assert b"NULL" in L.pcl_last_error()
    assert L.pcl_sgemv(0, 9, 4, 4, None, 4, None, 4, None, 0, None, 4, None) == pcl.PCL_ERR_INVALID_ARG
    assert L.pcl_gemm_u8s8_i32(None, 1 << 20, None, None, 4, 4, 4, 1 << 20, None) == pcl.PCL_ERR_RANGE
    assert L.pcl_pack_b_vnni(None, 8, 8, 15, None, None, None) == pcl.PCL_ERR_INVALID_ARG
    assert L.pcl_set_model_dims(0, 1) == pcl.PCL_ERR_INVALID_ARG
    # empty problems are valid no-ops
    assert L.pcl_sgemm(0, 0, 0, 4, 4, None, 4, None, 4, None, 0, None, 4, None) == pcl.PCL_OK
    assert L.pcl_s8_kpad(1) == 256 and L.pcl_s8_kpad(256) == 256 and L.pcl_s8_kpad(257) == 512
    assert L.pcl_s8_packed_bytes(100, 3) == 3 * 256


def test_sgemm_ex_rejects_epilogue_operands_aliasing_c():
    """An epilogue operand sharing memory with C is refused before any device
    work: with the unfused path C is written before aux_in is read, so an
    in-place residual would add the product twice. (The pointers are never
    dereferenced: the check precedes every device call.)"""
    L = pcl.lib
    base, M, N, K = 1 << 20, 64, 64, 64
    A, B, C = base, base + (1 << 16), base + (1 << 17)
    EPI_RESID, EPI_GELU = 2, 1
    # aux_in == C, and aux_in starting inside C's last row
    for aux in (C, C + 4 * ((M - 1) * N + 8)):
        L.pcl_clear_error()
        assert L.pcl_sgemm_ex(0, 0, M, N, K, A, K, B, N, None, EPI_RESID, aux, None, N, C, N, None) == \
            pcl.PCL_ERR_INVALID_ARG
        assert b"overlaps C" in L.pcl_last_error()
    # the GELU pre-activation output may not overlap C either
    L.pcl_clear_error()
    assert L.pcl_sgemm_ex(0, 0, M, N, K, A, K, B, N, None, EPI_GELU, None, C + 256, N, C, N, None) == \
        pcl.PCL_ERR_INVALID_ARG
    L.pcl_clear_error()


def test_roofs_and_groups_check_arguments_first():
    import ctypes as C
    L = pcl.lib
    r = C.c_double(0)
    assert L.pcl_measure_peak_mfma(3, C.byref(r)) == pcl.PCL_ERR_INVALID_ARG
    assert L.pcl_measure_peak_mfma(0, None) == pcl.PCL_ERR_INVALID_ARG
    assert L.pcl_measure_bandwidth(1 << 20, (C.c_double * 4)()) == pcl.PCL_ERR_INVALID_ARG
    h = C.c_void_p()
    assert L.pcl_gemv_group_create(None, 0, C.byref(h)) == pcl.PCL_ERR_INVALID_ARG
    fake = 1 << 20
    bad = [pcl.GemvDesc(kind=7, M=1, N=4, K=4, X=fake, ldx=4, W=fake, ldw=4, Y=fake, ldy=4),
           pcl.GemvDesc(kind=pcl.GEMV_F32_N, M=9, N=4, K=4, X=fake, ldx=4, W=fake, ldw=4, Y=fake, ldy=4),
           pcl.GemvDesc(kind=pcl.GEMV_F32_N, M=1, N=6, K=4, X=fake, ldx=4, W=fake, ldw=6, Y=fake, ldy=6),
           pcl.GemvDesc(kind=pcl.GEMV_F32_T, M=1, N=4, K=6, X=fake, ldx=6, W=fake, ldw=6, Y=fake, ldy=4),
           pcl.GemvDesc(kind=pcl.GEMV_U8S8, M=1, N=4, K=300, X=fake, ldx=300, W=fake, ldw=304, Y=fake, ldy=4),
           pcl.GemvDesc(kind=pcl.GEMV_F32_N, M=1, N=4, K=0, X=fake, ldx=4, W=fake, ldw=4, Y=fake, ldy=4)]
    for d in bad:
        arr = (pcl.GemvDesc * 1)(d)
        assert L.pcl_gemv_group_create(arr, 1, C.byref(h)) == pcl.PCL_ERR_INVALID_ARG
        assert not h.value
    # 8 rows of 4096 fp32 activations would need 128 KB of LDS: refused
    big = pcl.GemvDesc(kind=pcl.GEMV_F32_T, M=8, N=64, K=4096, X=fake, ldx=4096, W=fake, ldw=4096, Y=fake, ldy=64)
    assert L.pcl_gemv_group_create((pcl.GemvDesc * 1)(big), 1, C.byref(h)) == pcl.PCL_ERR_RANGE
    L.pcl_clear_error()


def test_model_capture_checks_arguments_first():
    L = pcl.lib
    assert L.pcl_model_capture(None, 1) == pcl.PCL_ERR_INVALID_ARG
    assert L.pcl_model_capture_read(None, 0, pcl.CAP_QKV, None, None, None, None) == pcl.PCL_ERR_INVALID_ARG
    L.pcl_clear_error()


def test_attention_dims_must_split_into_heads():
    """d_model must be a multiple of n_heads for the device attention drop-ins
    (otherwise the last d_model % n_heads columns would be silently ignored)."""
    L = pcl.lib
    try:
        assert L.pcl_set_model_dims(1028, 10) == pcl.PCL_OK
        assert L.pcl_set_attn_dims(1, 4, 16) == pcl.PCL_OK
        L.pcl_clear_error()
        L.attn_fwd(None, None, None, None, None)
        assert L.pcl_last_status() == pcl.PCL_ERR_INVALID_ARG
        assert b"multiple of n_heads" in L.pcl_last_error()
    finally:
        L.pcl_clear_error()


def test_no_device_fails_loudly():
    if pcl.lib.pcl_init() == pcl.PCL_OK:
        pytest.skip("a GPU is present on this host")
    assert pcl.lib.pcl_init() == pcl.PCL_ERR_NO_DEVICE
    import numpy as np

    A = np.ones((4, 4), np.float32)
    C = np.full((4, 4), -1.0, np.float32)
    pcl.lib.pcl_clear_error()
    pcl.lib.matmul(pcl.ptr(A), pcl.ptr(A), pcl.ptr(C), 4, 4, 4)
    assert pcl.lib.pcl_last_status() == pcl.PCL_ERR_NO_DEVICE
    assert (C == -1.0).all()  # nothing was computed on the CPU instead
    assert pcl.lib.pcl_malloc(16) is None


def test_c_drivers_compile_and_link(tmp_path):
    drivers = os.path.join(ROOT, "pure-c-llm_amd", "drivers")
    srcs = [f for f in os.listdir(drivers) if f.endswith(".c")]
    assert srcs
    for src in srcs:
        path = os.path.join(drivers, src)
        program = "int main(" in open(path).read()
        out = tmp_path / src.replace(".c", "" if program else ".so")
        cmd = ["gcc", "-O2", "-std=c11", "-Wall", "-Werror", "-I" + os.path.join(ROOT, "include"), path,
               "-o", str(out), "-L" + os.path.join(ROOT, "pure-c-llm_amd"), "-lpcl_hip", "-lm", "-fopenmp"]
        if not program:
            cmd[1:1] = ["-shared", "-fPIC"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
