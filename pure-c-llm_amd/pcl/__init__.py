"""ctypes binding of libpcl_hip (include/pcl_hip.h) for tests and bench.py.

The product is the C ABI; this module only declares its prototypes, wraps
device buffers around numpy arrays and turns status codes into exceptions.
There is no fallback: if libpcl_hip.so is missing, importing this module
raises, and on a host without a gfx950 GPU every compute call fails with
PCL_ERR_NO_DEVICE.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REPO_DIR = os.path.dirname(PKG_DIR)
LIB_PATH = os.path.join(PKG_DIR, "libpcl_hip.so")
HEADER_PATH = os.path.join(REPO_DIR, "include", "pcl_hip.h")

PCL_OK = 0
PCL_ERR_INVALID_ARG = 1
PCL_ERR_HIP = 2
PCL_ERR_NO_DEVICE = 3
PCL_ERR_OOM = 4
PCL_ERR_UNSET_DIMS = 5
PCL_ERR_RANGE = 6
OP_N, OP_T = 0, 1
EPI_NONE, EPI_GELU, EPI_RESID, EPI_GELU_BWD = 0, 1, 2, 3
W_FP32, W_INT8 = 0, 1
CAP_QKV, CAP_O, CAP_FF1, CAP_FF2 = 0, 1, 2, 3

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is not built (run __graft_entry__.build() or make -C pure-c-llm_amd)")

lib = C.CDLL(LIB_PATH)

_vp = C.c_void_p
_i = C.c_int
_f = C.c_float
_sz = C.c_size_t
_cp = C.c_char_p

_PROTOS = {
    # status / set-up
    "pcl_init": (_i, []),
    "pcl_last_status": (_i, []),
    "pcl_last_error": (_cp, []),
    "pcl_clear_error": (None, []),
    "pcl_set_abort_on_error": (None, [_i]),
    "pcl_set_stream": (_i, [_vp]),
    "pcl_get_stream": (_vp, []),
    "pcl_stream_synchronize": (_i, []),
    "pcl_stream_create": (_vp, []),
    "pcl_stream_destroy": (_i, [_vp]),
    "pcl_release_scratch": (_i, [_vp]),
    "pcl_graph_begin": (_i, []),
    "pcl_graph_end": (_i, [C.POINTER(_vp)]),
    "pcl_graph_launch": (_i, [_vp]),
    "pcl_graph_destroy": (_i, [_vp]),
    "pcl_device_info": (_i, [_cp, _i, C.POINTER(_i), C.POINTER(_i)]),
    "pcl_malloc": (_vp, [_sz]),
    "pcl_free": (_i, [_vp]),
    "pcl_memcpy_h2d": (_i, [_vp, _vp, _sz]),
    "pcl_memcpy_d2h": (_i, [_vp, _vp, _sz]),
    "pcl_memcpy_d2d": (_i, [_vp, _vp, _sz]),
    "pcl_memset": (_i, [_vp, _i, _sz]),
    "pcl_event_create": (_vp, []),
    "pcl_event_record": (_i, [_vp]),
    "pcl_event_elapsed_ms": (_i, [_vp, _vp, C.POINTER(_f)]),
    "pcl_event_destroy": (_i, [_vp]),
    "pcl_set_model_dims": (_i, [_i, _i]),
    "pcl_set_attn_dims": (_i, [_i, _i, _i]),
    # host-pointer drop-ins
    "matmul": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "matmul_forward": (None, [_vp, _vp, _vp, _vp, _i, _i, _i]),
    "matmul_backward": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i]),
    "tied_head_forward": (None, [_vp, _vp, _vp, _i]),
    "tied_head_backward": (None, [_vp, _vp, _vp, _vp, _vp, _i]),
    "lm_head": (None, [_vp, _vp, _vp, _i]),
    "proj_token": (None, [_vp, _vp, _vp, _vp, _i, _i]),
    "matvec": (None, [_vp, _vp, _vp, _vp, _i, _i]),
    "quantize_A": (_f, [_vp, _vp, _i, _i, _i]),
    "quantize_B_pack": (None, [_vp, _vp, _vp, _vp, _i, _i, _i]),
    "gemm_int8_kernel": (None, [_vp, _i, _vp, _vp, _vp, _vp, _i, _i]),
    "attention_forward": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "cross_entropy": (C.c_float, [_vp, _vp, _vp, _i]),
    "attention_backward": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i]),
    # device-pointer drop-ins
    "gpu_init": (None, []),
    "gemm_nn": (None, [_vp, _vp, _vp, _vp, _i, _i, _i]),
    "gemm_nt": (None, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "gemm_tn": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "bias_bwd": (None, [_vp, _vp, _i, _i]),
    "attn_fwd": (None, [_vp, _vp, _vp, _vp, _vp]),
    "ce_fwd_bwd": (None, [_vp, _vp, _vp, _vp]),
    "gelu_fwd": (None, [_vp, _vp, C.c_long]),
    "gelu_bwd": (None, [_vp, _vp, _vp, C.c_long]),
    "vec_add": (None, [_vp, _vp, _vp, C.c_long]),
    "attn_bwd": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    # native
    "pcl_sgemm": (_i, [_i, _i, _i, _i, _i, _vp, _i, _vp, _i, _vp, _i, _vp, _i, _vp]),
    "pcl_sgemv": (_i, [_i, _i, _i, _i, _vp, _i, _vp, _i, _vp, _i, _vp, _i, _vp]),
    "pcl_sgemv_noalloc": (_i, [_i, _i, _i, _i, _vp, _i, _vp, _i, _vp, _i, _vp, _i, _vp]),
    "pcl_bias_bwd": (_i, [_vp, _vp, _i, _i, _i, _vp]),
    "pcl_sgemm_ex": (_i, [_i, _i, _i, _i, _i, _vp, _i, _vp, _i, _vp, _i, _vp, _vp, _i, _vp, _i, _vp]),
    "pcl_gelu_fwd": (_i, [_vp, _vp, C.c_long, _vp]),
    "pcl_gelu_bwd": (_i, [_vp, _vp, _vp, C.c_long, _vp]),
    "pcl_vec_add": (_i, [_vp, _vp, _vp, C.c_long, _vp]),
    "pcl_attn_fwd": (_i, [_vp, _vp, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i, _vp]),
    "pcl_attn_fwd_lse": (_i, [_vp, _vp, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i, _vp]),
    "pcl_attn_bwd": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _vp]),
    "pcl_attn_bwd_ex": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _i, _i,
                             _i, _vp]),
    "pcl_cross_entropy": (_i, [_vp, _i, _vp, _vp, _i, _i, _i, _vp, _vp]),
    "pcl_head_ce": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp, _vp, _vp, C.c_long, _vp]),
    "pcl_s8_kpad": (_i, [_i]),
    "pcl_s8_packed_bytes": (_sz, [_i, _i]),
    "pcl_pack_b_s8": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp]),
    "pcl_pack_b_vnni": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp]),
    "pcl_gemm_u8s8_i32": (_i, [_vp, _i, _vp, _vp, _i, _i, _i, _i, _vp]),
    "pcl_gemm_u8s8_dq": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "pcl_gemv_u8s8_i32": (_i, [_vp, _i, _vp, _vp, _i, _i, _i, _i, _vp]),
    "pcl_gemv_u8s8_dq": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "pcl_quantize_a_tensor": (_i, [_vp, _i, _i, _vp, _i, _vp, _vp]),
    "pcl_quantize_a_rows": (_i, [_vp, _i, _i, _vp, _i, _vp, _vp]),
    "pcl_quantize_b_cols": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp]),
    "pcl_quantize_b_vnni": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp]),
    # a checkpoint on the GPU
    "pcl_model_load": (_vp, [_cp]),
    "pcl_model_load_ex": (_vp, [_cp, _i]),
    "pcl_model_header": (_i, [_vp, _vp]),
    "pcl_model_forward": (_i, [_vp, _i, _i, _vp]),
    "pcl_model_generate": (_i, [_vp, _vp, _i, _i, _vp, _i]),
    "pcl_model_free": (None, [_vp]),
    "pcl_model_capture": (_i, [_vp, _i]),
    "pcl_model_capture_read": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp]),
}


class GemvDesc(C.Structure):
    """struct pcl_gemv_desc (include/pcl_hip.h): one product of a GEMV group."""
    _fields_ = [("kind", _i), ("M", _i), ("N", _i), ("K", _i),
                ("X", _vp), ("ldx", _i), ("W", _vp), ("ldw", _i),
                ("bias", _vp), ("accumulate", _i),
                ("col_off", _vp), ("sa", _vp), ("sb", _vp),
                ("Y", _vp), ("ldy", _i)]


GEMV_F32_N, GEMV_F32_T, GEMV_U8S8 = 0, 1, 2
_PROTOS["pcl_measure_peak_mfma"] = (_i, [_i, C.POINTER(C.c_double)])
_PROTOS["pcl_measure_bandwidth"] = (_i, [C.c_long, C.POINTER(C.c_double)])
_PROTOS["pcl_measure_lds_feed"] = (_i, [_i, _i, _i, C.POINTER(C.c_double)])
_PROTOS["pcl_measure_tile_read"] = (_i, [_i, _i, _i, C.POINTER(C.c_double)])
_PROTOS["pcl_gemv_group_create"] = (_i, [C.POINTER(GemvDesc), _i, C.POINTER(_vp)])
_PROTOS["pcl_gemv_group_run"] = (_i, [_vp, _vp])
_PROTOS["pcl_gemv_group_free"] = (None, [_vp])

for _name, (_res, _args) in _PROTOS.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


class PclError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"libpcl_hip status {status}: {msg}")
        self.status = status


def last_error() -> str:
    return (lib.pcl_last_error() or b"").decode()


def check(status: int) -> None:
    if status != PCL_OK:
        raise PclError(status, last_error())


def check_void() -> None:
    """Raise if the last void drop-in on this thread recorded a failure."""
    st = lib.pcl_last_status()
    if st != PCL_OK:
        msg = last_error()
        lib.pcl_clear_error()
        raise PclError(st, msg)


def header_functions(path: str = HEADER_PATH) -> list[str]:
    """Names of every function declared in include/pcl_hip.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = []
    for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b([A-Za-z_]\w*)\s*\(([^;{]*?)\)\s*;", text, flags=re.M):
        names.append(m.group(1))
    return names


def ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class DeviceBuffer:
    """A device allocation made by pcl_malloc, freed on close()/GC."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = lib.pcl_malloc(max(self.nbytes, 16))
        if not p:
            raise PclError(lib.pcl_last_status(), last_error())
        self.ptr = p

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            check(lib.pcl_memcpy_h2d(b.ptr, a.ctypes.data_as(C.c_void_p), a.nbytes))
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib.pcl_memcpy_h2d(self.ptr, a.ctypes.data_as(C.c_void_p), a.nbytes))

    def download(self, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        if out.nbytes:
            check(lib.pcl_memcpy_d2h(out.ctypes.data_as(C.c_void_p), self.ptr, out.nbytes))
        return out

    def close(self) -> None:
        if getattr(self, "ptr", None):
            lib.pcl_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def dev(a: np.ndarray) -> DeviceBuffer:
    return DeviceBuffer.from_array(a)


def empty(shape, dtype) -> DeviceBuffer:
    return DeviceBuffer(int(np.prod(shape)) * np.dtype(dtype).itemsize)


def device_info() -> dict:
    name = C.create_string_buffer(256)
    cus, clk = _i(0), _i(0)
    check(lib.pcl_device_info(name, 256, C.byref(cus), C.byref(clk)))
    return {"name": name.value.decode(), "cus": cus.value, "clock_khz": clk.value}


def sync() -> None:
    check(lib.pcl_stream_synchronize())


class GemvGroup:
    """A pcl_gemv_group over a list of GemvDesc (freed on close()/GC). The
    caller keeps the buffers the descriptors point to alive."""

    def __init__(self, descs):
        arr = (GemvDesc * len(descs))(*descs)
        h = _vp()
        check(lib.pcl_gemv_group_create(arr, len(descs), C.byref(h)))
        self.handle = h.value

    def run(self, stream=None) -> None:
        check(lib.pcl_gemv_group_run(self.handle, stream))

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib.pcl_gemv_group_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
