"""ctypes bindings of libnncpu_hip.so (include/nncpu_hip.h).

Loading fails loudly: there is no CPU fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes as C
import os
import re
import subprocess

_PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(_PKG)
LIB_PATH = os.path.join(_PKG, "lib", "libnncpu_hip.so")
HEADER = os.path.join(ROOT, "include", "nncpu_hip.h")

NNH_OK, NNH_E_INVALID, NNH_E_OOM, NNH_E_DEVICE, NNH_E_STATE = 0, 1, 2, 3, 4
NNH_Q8_0, NNH_Q4S, NNH_BF16 = 1, 2, 3
NNH_ACT_F32, NNH_ACT_I8, NNH_ACT_MXI8 = 0, 1, 2
NNH_NOALLOC_SCRATCH_BYTES = 64 << 20


class NnhError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"nncpu_hip error {code}: {msg}")
        self.code = code


class InvalidArgument(NnhError, ValueError):
    """A violated precondition: where the reference's kernels panic."""


class DeviceOutOfMemory(NnhError, MemoryError):
    """ErrorKind::OutOfMemory."""


_lib = None


def build() -> None:
    """Compile libnncpu_hip.so for gfx950 with its Makefile."""
    subprocess.run(["make", "-s", "-C", os.path.join(_PKG, "csrc")], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built: run __graft_entry__.build() (no CPU fallback exists)")
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def declared_functions() -> list[str]:
    """Names of the functions include/nncpu_hip.h declares."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(nnh_\w+)\s*\(", text, flags=re.M)))


def _declare(L):
    vp, sz, i32 = C.c_void_p, C.c_size_t, C.c_int
    P = C.POINTER
    L.nnh_init.argtypes, L.nnh_init.restype = [i32], i32
    L.nnh_last_error.argtypes, L.nnh_last_error.restype = [], C.c_char_p
    L.nnh_upload_q8_0.argtypes, L.nnh_upload_q8_0.restype = [vp, vp, sz, sz, P(vp)], i32
    L.nnh_upload_q4.argtypes, L.nnh_upload_q4.restype = [vp, vp, vp, sz, sz, P(vp)], i32
    L.nnh_upload_bf16.argtypes, L.nnh_upload_bf16.restype = [vp, sz, sz, P(vp)], i32
    L.nnh_model_argmax_work_bytes.argtypes, L.nnh_model_argmax_work_bytes.restype = [vp], sz
    L.nnh_model_argmax_dev.argtypes, L.nnh_model_argmax_dev.restype = [vp, vp, vp, vp, vp, vp], i32
    L.nnh_dequantize_dev.argtypes, L.nnh_dequantize_dev.restype = [C.c_uint32, vp, sz, vp, sz, vp], i32
    L.nnh_upload_gguf.argtypes, L.nnh_upload_gguf.restype = [C.c_uint32, vp, sz, sz, sz, i32, P(vp)], i32
    L.nnh_upload.argtypes, L.nnh_upload.restype = [i32, vp, sz, sz, P(vp)], i32
    L.nnh_free.argtypes, L.nnh_free.restype = [vp], None
    L.nnh_encode_dev.argtypes, L.nnh_encode_dev.restype = [i32, vp, sz, sz, P(vp), vp], i32
    L.nnh_weight_download.argtypes, L.nnh_weight_download.restype = [vp, vp, sz], i32
    L.nnh_weight_info.argtypes, L.nnh_weight_info.restype = [vp, P(i32), P(sz), P(sz)], i32
    L.nnh_weight_prepare.argtypes, L.nnh_weight_prepare.restype = [vp, i32, sz], i32
    L.nnh_stream_reserve.argtypes, L.nnh_stream_reserve.restype = [vp, i32, sz, vp], i32
    L.nnh_stream_release.argtypes, L.nnh_stream_release.restype = [vp], i32
    L.nnh_weight_device_bytes.argtypes, L.nnh_weight_device_bytes.restype = [vp], sz
    L.nnh_model_gemv.argtypes, L.nnh_model_gemv.restype = [vp, vp, vp, i32], i32
    L.nnh_gemv_batch.argtypes, L.nnh_gemv_batch.restype = [vp, vp, sz, vp, sz, sz, i32], i32
    L.nnh_model_argmax.argtypes, L.nnh_model_argmax.restype = [vp, vp, P(sz), i32], i32
    L.nnh_gemv_batch_dev.argtypes, L.nnh_gemv_batch_dev.restype = [vp, vp, sz, vp, sz, sz, i32, vp], i32
    L.nnh_gemv_rmsnorm_dev.argtypes = [vp, vp, vp, vp, C.c_float, vp, vp, vp, vp, vp]
    L.nnh_gemv_rmsnorm_dev.restype = i32
    L.nnh_gemv_rmsnorm_act_dev.argtypes = [vp, i32, vp, vp, vp, C.c_float, vp, vp, vp, vp, vp]
    L.nnh_gemv_rmsnorm_act_dev.restype = i32
    L.nnh_gemv_batch_dev_noalloc.argtypes = [vp, vp, sz, vp, sz, sz, i32, vp]
    L.nnh_gemv_batch_dev_noalloc.restype = i32
    L.nnh_act_layout.argtypes, L.nnh_act_layout.restype = [sz, sz, P(sz), P(sz), P(sz)], i32
    L.nnh_quantize_act_dev.argtypes, L.nnh_quantize_act_dev.restype = [vp, sz, sz, sz, vp, vp], i32
    L.nnh_gemv_i8_dev.argtypes, L.nnh_gemv_i8_dev.restype = [vp, vp, sz, vp, sz, vp], i32
    L.nnh_act_layout_ex.argtypes, L.nnh_act_layout_ex.restype = [i32, sz, sz, P(sz), P(sz), P(sz)], i32
    L.nnh_quantize_act_ex_dev.argtypes, L.nnh_quantize_act_ex_dev.restype = [i32, vp, sz, sz, sz, vp, vp], i32
    L.nnh_gemv_act_dev.argtypes, L.nnh_gemv_act_dev.restype = [vp, i32, vp, sz, vp, sz, vp], i32
    L.nnh_block_dots_dev.argtypes, L.nnh_block_dots_dev.restype = [vp, vp, sz, vp, vp], i32
    L.nnh_sync.argtypes, L.nnh_sync.restype = [vp], i32
    L.nnh_weight_device_data.argtypes, L.nnh_weight_device_data.restype = [vp], vp
    L.nnh_weight_f32_layout.argtypes, L.nnh_weight_f32_layout.restype = [vp, vp], i32
    L.nnh_argmax_work_bytes.argtypes, L.nnh_argmax_work_bytes.restype = [sz], sz
    L.nnh_argmax_dev.argtypes, L.nnh_argmax_dev.restype = [vp, sz, vp, vp, vp], i32


def check(rc: int) -> None:
    if rc == NNH_OK:
        return
    msg = lib().nnh_last_error().decode(errors="replace")
    if rc == NNH_E_INVALID:
        raise InvalidArgument(rc, msg)
    if rc == NNH_E_OOM:
        raise DeviceOutOfMemory(rc, msg)
    raise NnhError(rc, msg)
