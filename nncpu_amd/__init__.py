"""nncpu_amd: nncpu's quantized matmul on MI355X (gfx950), behind nncpu's own dispatch.

The host-side mirror of the reference's matmul dispatch
(crates/nncpu/src/model/mod.rs:417-444 ``model_gemv``,
crates/nncpu/src/model/forward.rs:15-58 ``gemv_batch``,
crates/nncpu/src/model/forward.rs:989-1011 ``model_argmax``), calling the C-ABI
of ``lib/libnncpu_hip.so`` (``include/nncpu_hip.h``). Same names and argument
meaning as the reference; a violated precondition raises ``InvalidArgument``
where the reference panics (kernels/mod.rs:12-14). Every call runs on the GPU;
there is no CPU fallback, and importing fails if the library is not built.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import (NNH_ACT_F32, NNH_ACT_I8, NNH_ACT_MXI8, NNH_BF16, NNH_Q4S, NNH_Q8_0, DeviceOutOfMemory, InvalidArgument,
                   NnhError, build, check, declared_functions, lib)

Q8_0 = NNH_Q8_0
Q4S = NNH_Q4S
BF16 = NNH_BF16
ACT_F32 = NNH_ACT_F32
ACT_I8 = NNH_ACT_I8
ACT_MXI8 = NNH_ACT_MXI8

__all__ = [
    "Q8_0", "Q4S", "BF16", "ACT_F32", "ACT_I8", "ACT_MXI8", "Weight", "init", "model_gemv", "gemv_batch", "model_argmax",
    "gemv_batch_dev", "gemv_batch_dev_noalloc", "model_argmax_dev", "model_argmax_work_bytes", "dequantize_dev", "act_layout", "quantize_act_dev", "gemv_i8_dev", "block_dots_dev", "sync",
    "act_layout_ex", "quantize_act_ex_dev", "gemv_act_dev", "stream_reserve", "stream_release",
    "NnhError", "InvalidArgument", "DeviceOutOfMemory", "build", "declared_functions",
]


def _ptr(a: np.ndarray) -> C.c_void_p:
    return a.ctypes.data_as(C.c_void_p)


def init(device: int = 0) -> None:
    check(lib().nnh_init(device))


class Weight:
    """One uploaded matrix: the device side of a reference ``Tensor``
    (runtime.rs:69-75) whose ``dtype`` is ``DType::Q8_0``, ``DType::Q4S`` or
    ``DType::BF16``."""

    def __init__(self, handle: C.c_void_p, dtype: int, rows: int, cols: int):
        self._h = handle
        self.dtype, self._rows, self._cols = dtype, rows, cols

    @classmethod
    def from_split(cls, dtype: int, data: np.ndarray, rows: int, cols: int) -> "Weight":
        """Upload from one buffer in the split layout Tensor.data points at."""
        data = np.ascontiguousarray(data).view(np.uint8)
        n = rows * cols
        need = 2 * n if dtype == BF16 else (n + n // 16) if dtype == Q8_0 else (n // 2 + n // 8)
        if (dtype == BF16 or cols % 32 == 0) and data.size < need:
            raise InvalidArgument(1, "split buffer too short")
        h = C.c_void_p()
        check(lib().nnh_upload(dtype, _ptr(data), rows, cols, C.byref(h)))
        return cls(h, dtype, rows, cols)

    @classmethod
    def q8_0(cls, qs: np.ndarray, scales: np.ndarray, rows: int, cols: int) -> "Weight":
        qs = np.ascontiguousarray(qs).view(np.int8)
        scales = np.ascontiguousarray(scales).view(np.uint16)
        if cols % 32 == 0 and (qs.size < rows * cols or scales.size < rows * cols // 32):
            raise InvalidArgument(1, "q8_0 parts too short")
        h = C.c_void_p()
        check(lib().nnh_upload_q8_0(_ptr(qs), _ptr(scales), rows, cols, C.byref(h)))
        return cls(h, Q8_0, rows, cols)

    @classmethod
    def q4(cls, qs: np.ndarray, scales: np.ndarray, biases: np.ndarray, rows: int, cols: int) -> "Weight":
        qs = np.ascontiguousarray(qs).view(np.uint8)
        scales = np.ascontiguousarray(scales).view(np.uint16)
        biases = np.ascontiguousarray(biases).view(np.uint16)
        nb = rows * cols // 32
        if cols % 32 == 0 and (qs.size < rows * cols // 2 or scales.size < nb or biases.size < nb):
            raise InvalidArgument(1, "q4 parts too short")
        h = C.c_void_p()
        check(lib().nnh_upload_q4(_ptr(qs), _ptr(scales), _ptr(biases), rows, cols, C.byref(h)))
        return cls(h, Q4S, rows, cols)

    @classmethod
    def bf16(cls, w: np.ndarray, rows: int, cols: int) -> "Weight":
        """Upload BF16 weights (rows x cols values as Tensor::bf16() views them; any width)."""
        w = np.ascontiguousarray(w).view(np.uint16)
        if w.size < rows * cols:
            raise InvalidArgument(1, "bf16 weights too short")
        h = C.c_void_p()
        check(lib().nnh_upload_bf16(_ptr(w), rows, cols, C.byref(h)))
        return cls(h, BF16, rows, cols)

    @classmethod
    def from_gguf(cls, ggml_type: int, blocks: np.ndarray, rows: int, cols: int, dtype: int) -> "Weight":
        """Decode one matrix's GGUF blocks on the device (kernels/quant.rs:107-156) and
        re-encode it to ``dtype`` (model/load.rs:182-206)."""
        blocks = np.ascontiguousarray(blocks).view(np.uint8)
        h = C.c_void_p()
        check(lib().nnh_upload_gguf(ggml_type, _ptr(blocks), blocks.size, rows, cols, dtype, C.byref(h)))
        return cls(h, dtype, rows, cols)

    @classmethod
    def encode_dev(cls, dtype: int, w_ptr: int, rows: int, cols: int, stream: int = 0) -> "Weight":
        """Encode f32 weights already in device memory with nncpu's re-encoder
        (kernels/quant.rs:31-95; BF16: f32_to_bf16 per value, load.rs:198-202) on
        the device."""
        h = C.c_void_p()
        check(lib().nnh_encode_dev(dtype, w_ptr, rows, cols, C.byref(h), stream or None))
        return cls(h, dtype, rows, cols)

    def split_bytes(self) -> int:
        n = self._rows * self._cols
        if self.dtype == BF16:
            return 2 * n
        return n + n // 16 if self.dtype == Q8_0 else n // 2 + n // 8

    def download(self) -> np.ndarray:
        """The weight in nncpu's split layout, as host bytes."""
        out = np.empty(self.split_bytes(), np.uint8)
        check(lib().nnh_weight_download(self.handle, _ptr(out), out.size))
        return out

    def prepare(self, act: int = ACT_F32, n_tok: int = 1) -> "Weight":
        """Build the device layouts a call with ``act`` over ``n_tok`` vectors
        reads (otherwise built on the first such call)."""
        check(lib().nnh_weight_prepare(self.handle, act, n_tok))
        return self

    def device_bytes(self) -> int:
        """Device memory this weight holds now."""
        return int(lib().nnh_weight_device_bytes(self.handle))

    def rows(self) -> int:
        """Rows: the output length of a gemv over this matrix (runtime.rs:103-107)."""
        return self._rows

    def cols(self) -> int:
        """Columns: the input length of a gemv (runtime.rs:97-101)."""
        return self._cols

    @property
    def handle(self) -> C.c_void_p:
        if self._h is None:
            raise InvalidArgument(1, "weight was freed")
        return self._h

    def free(self) -> None:
        if self._h is not None:
            lib().nnh_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def model_gemv(w: Weight, x: np.ndarray, y: np.ndarray | None = None, act: int = ACT_F32) -> np.ndarray:
    """y[..rows] = W x[..cols] for one vector (model/mod.rs:417-444)."""
    x = np.ascontiguousarray(x, np.float32)
    if x.size < w.cols():
        raise InvalidArgument(1, "x shorter than cols")
    out = np.empty(w.rows(), np.float32) if y is None else y
    if out.dtype != np.float32 or not out.flags.c_contiguous or out.size < w.rows():
        raise InvalidArgument(1, "y must be a contiguous f32 array of at least rows values")
    check(lib().nnh_model_gemv(w.handle, _ptr(x), _ptr(out), act))
    return out


def gemv_batch(t: Weight, x: np.ndarray, x_stride: int, y: np.ndarray, y_stride: int, n_tok: int,
               act: int = ACT_F32) -> None:
    """``n_tok`` vectors of x (``x_stride`` apart) against one pass over the
    weights, into ``n_tok`` outputs of y (``y_stride`` apart), in place
    (model/forward.rs:15-58). The Q4 block sums are formed on the device, so
    the reference's ``xsum`` scratch argument has no counterpart here."""
    if n_tok == 0:
        return
    x = np.ascontiguousarray(x, np.float32)
    if x.size < (n_tok - 1) * x_stride + t.cols():
        raise InvalidArgument(1, "x too short for n_tok vectors at x_stride")
    if y.dtype != np.float32 or not y.flags.c_contiguous or y.size < (n_tok - 1) * y_stride + t.rows():
        raise InvalidArgument(1, "y must be a contiguous f32 array covering n_tok vectors at y_stride")
    check(lib().nnh_gemv_batch(t.handle, _ptr(x), x_stride, _ptr(y), y_stride, n_tok, act))


def model_argmax(w: Weight, x: np.ndarray, act: int = ACT_F32) -> int:
    """Row of the first largest logit of W x (model/forward.rs:989-1011)."""
    x = np.ascontiguousarray(x, np.float32)
    if x.size < w.cols():
        raise InvalidArgument(1, "x shorter than cols")
    out = C.c_size_t(0)
    check(lib().nnh_model_argmax(w.handle, _ptr(x), C.byref(out), act))
    return int(out.value)


# ---- device-resident entry points (device pointers as ints) -----------------------

def gemv_batch_dev(w: Weight, x_ptr: int, x_stride: int, y_ptr: int, y_stride: int, n_tok: int,
                   act: int = ACT_F32, stream: int = 0) -> None:
    check(lib().nnh_gemv_batch_dev(w.handle, x_ptr, x_stride, y_ptr, y_stride, n_tok, act, stream or None))


def gemv_rmsnorm_dev(w: Weight, x_ptr: int, r_ptr: int, gamma_ptr: int, eps: float, x_out_ptr: int, rec_ptr: int,
                     normed_ptr: int, y_ptr: int, stream: int = 0, act: int = ACT_F32) -> None:
    """y = W ((v * rms(v)) * gamma), v = x + r (r_ptr 0: v = x), in the
    activation mode `act` (ACT_F32 bit-exact, or ACT_I8: the normed input
    quantized to Q8_0 blocks); v also to x_out / rec when non-zero (device
    pointers)."""
    if act == ACT_F32:
        check(lib().nnh_gemv_rmsnorm_dev(w.handle, x_ptr, r_ptr or None, gamma_ptr, eps, x_out_ptr or None,
                                         rec_ptr or None, normed_ptr, y_ptr, stream or None))
    else:
        check(lib().nnh_gemv_rmsnorm_act_dev(w.handle, act, x_ptr, r_ptr or None, gamma_ptr, eps, x_out_ptr or None,
                                             rec_ptr or None, normed_ptr, y_ptr, stream or None))


def gemv_batch_dev_noalloc(w: Weight, x_ptr: int, x_stride: int, y_ptr: int, y_stride: int, n_tok: int,
                           act: int = ACT_F32, stream: int = 0) -> None:
    """gemv_batch_dev with the library's fixed device scratch: allocates
    nothing (the weight must be prepared for (act, n_tok) first)."""
    check(lib().nnh_gemv_batch_dev_noalloc(w.handle, x_ptr, x_stride, y_ptr, y_stride, n_tok, act, stream or None))


def model_argmax_work_bytes(w: Weight) -> int:
    return int(lib().nnh_model_argmax_work_bytes(w.handle))


def model_argmax_dev(w: Weight, x_ptr: int, logits_ptr: int, work_ptr: int, out_ptr: int, stream: int = 0) -> None:
    """model_argmax on device buffers (f32 activations); the row lands in the u64 at out_ptr."""
    check(lib().nnh_model_argmax_dev(w.handle, x_ptr, logits_ptr, work_ptr, out_ptr, stream or None))


def act_layout(cols: int, n_tok: int) -> tuple[int, int, int]:
    """(offset of the BF16 scales, offset of the f64 pairs, total bytes)."""
    a, b, c = C.c_size_t(), C.c_size_t(), C.c_size_t()
    check(lib().nnh_act_layout(cols, n_tok, C.byref(a), C.byref(b), C.byref(c)))
    return a.value, b.value, c.value


def act_layout_ex(act: int, cols: int, n_tok: int) -> tuple[int, int, int]:
    """act_layout for either int8 mode (ACT_I8, ACT_MXI8)."""
    a, b, c = C.c_size_t(), C.c_size_t(), C.c_size_t()
    check(lib().nnh_act_layout_ex(act, cols, n_tok, C.byref(a), C.byref(b), C.byref(c)))
    return a.value, b.value, c.value


def quantize_act_ex_dev(act: int, x_ptr: int, x_stride: int, cols: int, n_tok: int, buf_ptr: int,
                        stream: int = 0) -> None:
    check(lib().nnh_quantize_act_ex_dev(act, x_ptr, x_stride, cols, n_tok, buf_ptr, stream or None))


def gemv_act_dev(w: Weight, act: int, buf_ptr: int, n_tok: int, y_ptr: int, y_stride: int, stream: int = 0) -> None:
    check(lib().nnh_gemv_act_dev(w.handle, act, buf_ptr, n_tok, y_ptr, y_stride, stream or None))


def quantize_act_dev(x_ptr: int, x_stride: int, cols: int, n_tok: int, act_ptr: int, stream: int = 0) -> None:
    check(lib().nnh_quantize_act_dev(x_ptr, x_stride, cols, n_tok, act_ptr, stream or None))


def gemv_i8_dev(w: Weight, act_ptr: int, n_tok: int, y_ptr: int, y_stride: int, stream: int = 0) -> None:
    check(lib().nnh_gemv_i8_dev(w.handle, act_ptr, n_tok, y_ptr, y_stride, stream or None))


def block_dots_dev(w: Weight, act_ptr: int, n_tok: int, P_ptr: int, stream: int = 0) -> None:
    check(lib().nnh_block_dots_dev(w.handle, act_ptr, n_tok, P_ptr, stream or None))


def dequantize_dev(ggml_type: int, blocks_ptr: int, nbytes: int, dst_ptr: int, n: int, stream: int = 0) -> None:
    """kernels/quant.rs:107-156 on the device: n values of GGUF blocks into f32 dst."""
    check(lib().nnh_dequantize_dev(ggml_type, blocks_ptr, nbytes, dst_ptr, n, stream or None))


def stream_reserve(w: Weight, act: int, n_tok: int, stream: int = 0) -> None:
    """Build the layouts and size ``stream``'s scratch for a call (w, act, n_tok)
    ahead of time, so such calls on ``stream`` allocate nothing (graph capture)."""
    check(lib().nnh_stream_reserve(w.handle, act, n_tok, stream or None))


def stream_release(stream: int = 0) -> None:
    """Free the library's scratch for ``stream`` (waits for its queued work)."""
    check(lib().nnh_stream_release(stream or None))


def sync(stream: int = 0) -> None:
    check(lib().nnh_sync(stream or None))
