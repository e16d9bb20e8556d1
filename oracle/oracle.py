"""ctypes front end of the CPU oracle (oracle.cpp, avx2.cpp).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
bench.py's cpu_baseline leg, never by the product package ``nncpu_amd``.

Array helpers build nncpu's split weight layouts (crates/nncpu/src/runtime.rs:52-63,
136-164) from f32 matrices with the restated re-encoder (kernels/quant.rs:31-95),
and run the restated kernels on them.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

Q8_0 = 1
Q4S = 2

_lib = None


def build() -> None:
    """Compile liboracle.so with its Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def _declare(L):
    vp, sz, f32, i32 = C.c_void_p, C.c_size_t, C.c_float, C.c_int
    L.or_bf16_to_f32.argtypes, L.or_bf16_to_f32.restype = [C.c_uint16], f32
    L.or_f32_to_bf16.argtypes, L.or_f32_to_bf16.restype = [f32], C.c_uint16
    L.or_rint.argtypes, L.or_rint.restype = [f32], C.c_int32
    L.or_quantize_q8_0.argtypes = [vp, sz, vp, vp]
    L.or_quantize_q4.argtypes = [vp, sz, vp, vp, vp]
    L.or_block_sums.argtypes = [vp, sz, vp]
    L.or_dot_bf16_f32.argtypes, L.or_dot_bf16_f32.restype = [vp, vp, sz], f32
    L.or_gemv_q8_0_batch.argtypes, L.or_gemv_q8_0_batch.restype = [vp, vp, vp, sz, vp, sz, sz, sz, sz], i32
    L.or_gemv_q4_batch.argtypes, L.or_gemv_q4_batch.restype = [vp, vp, vp, vp, sz, vp, sz, vp, sz, sz, sz, sz], i32
    L.or_gemv_batch.argtypes, L.or_gemv_batch.restype = [i32, vp, sz, sz, vp, sz, vp, sz, sz], i32
    L.or_argmax.argtypes, L.or_argmax.restype = [vp, sz], sz
    L.or_gemv_bf16.argtypes = [vp, vp, vp, sz, sz]
    L.or_gemv_bf16_batch.argtypes = [vp, vp, sz, vp, sz, sz, sz, sz]
    L.or_gemv_bf16_argmax.argtypes, L.or_gemv_bf16_argmax.restype = [vp, vp, sz, sz], sz
    L.or_dequantize_to_f32.argtypes, L.or_dequantize_to_f32.restype = [C.c_uint32, vp, sz, vp, sz], i32
    L.or_block_dots.argtypes = [i32, vp, sz, sz, vp, vp]
    L.or_dequant_act.argtypes = [vp, vp, sz, vp]
    L.or_gemv_i8_exact.argtypes = [i32, vp, sz, sz, vp, vp, vp]
    L.or_rng_init.argtypes = [C.POINTER(C.c_uint64), C.c_uint64]
    L.or_rng_next.argtypes, L.or_rng_next.restype = [C.POINTER(C.c_uint64)], C.c_uint64
    L.or_rng_uniform.argtypes = [C.POINTER(C.c_uint64), sz, f32, f32, vp]
    L.or_rng_normals.argtypes = [C.POINTER(C.c_uint64), sz, f32, vp]
    L.avx_available.restype = i32
    L.avx_set_threads.argtypes = [i32]
    L.avx_threads.restype = i32
    L.avx_gemv_batch.argtypes, L.avx_gemv_batch.restype = [i32, vp, sz, sz, vp, sz, vp, sz, sz], i32
    L.avx_stream_gbs.argtypes, L.avx_stream_gbs.restype = [sz, i32], C.c_double


# ---- scalars ---------------------------------------------------------------------

def bf16_to_f32(v: int) -> float:
    return lib().or_bf16_to_f32(v)


def f32_to_bf16(v: float) -> int:
    return lib().or_f32_to_bf16(v)


def rint(v: float) -> int:
    return lib().or_rint(v)


def bf16_array_to_f32(a: np.ndarray) -> np.ndarray:
    """Exact BF16 -> F32 (runtime.rs:10-13), vectorised."""
    return (a.astype(np.uint32) << 16).view(np.float32)


# ---- deterministic data: kernels/tests.rs:9-50 ----------------------------------

class Rng:
    """xorshift64* with Box-Muller normals, as the reference's test Rng."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(0)
        lib().or_rng_init(C.byref(self.state), C.c_uint64(seed & (2**64 - 1)))

    def next_u64(self) -> int:
        return lib().or_rng_next(C.byref(self.state))

    def vec(self, n: int, lo: float, hi: float) -> np.ndarray:
        out = np.empty(n, np.float32)
        lib().or_rng_uniform(C.byref(self.state), n, lo, hi, _p(out))
        return out

    def normals(self, n: int, sd: float) -> np.ndarray:
        out = np.empty(n, np.float32)
        lib().or_rng_normals(C.byref(self.state), n, sd, _p(out))
        return out


# ---- re-encoder (quant.rs:31-95) and split layouts ------------------------------

def quantize_q8_0(src: np.ndarray):
    src = np.ascontiguousarray(src, np.float32).ravel()
    n = src.size
    assert n % 32 == 0
    qs = np.empty(n, np.int8)
    sc = np.empty(n // 32, np.uint16)
    lib().or_quantize_q8_0(_p(src), n, _p(qs), _p(sc))
    return qs, sc


def quantize_q4(src: np.ndarray):
    src = np.ascontiguousarray(src, np.float32).ravel()
    n = src.size
    assert n % 32 == 0
    qs = np.empty(n // 2, np.uint8)
    sc = np.empty(n // 32, np.uint16)
    bi = np.empty(n // 32, np.uint16)
    lib().or_quantize_q4(_p(src), n, _p(qs), _p(sc), _p(bi))
    return qs, sc, bi


def pack_q8(qs: np.ndarray, sc: np.ndarray) -> np.ndarray:
    """One buffer in the Q8_0 split layout: i8 qs[n], then bf16 scales[n/32]."""
    return np.concatenate([qs.view(np.uint8).ravel(), sc.view(np.uint8).ravel()])


def pack_q4(qs: np.ndarray, sc: np.ndarray, bi: np.ndarray) -> np.ndarray:
    """One buffer in the Q4 split layout: u8 qs[n/2], bf16 scales[n/32], bf16 biases[n/32]."""
    return np.concatenate([qs.ravel(), sc.view(np.uint8).ravel(), bi.view(np.uint8).ravel()])


class QMatrix:
    """A matrix re-encoded by the restated nncpu encoder, in one split-layout buffer."""

    def __init__(self, dtype: int, rows: int, cols: int, parts):
        self.dtype, self.rows, self.cols = dtype, rows, cols
        self.parts = parts
        self.buf = pack_q8(*parts) if dtype == Q8_0 else pack_q4(*parts)

    @staticmethod
    def from_f32(dtype: int, w: np.ndarray) -> "QMatrix":
        rows, cols = w.shape
        parts = quantize_q8_0(w) if dtype == Q8_0 else quantize_q4(w)
        return QMatrix(dtype, rows, cols, parts)

    @staticmethod
    def from_split(dtype: int, rows: int, cols: int, buf: np.ndarray) -> "QMatrix":
        """Wrap bytes in the split layout (runtime.rs:136-164)."""
        buf = np.ascontiguousarray(buf).view(np.uint8)
        n = rows * cols
        if dtype == Q8_0:
            parts = (buf[:n].view(np.int8), buf[n:n + n // 16].view(np.uint16))
        else:
            parts = (buf[:n // 2], buf[n // 2:n // 2 + n // 16].view(np.uint16),
                     buf[n // 2 + n // 16:n // 2 + n // 8].view(np.uint16))
        return QMatrix(dtype, rows, cols, parts)

    def dequant_quants(self) -> np.ndarray:
        """The integer quants in element order, [rows][cols] (Q4: byte i of a
        block holds element i low, element i + 16 high; runtime.rs:58-62)."""
        if self.dtype == Q8_0:
            return self.parts[0].astype(np.int32).reshape(self.rows, self.cols)
        blk = self.parts[0].reshape(-1, 16)
        return np.concatenate([blk & 15, blk >> 4], axis=1).astype(np.int32).reshape(self.rows, self.cols)

    def dequant(self) -> np.ndarray:
        """f32 weights the kernels multiply by (kernels/tests.rs:380-397)."""
        if self.dtype == Q8_0:
            qs, sc = self.parts
            s = bf16_array_to_f32(sc).repeat(32)
            return (qs.astype(np.float32) * s).reshape(self.rows, self.cols)
        qs, sc, bi = self.parts
        s = bf16_array_to_f32(sc)
        b = bf16_array_to_f32(bi)
        blk = qs.reshape(-1, 16)
        q = np.concatenate([blk & 15, blk >> 4], axis=1).astype(np.float32)  # elements 0..15, 16..31
        return (q * s[:, None] + b[:, None]).reshape(self.rows, self.cols)


# ---- kernels -----------------------------------------------------------------------

def block_sums(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size // 32, np.float32)
    lib().or_block_sums(_p(x), x.size, _p(out))
    return out


def dot_bf16_f32(a: np.ndarray, b: np.ndarray) -> float:
    a = np.ascontiguousarray(a, np.uint16)
    b = np.ascontiguousarray(b, np.float32)
    return lib().or_dot_bf16_f32(_p(a), _p(b), a.size)


def gemv_batch(m: QMatrix, x: np.ndarray, n_tok: int = 1, x_stride: int | None = None,
               y_stride: int | None = None, backend: str = "scalar") -> np.ndarray:
    """model/forward.rs:15-58 on the scalar (oracle.cpp) or AVX2 (avx2.cpp) restatement."""
    x = np.ascontiguousarray(x, np.float32)
    xs = m.cols if x_stride is None else x_stride
    ys = m.rows if y_stride is None else y_stride
    assert x.size >= (n_tok - 1) * xs + m.cols
    y = np.zeros((n_tok - 1) * ys + m.rows, np.float32)
    fn = lib().or_gemv_batch if backend == "scalar" else lib().avx_gemv_batch
    rc = fn(m.dtype, _p(m.buf), m.rows, m.cols, _p(x), xs, _p(y), ys, n_tok)
    if rc != 0:
        raise ValueError("gemv precondition violated")
    return y


def argmax(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, np.float32)
    return lib().or_argmax(_p(v), v.size)


# ---- BF16 weights (kernels/mod.rs:337-406, 454-485; scalar.rs:555-628) -------------

BF16 = 3


def f32_array_to_bf16(a: np.ndarray) -> np.ndarray:
    """runtime.rs:15-21 round to nearest even, vectorised (WeightFormat::Bf16's encoder, load.rs:198-202)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def gemv_bf16(w: np.ndarray, x: np.ndarray, rows: int, cols: int, n_tok: int = 1,
              x_stride: int | None = None, y_stride: int | None = None) -> np.ndarray:
    """gemv_bf16 / gemv_bf16_batch on the scalar restatement."""
    w = np.ascontiguousarray(w, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    xs = cols if x_stride is None else x_stride
    ys = rows if y_stride is None else y_stride
    assert w.size >= rows * cols and x.size >= (n_tok - 1) * xs + cols
    y = np.zeros((n_tok - 1) * ys + rows, np.float32)
    lib().or_gemv_bf16_batch(_p(w), _p(x), xs, _p(y), ys, rows, cols, n_tok)
    return y


# gguf.rs:335-355 (decodable types): ggml type code -> (bytes, elements) per block.
GGML_BLOCKS = {0: (4, 1), 1: (2, 1), 30: (2, 1), 2: (18, 32), 3: (20, 32), 6: (22, 32), 7: (24, 32),
               8: (34, 32), 12: (144, 256), 13: (176, 256), 14: (210, 256)}


def dequantize_to_f32(ggml_type: int, blocks: np.ndarray, n: int, fill: float = 9.0):
    """kernels/quant.rs:107-156: (ok, dst); dst is left at `fill` when not ok."""
    blocks = np.ascontiguousarray(blocks).view(np.uint8)
    dst = np.full(n, fill, np.float32)
    ok = lib().or_dequantize_to_f32(ggml_type, _p(blocks), blocks.size, _p(dst), n)
    return bool(ok), dst


def gemv_bf16_argmax(w: np.ndarray, x: np.ndarray, rows: int, cols: int) -> int:
    w = np.ascontiguousarray(w, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    return lib().or_gemv_bf16_argmax(_p(w), _p(x), rows, cols)


def quantize_act(x: np.ndarray):
    """The int8-block activation quantizer: nncpu's own Q8_0 encoder on x."""
    return quantize_q8_0(x)


def mx_exponent(amax: np.ndarray) -> np.ndarray:
    """Exponent of the MX block scale (the library's NNH_ACT_MXI8; no
    counterpart in nncpu, which never quantizes activations): the least E
    with 127 * 2^E >= amax, clamped to [-126, 127], read off the f32 bits.
    amax = (1 + f) 2^e: 127 * 2^(e-6) = 1.984375 * 2^e covers it unless
    f > 0.984375 (mantissa field above 0x7E0000). Pinned against a direct
    search over E by tests/test_mx.py."""
    u = np.ascontiguousarray(amax, np.float32).view(np.uint32).astype(np.int64)
    be = u >> 23
    e = be - 127 - 6 + ((u & 0x7FFFFF) > 0x7E0000)
    e = np.where(be == 0, -126, e)
    return np.clip(e, -126, 127)


def quantize_act_mx(x: np.ndarray):
    """MX int8 activation blocks: per block of 32, scale 2^E (mx_exponent of
    the block's largest |x|, NaNs skipped), q = rint(x / 2^E) ties to even,
    NaN -> 0, clamped to +-127; an all-zero (or all-NaN) block gets scale 0
    and q = 0. Returns (q int8, scales as BF16 bits)."""
    xb = np.ascontiguousarray(x, np.float32).reshape(-1, 32)
    a = np.abs(xb)
    a = np.where(np.isnan(a), np.float32(0), a)
    amax = a.max(axis=1)
    E = mx_exponent(amax)
    zero = ~(amax > 0)
    with np.errstate(invalid="ignore", over="ignore"):
        v = np.ldexp(xb.astype(np.float64), -E[:, None])  # exact: a power-of-two scaling
        r = np.rint(v)
    r = np.where(np.isnan(r), 0.0, r)
    q = np.clip(r, -127, 127).astype(np.int8)
    q[zero] = 0
    scale = np.where(zero, np.float32(0), np.ldexp(np.float32(1), E).astype(np.float32)).astype(np.float32)
    return q.reshape(-1), (scale.view(np.uint32) >> 16).astype(np.uint16)


def mx_limbs(X: np.ndarray):
    """X = hi + lo as two BF16 values: hi = X's top 8 significant bits (its f32
    bits with the low half cleared), lo = X - hi (exact for X of at most 16
    significant bits). Returns both as BF16 bits."""
    X = np.ascontiguousarray(X, np.float32)
    hb = X.view(np.uint32) & np.uint32(0xFFFF0000)
    lo = (X - hb.view(np.float32)).astype(np.float32)
    return (hb >> 16).astype(np.uint16), (lo.view(np.uint32) >> 16).astype(np.uint16)


def gemm_exact(m: "QMatrix", qx: np.ndarray, sx: np.ndarray, n_tok: int):
    """Batched restatement of or_gemv_i8_exact in numpy for many vectors:
    y[t][r] = sum_b s_w[r,b] s_x[t,b] P_b[t][r] (+ Q4: bias[r,b] s_x[t,b]
    sum_k q_x[t,32b+k]), each block term exact in f64 (integer block dots by
    f64 matmuls of integers below 2^53), summed in f64. Returns (y as f64,
    sum of |terms| as f64), both [n_tok][rows]."""
    rows, cols = m.rows, m.cols
    nb = cols // 32
    wq = m.dequant_quants().astype(np.float64).reshape(rows, nb, 32)
    sw = bf16_array_to_f32(m.parts[1]).astype(np.float64).reshape(rows, nb)
    q = np.asarray(qx, np.int8).astype(np.float64).reshape(n_tok, nb, 32)
    s = bf16_array_to_f32(np.asarray(sx, np.uint16)).astype(np.float64).reshape(n_tok, nb)
    y = np.zeros((n_tok, rows))
    mag = np.zeros((n_tok, rows))
    for b in range(nb):
        P = q[:, b, :] @ wq[:, b, :].T  # exact integers
        t = P * (s[:, b][:, None] * sw[:, b][None, :])
        if m.dtype == Q4S:
            bi = bf16_array_to_f32(m.parts[2]).astype(np.float64).reshape(rows, nb)
            t = t + (s[:, b] * q[:, b, :].sum(axis=1))[:, None] * bi[:, b][None, :]
        y += t
        mag += np.abs(t)
    return y, mag


def dequant_act(qx: np.ndarray, sx: np.ndarray) -> np.ndarray:
    out = np.empty(qx.size, np.float32)
    lib().or_dequant_act(_p(np.ascontiguousarray(qx)), _p(np.ascontiguousarray(sx)), qx.size, _p(out))
    return out


def block_dots(m: QMatrix, qx: np.ndarray) -> np.ndarray:
    P = np.empty(m.rows * (m.cols // 32), np.int32)
    qs = m.parts[0]
    lib().or_block_dots(m.dtype, _p(qs), m.rows, m.cols, _p(np.ascontiguousarray(qx)), _p(P))
    return P.reshape(m.rows, m.cols // 32)


def gemv_i8_exact(m: QMatrix, qx: np.ndarray, sx: np.ndarray) -> np.ndarray:
    y = np.empty(m.rows, np.float32)
    lib().or_gemv_i8_exact(m.dtype, _p(m.buf), m.rows, m.cols, _p(np.ascontiguousarray(qx)),
                           _p(np.ascontiguousarray(sx)), _p(y))
    return y


def avx_available() -> bool:
    return bool(lib().avx_available())


def avx_set_threads(n: int) -> None:
    lib().avx_set_threads(n)


def avx_threads() -> int:
    return lib().avx_threads()


def avx_stream_gbs(nbytes: int = 512 << 20, reps: int = 3) -> float:
    return lib().avx_stream_gbs(nbytes, reps)
