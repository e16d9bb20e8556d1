"""GGUF files for the config-1 model: a writer, a reader, and the seeded
random-init Gemma-3 model file.

The writer mirrors the reference's test writer (crates/nncpu/src/gguf.rs:
656-778): GGUF v3, metadata, then tensor infos whose data offsets are each
tensor's bytes rounded up to 32, the data section aligned to 32. It streams
tensor data to the file, so a 1B-parameter model never sits in host memory
whole. The reader parses what the writer writes (and any GGUF v2/v3 file
with the same value types) and hands out tensor data as memory-mapped
arrays, as the reference's reader does (gguf.rs:261-332, 559-649).

`write_gemma3` draws every tensor with the reference's test generator
(xorshift64* + Box-Muller, kernels/tests.rs:9-50, in libnncpu_gemma.so's
nng_rng_normals): matrices 0.02 N(0,1) stored as BF16 (ggml type 30) or F32,
norm vectors 1 + 0.1 N(0,1) as F32. nncpu's loader decodes each matrix to
f32 and re-encodes it to its Q8_0 / Q4 layout (model/load.rs:182-243);
`nncpu_amd.gemma.Gemma3.from_gguf` does the same on the device through
nnh_upload_gguf.
"""
from __future__ import annotations

import ctypes as C
import os
import struct

import numpy as np

GGUF_MAGIC = 0x46554747  # "GGUF"
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
GGML_F32, GGML_F16, GGML_BF16 = 0, 1, 30
_SCALAR = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f", T_BOOL: "<?",
           T_U64: "<Q", T_I64: "<q", T_F64: "<d"}
ALIGN = 32


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


class GgufWriter:
    """Metadata and tensors, written as gguf.rs:656-778's GgufWriter writes them.
    Tensor data is given as a callable producing the bytes when the file is
    written (or as bytes)."""

    def __init__(self):
        self.kv: list[tuple[str, bytes]] = []
        self.tensors: list[tuple[str, list[int], int, int, object]] = []

    def _put(self, key: str, body: bytes):
        self.kv.append((key, body))
        return self

    def u32(self, key: str, v: int):
        return self._put(key, struct.pack("<II", T_U32, v))

    def i32(self, key: str, v: int):
        return self._put(key, struct.pack("<Ii", T_I32, v))

    def f32(self, key: str, v: float):
        return self._put(key, struct.pack("<If", T_F32, v))

    def bool(self, key: str, v: bool):
        return self._put(key, struct.pack("<IB", T_BOOL, 1 if v else 0))

    def str(self, key: str, v: str):
        return self._put(key, struct.pack("<I", T_STR) + _str(v))

    def strs(self, key: str, v: list[str]):
        return self._put(key, struct.pack("<IIQ", T_ARR, T_STR, len(v)) + b"".join(_str(s) for s in v))

    def f32s(self, key: str, v):
        a = np.ascontiguousarray(v, "<f4")
        return self._put(key, struct.pack("<IIQ", T_ARR, T_F32, a.size) + a.tobytes())

    def i32s(self, key: str, v):
        a = np.ascontiguousarray(v, "<i4")
        return self._put(key, struct.pack("<IIQ", T_ARR, T_I32, a.size) + a.tobytes())

    def tensor(self, name: str, ne: list[int], ggml_type: int, nbytes: int, data):
        """A tensor of `nbytes` bytes, ne[0] the row length (GGUF order);
        `data` is bytes or a callable returning them."""
        self.tensors.append((name, list(ne), ggml_type, nbytes, data))
        return self

    def write(self, path: str) -> None:
        with open(path, "wb") as f:
            f.write(struct.pack("<IIQQ", GGUF_MAGIC, 3, len(self.tensors), len(self.kv)))
            for k, body in self.kv:
                f.write(_str(k))
                f.write(body)
            offsets, off = [], 0
            for name, ne, ty, nbytes, _ in self.tensors:
                f.write(_str(name))
                f.write(struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne))
                f.write(struct.pack("<IQ", ty, off))
                offsets.append(off)
                off += (nbytes + ALIGN - 1) // ALIGN * ALIGN
            pos = f.tell()
            f.write(b"\0" * ((ALIGN - pos % ALIGN) % ALIGN))
            base = f.tell()
            for (name, _, _, nbytes, data), o in zip(self.tensors, offsets):
                f.seek(base + o)
                b = data() if callable(data) else data
                b = memoryview(np.ascontiguousarray(b)).cast("B") if isinstance(b, np.ndarray) else memoryview(b)
                if len(b) != nbytes:
                    raise ValueError(f"tensor {name}: {len(b)} bytes, declared {nbytes}")
                f.write(b)
            # The file ends after the last tensor's bytes (gguf.rs:763-767).
            f.truncate(base + (offsets[-1] + self.tensors[-1][3] if self.tensors else 0))


class GgufTensor:
    def __init__(self, name: str, ne: list[int], ggml_type: int, data: np.ndarray):
        self.name, self.ne, self.ggml_type, self.data = name, ne, ggml_type, data

    @property
    def rows(self) -> int:
        return int(np.prod(self.ne[1:])) if len(self.ne) > 1 else 1

    @property
    def cols(self) -> int:
        return self.ne[0]


def _block(ggml_type: int) -> tuple[int, int]:
    """(bytes, values) per block of the types nncpu decodes (gguf.rs:335-359)."""
    return {0: (4, 1), 1: (2, 1), 30: (2, 1), 2: (18, 32), 3: (20, 32), 6: (22, 32), 7: (24, 32), 8: (34, 32),
            12: (144, 256), 13: (176, 256), 14: (210, 256)}[ggml_type]


class GgufFile:
    """A GGUF v2/v3 file: its metadata (`kv`) and tensors (memory-mapped)."""

    def __init__(self, path: str):
        self.path = path
        self.map = np.memmap(path, dtype=np.uint8, mode="r")
        self.pos = 0
        magic, version = self._unpack("<II")
        if magic != GGUF_MAGIC or version not in (2, 3):
            raise ValueError(f"{path}: not a GGUF v2/v3 file")
        n_tensors, n_kv = self._unpack("<QQ")
        self.kv = {}
        for _ in range(n_kv):
            k = self._string()
            (ty,) = self._unpack("<I")
            self.kv[k] = self._value(ty)
        infos = []
        for _ in range(n_tensors):
            name = self._string()
            (nd,) = self._unpack("<I")
            ne = list(self._unpack("<" + "Q" * nd))
            ty, off = self._unpack("<IQ")
            infos.append((name, ne, ty, off))
        align = int(self.kv.get("general.alignment", ALIGN))
        base = (self.pos + align - 1) // align * align
        self.tensors = {}
        for name, ne, ty, off in infos:
            bb, bv = _block(ty)
            n = int(np.prod(ne))
            nbytes = n // bv * bb
            if base + off + nbytes > self.map.size:
                raise ValueError(f"{path}: tensor {name} lies outside the file")
            self.tensors[name] = GgufTensor(name, ne, ty, self.map[base + off:base + off + nbytes])

    def _unpack(self, fmt: str):
        n = struct.calcsize(fmt)
        out = struct.unpack_from(fmt, self.map, self.pos)
        self.pos += n
        return out

    def _string(self) -> str:
        (n,) = self._unpack("<Q")
        s = bytes(self.map[self.pos:self.pos + n]).decode("utf-8", errors="replace")
        self.pos += n
        return s

    def _value(self, ty: int):
        if ty == T_STR:
            return self._string()
        if ty == T_ARR:
            et, n = self._unpack("<IQ")
            if et == T_STR:
                return [self._string() for _ in range(n)]
            fmt = _SCALAR[et]
            a = np.frombuffer(self.map, dtype=np.dtype(fmt), count=n, offset=self.pos).copy()
            self.pos += n * a.itemsize
            return a
        (v,) = self._unpack(_SCALAR[ty])
        return v


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """f32 -> BF16 bits, round to nearest even (runtime.rs:15-21)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def _rng_lib():
    from .gemma import GEMMA_LIB
    L = C.CDLL(GEMMA_LIB)
    L.nng_rng_normals.argtypes = [C.c_uint64, C.c_size_t, C.c_float, C.c_float, C.c_size_t, C.c_int, C.c_void_p]
    L.nng_rng_normals.restype = None
    return L


RNG_CHUNK = 1 << 20


def normals(seed: int, n: int, mean: float, sd: float, threads: int | None = None) -> np.ndarray:
    """n values mean + sd N(0,1) from the reference's test generator, chunk c
    of RNG_CHUNK values seeded with seed + c."""
    out = np.empty(n, np.float32)
    th = threads or min(16, os.cpu_count() or 1)
    _rng_lib().nng_rng_normals(seed & (2**64 - 1), n, mean, sd, RNG_CHUNK, th, out.ctypes.data_as(C.c_void_p))
    return out


def gemma3_tensors(cfg) -> list[tuple[str, int, int, str]]:
    """(name, rows, cols, role) of a Gemma-3 model in file order (model/load.rs:
    1029-1181 names); role 'matrix' or 'norm'."""
    E, hd, ff = cfg.n_embd, cfg.head_dim, cfg.n_ff
    out = [("token_embd.weight", cfg.n_vocab, E, "matrix")]
    for li in range(cfg.n_layer):
        b = f"blk.{li}."
        out += [(b + "attn_norm.weight", 1, E, "norm"), (b + "attn_q.weight", cfg.n_head * hd, E, "matrix"),
                (b + "attn_k.weight", cfg.n_kv * hd, E, "matrix"), (b + "attn_v.weight", cfg.n_kv * hd, E, "matrix"),
                (b + "attn_q_norm.weight", 1, hd, "norm"), (b + "attn_k_norm.weight", 1, hd, "norm"),
                (b + "attn_output.weight", E, cfg.n_head * hd, "matrix"),
                (b + "post_attention_norm.weight", 1, E, "norm"), (b + "ffn_norm.weight", 1, E, "norm"),
                (b + "ffn_gate.weight", ff, E, "matrix"), (b + "ffn_up.weight", ff, E, "matrix"),
                (b + "ffn_down.weight", E, ff, "matrix"), (b + "post_ffw_norm.weight", 1, E, "norm")]
    out.append(("output_norm.weight", 1, E, "norm"))
    return out


def write_gemma3(path: str, cfg, seed: int, matrix_type: int = GGML_BF16, threads: int | None = None) -> None:
    """A Gemma-3-architecture GGUF with seeded random weights: tensor i drawn
    from seeds (seed << 32) + (i << 24) + chunk (matrices 0.02 N(0,1), norms
    1 + 0.1 N(0,1)), a synthetic vocabulary of n_vocab token strings, and the
    gemma3 keys model/load.rs:431-595 reads (sliding window every 6th layer
    global, as load.rs:1147-1165 derives it for gemma3)."""
    if matrix_type not in (GGML_F32, GGML_BF16):
        raise ValueError("matrices are written as F32 or BF16")
    w = GgufWriter()
    a = "gemma3."
    w.str("general.architecture", "gemma3").str("general.name", "nncpu-amd random gemma3")
    w.u32("general.alignment", ALIGN)
    w.u32(a + "context_length", cfg.n_ctx).u32(a + "embedding_length", cfg.n_embd)
    w.u32(a + "block_count", cfg.n_layer).u32(a + "feed_forward_length", cfg.n_ff)
    w.u32(a + "attention.head_count", cfg.n_head).u32(a + "attention.head_count_kv", cfg.n_kv)
    w.u32(a + "attention.key_length", cfg.head_dim).u32(a + "attention.value_length", cfg.head_dim)
    w.f32(a + "attention.layer_norm_rms_epsilon", cfg.rms_eps).f32(a + "rope.freq_base", cfg.rope_base)
    w.u32(a + "attention.sliding_window", cfg.window)
    w.str("tokenizer.ggml.model", "llama")
    w.strs("tokenizer.ggml.tokens", [f"<t{i}>" for i in range(cfg.n_vocab)])
    w.f32s("tokenizer.ggml.scores", np.zeros(cfg.n_vocab, np.float32))
    w.i32s("tokenizer.ggml.token_type", np.ones(cfg.n_vocab, np.int32))
    w.u32("tokenizer.ggml.bos_token_id", 2).u32("tokenizer.ggml.eos_token_id", 1)
    for i, (name, rows, cols, role) in enumerate(gemma3_tensors(cfg)):
        tseed = (seed << 32) + (i << 24)
        n = rows * cols
        if role == "norm":
            w.tensor(name, [cols], GGML_F32, 4 * n, lambda s=tseed, n=n: normals(s, n, 1.0, 0.1, threads))
        elif matrix_type == GGML_BF16:
            w.tensor(name, [cols, rows], GGML_BF16, 2 * n, lambda s=tseed, n=n: bf16_bits(normals(s, n, 0.0, 0.02, threads)))
        else:
            w.tensor(name, [cols, rows], GGML_F32, 4 * n, lambda s=tseed, n=n: normals(s, n, 0.0, 0.02, threads))
    w.write(path)
