"""Gemma-3 decode through the GPU matmul.

A Gemma-3-architecture model loaded from a GGUF file (nncpu_amd.gguf writes
the seeded random-init one: matrices 0.02*N(0,1) as BF16, norms
1 + 0.1*N(0,1)), every matrix decoded and re-encoded to nncpu's Q8_0 (or Q4)
layout on the device (nncpu's load-time decode and encoder, bit for bit). The
forward pass is nncpu's
(nncpu_amd/host/gemma3.cpp, restating crates/nncpu/src/model/forward.rs) on
the CPU; its weight matmuls run through `nnh_gemv_batch` in the bit-exact
f32 mode and the greedy lm_head through `nnh_model_argmax`. The prompt is
evaluated in 16-token batches (session/engine.rs:362-380, PREFILL_BATCH).

`Gemma3.generate_device` runs the same prefill, then decodes on the GPU
alone (nncpu_amd/host/gemma3_gpu.hip): one persistent kernel runs every
layer of a step with the CPU restatement's arithmetic, then the lm_head
argmax; the step is captured in a HIP graph and replayed per token.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import ACT_F32, Q8_0, Weight, check, lib
from ._lib import _PKG

GEMMA_LIB = os.path.join(_PKG, "lib", "libnncpu_gemma.so")


class NngConfig(C.Structure):
    _fields_ = [("n_layer", C.c_int), ("n_embd", C.c_int), ("n_head", C.c_int), ("n_kv", C.c_int),
                ("head_dim", C.c_int), ("n_ff", C.c_int), ("n_vocab", C.c_int), ("n_ctx", C.c_int),
                ("rms_eps", C.c_float), ("rope_base", C.c_float), ("rope_base_swa", C.c_float),
                ("attn_scale", C.c_float), ("window", C.c_int), ("swa_period", C.c_int), ("wtype", C.c_int),
                ("arch", C.c_int), ("rope_mode", C.c_int)]  # arch 0 Gemma-3, 1 Llama, 2 Qwen2; rope_mode 0 NeoX, 1 Norm


class NngGpuCtx(C.Structure):
    _fields_ = [("w", C.POINTER(C.c_void_p)), ("n", C.c_int), ("act", C.c_int)]


def gemma3_1b_config(n_ctx: int = 256, n_layer: int = 26, n_vocab: int = 262144) -> NngConfig:
    """Gemma-3-1B's architecture (26 layers, d 1152, FFN 6912, 4 query heads /
    1 KV head, head_dim 256, vocab 262144, sliding window 512 with every 6th
    layer global, RoPE bases 1e6 / 1e4, attention scale 1/16)."""
    return NngConfig(n_layer=n_layer, n_embd=1152, n_head=4, n_kv=1, head_dim=256, n_ff=6912, n_vocab=n_vocab,
                     n_ctx=n_ctx, rms_eps=1e-6, rope_base=1e6, rope_base_swa=1e4, attn_scale=1.0 / 16.0,
                     window=512, swa_period=6, wtype=Q8_0)


def matrix_shapes(cfg: NngConfig) -> list[tuple[int, int]]:
    """(rows, cols) of matrix id = 7*layer + {q, k, v, o, gate, up, down}; the tied lm_head last."""
    E, hd, ff = cfg.n_embd, cfg.head_dim, cfg.n_ff
    per = [(cfg.n_head * hd, E), (cfg.n_kv * hd, E), (cfg.n_kv * hd, E), (E, cfg.n_head * hd),
           (ff, E), (ff, E), (E, ff)]
    return per * cfg.n_layer + [(cfg.n_vocab, E)]


def _gemma_lib():
    L = C.CDLL(GEMMA_LIB)
    L.nng_create.argtypes = [C.POINTER(NngConfig), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
    L.nng_create.restype = C.c_void_p
    L.nng_free.argtypes = [C.c_void_p]
    L.nng_error.argtypes, L.nng_error.restype = [C.c_void_p], C.c_char_p
    L.nng_generate.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_void_p,
                               C.c_void_p, C.POINTER(C.c_size_t), C.POINTER(C.c_double), C.POINTER(C.c_double)]
    L.nng_generate.restype = C.c_int
    L.nng_forward.argtypes, L.nng_forward.restype = [C.c_void_p, C.c_void_p, C.c_size_t], C.c_int
    L.nng_argmax_last.argtypes, L.nng_argmax_last.restype = [C.c_void_p, C.c_size_t, C.POINTER(C.c_int32)], C.c_int
    L.nng_state.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.POINTER(C.c_size_t),
                            C.POINTER(C.POINTER(C.c_uint64)), C.POINTER(C.c_size_t)]
    L.nng_fnv_many.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p]
    L.nngd_create.argtypes = [C.POINTER(NngConfig), C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_void_p)]
    L.nngd_create.restype = C.c_int
    L.nngd_free.argtypes = [C.c_void_p]
    L.nngd_error.argtypes, L.nngd_error.restype = [C.c_void_p], C.c_char_p
    L.nngd_decode.argtypes = [C.c_void_p, C.c_void_p, C.c_int32, C.c_int, C.c_void_p, C.c_void_p,
                              C.POINTER(C.c_double)]
    L.nngd_decode.restype = C.c_int
    return L


def gemma3_config_from_kv(kv: dict, n_ctx: int, dtype: int, path: str = "") -> NngConfig:
    """A Gemma-3 GGUF's hyperparameters as nncpu's loader reads them
    (model/load.rs:431-595, 1147-1165). Models these forwards cannot run as
    the reference would (RoPE linear scaling, every layer sliding, a
    non-periodic sliding pattern) raise ValueError."""
    a = "gemma3."
    E, nh = int(kv[a + "embedding_length"]), int(kv[a + "attention.head_count"])
    hd = int(kv.get(a + "attention.key_length", E // nh))
    n_layer = int(kv[a + "block_count"])
    # RoPE linear scaling (load.rs:550-554) scales the global layers'
    # positions (forward.rs:296-304; Gemma-3 4B/12B/27B); neither forward
    # here carries that scale, so such a model is refused, not run wrong.
    if kv.get(a + "rope.scaling.type", "") == "linear" and float(kv.get(a + "rope.scaling.factor", 0.0)) > 0.0:
        raise ValueError(f"{path}: RoPE linear scaling is not supported by these forwards")
    base = float(kv.get(a + "rope.freq_base", 10000.0))
    base_swa = float(kv.get(a + "rope.freq_base_swa", 0.0))
    base_swa = base_swa if base_swa > 0.0 else 10000.0  # load.rs:486-492: gemma3's unstored local theta
    window = max(int(kv.get(a + "attention.sliding_window", 0)), 0)
    # Sliding layers (load.rs:1147-1165): a per-layer array, else every
    # `period`-th layer global (default 6), none when the window is 0.
    pat = kv.get(a + "attention.sliding_window_pattern")
    period = 6
    if isinstance(pat, (list, tuple, np.ndarray)) and len(pat) == n_layer:
        flags = [int(v) != 0 for v in pat]
        globals_ = [i for i, v in enumerate(flags) if not v]
        period = globals_[0] + 1 if globals_ else 0
        if period > 0 and [(i + 1) % period != 0 for i in range(n_layer)] != flags:
            raise ValueError(f"{path}: a sliding-window layer pattern that is not periodic is not supported")
    elif pat is not None and not isinstance(pat, (list, tuple, np.ndarray)):
        period = int(pat)
    if window == 0:
        period = 0  # no layer slides, every layer takes the global RoPE base
    elif period <= 0:
        raise ValueError(f"{path}: every layer sliding (pattern <= 0) is not supported")
    cfg = NngConfig(n_layer=n_layer, n_embd=E, n_head=nh,
                    n_kv=int(kv.get(a + "attention.head_count_kv", nh)), head_dim=hd,
                    n_ff=int(kv[a + "feed_forward_length"]), n_vocab=len(kv["tokenizer.ggml.tokens"]),
                    n_ctx=n_ctx, rms_eps=float(kv.get(a + "attention.layer_norm_rms_epsilon", 1e-6)),
                    rope_base=base, rope_base_swa=base_swa,
                    attn_scale=float(kv.get(a + "attention.scale", 1.0 / hd ** 0.5)),
                    window=window, swa_period=period, wtype=dtype)
    return cfg


class Gemma3:
    """Device weights of a Gemma-3 model (nncpu's Q8_0 or Q4 layout), plus
    the host copies (norms, the embedding table) the CPU forward reads."""

    def __init__(self, cfg: NngConfig, weights: list[Weight], norms: np.ndarray):
        self.cfg = cfg
        self.shapes = matrix_shapes(cfg)
        self.weights = weights
        self.norms = np.ascontiguousarray(norms, np.float32)
        self.token_embd = self.weights[-1].download()  # the tied embedding / lm_head table
        self._lib = _gemma_lib()

    @classmethod
    def from_gguf(cls, path: str, n_ctx: int = 256, dtype: int = Q8_0) -> "Gemma3":
        """Load a Gemma-3 GGUF as nncpu's loader does (model/load.rs:881-1288
        for the hyperparameters and names): every matrix decoded from its
        ggml type to f32 and re-encoded to `dtype` on the device
        (nnh_upload_gguf: load.rs:182-243 on the GPU), the norm vectors as
        f32, the lm_head tied to token_embd (model/mod.rs:366-372)."""
        from .gguf import GgufFile
        f = GgufFile(path)
        kv = f.kv
        if kv.get("general.architecture") != "gemma3":
            raise ValueError(f"{path}: not a gemma3 model")
        cfg = gemma3_config_from_kv(kv, n_ctx, dtype, path)

        def mat(name):
            t = f.tensors[name]
            return Weight.from_gguf(t.ggml_type, t.data, t.rows, t.cols, dtype)

        def vec(name):
            t = f.tensors[name]
            if t.ggml_type != 0:
                raise ValueError(f"{name}: norm vectors are read as F32")
            return np.asarray(t.data).view(np.float32)

        weights, norms = [], []
        for li in range(cfg.n_layer):
            b = f"blk.{li}."
            weights += [mat(b + n) for n in ("attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight",
                                              "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight")]
            norms += [vec(b + n) for n in ("attn_norm.weight", "attn_q_norm.weight", "attn_k_norm.weight",
                                            "post_attention_norm.weight", "ffn_norm.weight", "post_ffw_norm.weight")]
        weights.append(mat("token_embd.weight"))
        norms.append(vec("output_norm.weight"))
        return cls(cfg, weights, np.concatenate(norms))

    def generate(self, prompt: np.ndarray, n_gen: int, gemv_ptr: int, argmax_ptr: int | None, ctx,
                 batch: int = 16):
        """(tokens, per-layer hashes, prefill seconds, decode seconds)."""
        L = self._lib
        m = L.nng_create(C.byref(self.cfg), self.norms.ctypes.data_as(C.c_void_p),
                         self.token_embd.ctypes.data_as(C.c_void_p), gemv_ptr, argmax_ptr, C.cast(ctx, C.c_void_p))
        try:
            prompt = np.ascontiguousarray(prompt, np.int32)
            out = np.zeros(n_gen, np.int32)
            n_fwd = (len(prompt) + batch - 1) // batch + n_gen
            hashes = np.zeros(n_fwd * self.cfg.n_layer, np.uint64)
            nh, tp, td = C.c_size_t(), C.c_double(), C.c_double()
            rc = L.nng_generate(m, prompt.ctypes.data_as(C.c_void_p), len(prompt), batch, n_gen,
                                out.ctypes.data_as(C.c_void_p), hashes.ctypes.data_as(C.c_void_p), C.byref(nh),
                                C.byref(tp), C.byref(td))
            if rc != 0:
                raise RuntimeError(L.nng_error(m).decode())
            return out, hashes[:nh.value], tp.value, td.value
        finally:
            L.nng_free(m)

    def generate_gpu(self, prompt: np.ndarray, n_gen: int, act: int = ACT_F32):
        """The decode run with every matmul on the GPU."""
        arr = (C.c_void_p * len(self.weights))(*[w.handle for w in self.weights])
        ctx = NngGpuCtx(w=C.cast(arr, C.POINTER(C.c_void_p)), n=len(self.weights), act=act)
        self._keep = (arr, ctx)
        gemv = C.cast(self._lib.nng_gpu_gemv, C.c_void_p).value
        argmax = C.cast(self._lib.nng_gpu_argmax, C.c_void_p).value
        return self.generate(prompt, n_gen, gemv, argmax, C.pointer(ctx))

    def generate_device(self, prompt: np.ndarray, n_gen: int, batch: int = 16):
        """The prompt as in generate_gpu (CPU forward, GPU matmuls), then the
        decode resident on the GPU. (tokens, per-layer hashes, prefill
        seconds, decode seconds)."""
        import time
        L = self._lib
        arr = (C.c_void_p * len(self.weights))(*[w.handle for w in self.weights])
        ctx = NngGpuCtx(w=C.cast(arr, C.POINTER(C.c_void_p)), n=len(self.weights), act=ACT_F32)
        self._keep = (arr, ctx)
        gemv = C.cast(L.nng_gpu_gemv, C.c_void_p).value
        argmax = C.cast(L.nng_gpu_argmax, C.c_void_p).value
        m = L.nng_create(C.byref(self.cfg), self.norms.ctypes.data_as(C.c_void_p),
                         self.token_embd.ctypes.data_as(C.c_void_p), gemv, argmax, C.cast(C.pointer(ctx), C.c_void_p))
        try:
            t0 = time.perf_counter()
            prompt = np.ascontiguousarray(prompt, np.int32)
            last = 0
            for p in range(0, len(prompt), batch):
                n = min(batch, len(prompt) - p)
                if L.nng_forward(m, prompt[p:].ctypes.data_as(C.c_void_p), n):
                    raise RuntimeError(L.nng_error(m).decode())
                last = n
            tok = C.c_int32()
            if L.nng_argmax_last(m, last, C.byref(tok)):
                raise RuntimeError(L.nng_error(m).decode())
            t_prefill = time.perf_counter() - t0
            if getattr(self, "_dev", None) is None:
                md = C.c_void_p()
                rc = L.nngd_create(C.byref(self.cfg), self.norms.ctypes.data_as(C.c_void_p), arr, len(self.weights),
                                   max(n_gen, 1), C.byref(md))
                if rc:
                    msg = L.nngd_error(md).decode()
                    L.nngd_free(md)
                    raise RuntimeError(msg)
                self._dev = md
            E, nl = self.cfg.n_embd, self.cfg.n_layer
            out = np.zeros(n_gen, np.int32)
            record = np.zeros(max(n_gen - 1, 0) * nl * E, np.float32)
            secs = C.c_double()
            if L.nngd_decode(self._dev, m, tok.value, n_gen, out.ctypes.data_as(C.c_void_p),
                             record.ctypes.data_as(C.c_void_p), C.byref(secs)):
                raise RuntimeError(L.nngd_error(self._dev).decode())
            hp, nh = C.POINTER(C.c_uint64)(), C.c_size_t()
            L.nng_state(m, None, None, None, C.byref(hp), C.byref(nh))
            pre = np.ctypeslib.as_array(hp, shape=(nh.value,)).copy() if nh.value else np.zeros(0, np.uint64)
            dec = np.zeros(max(n_gen - 1, 0) * nl, np.uint64)
            L.nng_fnv_many(record.ctypes.data_as(C.c_void_p), E, len(dec), dec.ctypes.data_as(C.c_void_p))
            return out, np.concatenate([pre, dec]), t_prefill, secs.value
        finally:
            L.nng_free(m)

    def free(self):
        if getattr(self, "_dev", None) is not None:
            self._lib.nngd_free(self._dev)
            self._dev = None


def gemma3_1b_gguf(path: str | None = None, seed: int = 0x6E33A, n_ctx: int = 256, n_layer: int = 26,
                   n_vocab: int = 262144) -> str:
    """BASELINE config 1's model file: the Gemma-3-1B-architecture random-init
    GGUF from `seed` (nncpu_amd.gguf.write_gemma3, BF16 matrices), written to
    `path` (default: the temp directory) unless a file of that name exists."""
    import tempfile
    from .gguf import write_gemma3
    if path is None:
        path = os.path.join(tempfile.gettempdir(), f"nncpu-amd-gemma3-{n_layer}x{n_vocab}-{seed:x}.gguf")
    if not os.path.exists(path):
        tmp = path + f".tmp{os.getpid()}"
        write_gemma3(tmp, gemma3_1b_config(n_ctx=n_ctx, n_layer=n_layer, n_vocab=n_vocab), seed)
        os.replace(tmp, path)
    return path


def random_prompt(n: int, n_vocab: int, seed: int = 0x9A0) -> np.ndarray:
    """A uniform-random prompt of n token ids."""
    return np.random.default_rng(seed).integers(0, n_vocab, n).astype(np.int32)
