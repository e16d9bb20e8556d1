"""Gemma-3, Llama, Qwen2 and Qwen3 forward passes around the GPU matmul.

One model, two runs:

* `Model.cpu_generate`: the CPU forward of nncpu_amd/host/gemma3.cpp
  (crates/nncpu/src/model/forward.rs restated, for the four
  architectures: Qwen2's q/k/v biases, Qwen3's per-head q/k norms, SwiGLU,
  Llama's adjacent-pair RoPE)
  with every weight matmul through `nnh_gemv_batch`, the prompt in 16-token
  batches (session/engine.rs:362-380) and then greedy tokens;
* `DeviceForward`: the same forward resident on the GPU
  (nncpu_amd/host/layers_gpu.hip): norms, RoPE, the K/V cache, blockwise
  attention and the gated activations as HIP kernels with the CPU forward's
  arithmetic, every matmul through `nnh_gemv_batch_dev`. With the bit-exact
  f32 matmul both runs give the same tokens, per-layer hidden states and K/V
  cache bit for bit.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import ACT_F32, Q4S, Q8_0, Weight
from .gemma import NngConfig, NngGpuCtx, _gemma_lib, matrix_shapes

ARCH_GEMMA3, ARCH_LLAMA, ARCH_QWEN2, ARCH_QWEN3 = 0, 1, 2, 3
ROPE_NEOX, ROPE_NORM = 0, 1


def llama_config(n_layer: int, n_embd: int, n_head: int, n_kv: int, n_ff: int, n_vocab: int, n_ctx: int,
                 head_dim: int | None = None, rope_base: float = 500000.0, rms_eps: float = 1e-5,
                 wtype: int = Q8_0) -> NngConfig:
    """A Llama architecture (load.rs:538-566: adjacent-pair RoPE, attention
    scale 1/sqrt(head_dim), no embedding scale)."""
    hd = head_dim or n_embd // n_head
    return NngConfig(n_layer=n_layer, n_embd=n_embd, n_head=n_head, n_kv=n_kv, head_dim=hd, n_ff=n_ff,
                     n_vocab=n_vocab, n_ctx=n_ctx, rms_eps=rms_eps, rope_base=rope_base, rope_base_swa=rope_base,
                     attn_scale=float(np.float32(1.0) / np.sqrt(np.float32(hd))), window=0, swa_period=0,
                     wtype=wtype, arch=ARCH_LLAMA, rope_mode=ROPE_NORM)


def qwen2_config(n_layer: int, n_embd: int, n_head: int, n_kv: int, n_ff: int, n_vocab: int, n_ctx: int,
                 head_dim: int | None = None, rope_base: float = 1e6, rms_eps: float = 1e-6,
                 wtype: int = Q8_0) -> NngConfig:
    """A Qwen2 architecture (NeoX RoPE, q/k/v projection biases)."""
    cfg = llama_config(n_layer, n_embd, n_head, n_kv, n_ff, n_vocab, n_ctx, head_dim, rope_base, rms_eps, wtype)
    cfg.arch, cfg.rope_mode = ARCH_QWEN2, ROPE_NEOX
    return cfg


def qwen3_config(n_layer: int, n_embd: int, n_head: int, n_kv: int, n_ff: int, n_vocab: int, n_ctx: int,
                 head_dim: int | None = None, rope_base: float = 1e6, rms_eps: float = 1e-6,
                 wtype: int = Q8_0) -> NngConfig:
    """A Qwen3 architecture (NeoX RoPE, per-head q/k RMSNorm, no biases)."""
    cfg = llama_config(n_layer, n_embd, n_head, n_kv, n_ff, n_vocab, n_ctx, head_dim, rope_base, rms_eps, wtype)
    cfg.arch, cfg.rope_mode = ARCH_QWEN3, ROPE_NEOX
    return cfg


def qwen25_7b_config(n_ctx: int = 4096, n_layer: int = 28, wtype: int = Q8_0) -> NngConfig:
    """Qwen2.5-7B's architecture (d 3584, FFN 18944, 28 query / 4 KV heads of
    128, vocab 152064, RoPE base 1e6)."""
    return qwen2_config(n_layer, 3584, 28, 4, 18944, 152064, n_ctx, wtype=wtype)


def _lib():
    L = _gemma_lib()
    vp, sz, i32 = C.c_void_p, C.c_size_t, C.c_int
    L.nng_set_biases.argtypes, L.nng_set_biases.restype = [vp, vp], None
    L.nng_set_rope_freqs.argtypes, L.nng_set_rope_freqs.restype = [vp, vp], None
    L.nngl_create.argtypes = [C.POINTER(NngConfig), vp, vp, vp, vp, i32, vp, i32, i32, vp, C.POINTER(vp)]
    L.nngl_create.restype = i32
    L.nngl_free.argtypes, L.nngl_free.restype = [vp], None
    L.nngl_error.argtypes, L.nngl_error.restype = [vp], C.c_char_p
    L.nngl_forward.argtypes, L.nngl_forward.restype = [vp, vp, sz], i32
    L.nngl_forward_dev.argtypes, L.nngl_forward_dev.restype = [vp, vp, sz, sz], i32
    L.nngl_argmax_last.argtypes, L.nngl_argmax_last.restype = [vp, sz, C.POINTER(C.c_int32)], i32
    L.nngl_logits_last_dev.argtypes, L.nngl_logits_last_dev.restype = [vp, sz, vp], i32
    L.nngl_read.argtypes, L.nngl_read.restype = [vp, sz, vp, vp, vp, vp], i32
    L.nngl_pos.argtypes, L.nngl_pos.restype = [vp], sz
    L.nngl_set_pos.argtypes, L.nngl_set_pos.restype = [vp, sz], i32
    L.nngl_decode_step_dev.argtypes, L.nngl_decode_step_dev.restype = [vp, vp, vp], i32
    L.nngl_greedy_next_dev.argtypes, L.nngl_greedy_next_dev.restype = [vp, vp, vp, vp, vp], i32
    L.nngl_set_fused_quant.argtypes, L.nngl_set_fused_quant.restype = [vp, i32], i32
    L.nngl_set_fused_norm.argtypes, L.nngl_set_fused_norm.restype = [vp, i32], i32
    return L


def concat_rows(ws: list[Weight]) -> Weight:
    """One matrix of the rows of `ws` in order (the split layout's parts
    concatenated part by part): a fused [q; k; v] or [gate; up] as serving
    engines load them. Every row keeps its bytes, so its matmul bits too."""
    dtype, cols = ws[0].dtype, ws[0].cols()
    parts = []
    for w in ws:
        if w.dtype != dtype or w.cols() != cols:
            raise ValueError("concat_rows: matrices differ in format or width")
        d, n = w.download(), w.rows() * cols
        cuts = [n, n // 16] if dtype == Q8_0 else [n // 2, n // 16, n // 16]
        offs = np.cumsum([0] + cuts)
        parts.append([d[offs[i]:offs[i + 1]] for i in range(len(cuts))])
    data = np.concatenate([np.concatenate([p[i] for p in parts]) for i in range(len(parts[0]))])
    return Weight.from_split(dtype, data, sum(w.rows() for w in ws), cols)


def norm_stride(cfg: NngConfig) -> int:
    """Floats per layer in the norms array: attn, q, k, post_attn, ffn, post_ffw."""
    return 4 * cfg.n_embd + 2 * cfg.head_dim


class Model:
    """The device weights of one model (7 matrices per layer with nng_gemv_fn's
    ids, the lm_head last), its norm vectors (nng_create's layout), Qwen2's
    q/k/v biases and the embedding table (a Weight; the lm_head when tied)."""

    def __init__(self, cfg: NngConfig, weights: list[Weight], norms: np.ndarray, biases: np.ndarray | None = None,
                 embd: Weight | None = None, rope_ff: np.ndarray | None = None):
        self.cfg = cfg
        self.weights = weights
        self.norms = np.ascontiguousarray(norms, np.float32)
        self.biases = None if biases is None else np.ascontiguousarray(biases, np.float32)
        self.embd = embd if embd is not None else weights[-1]
        self.rope_ff = None if rope_ff is None else np.ascontiguousarray(rope_ff, np.float32)
        self._lib = _lib()

    @classmethod
    def random(cls, cfg: NngConfig, seed: int = 0x11A, dtype: int = Q8_0, tied: bool = True) -> "Model":
        """Random-init weights 0.02*N(0,1) (torch's generator on the GPU, then
        nncpu's encoder on the device), norms 1 + 0.1*N(0,1), Qwen2 biases
        0.02*N(0,1); the embedding table is the lm_head when `tied`."""
        import torch
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)

        def mat(rows, cols):
            w = torch.randn(rows * cols, generator=g, device="cuda").mul_(0.02)
            torch.cuda.synchronize()
            out = Weight.encode_dev(dtype, w.data_ptr(), rows, cols)
            del w
            return out

        weights = [mat(r, c) for r, c in matrix_shapes(cfg)]
        rng = np.random.default_rng(seed)
        norms = (1.0 + 0.1 * rng.standard_normal(norm_stride(cfg) * cfg.n_layer + cfg.n_embd)).astype(np.float32)
        biases = None
        if cfg.arch == ARCH_QWEN2:
            per = (cfg.n_head + 2 * cfg.n_kv) * cfg.head_dim
            biases = (0.02 * rng.standard_normal(per * cfg.n_layer)).astype(np.float32)
        embd = None if tied else mat(cfg.n_vocab, cfg.n_embd)
        cfg.wtype = 2 if dtype == Q4S else Q8_0
        return cls(cfg, weights, norms, biases, embd)

    def cpu_generate(self, prompt: np.ndarray, n_gen: int, batch: int = 16, act: int = ACT_F32):
        """The CPU forward with GPU matmuls: (tokens, per-layer hashes of each
        forward, K cache, V cache) (the caches as [n_layer][n_ctx][kv_dim] BF16)."""
        L = self._lib
        arr = (C.c_void_p * len(self.weights))(*[w.handle for w in self.weights])
        ctx = NngGpuCtx(w=C.cast(arr, C.POINTER(C.c_void_p)), n=len(self.weights), act=act)
        table = self.embd.download()
        gemv = C.cast(L.nng_gpu_gemv, C.c_void_p).value
        argmax = C.cast(L.nng_gpu_argmax, C.c_void_p).value
        m = L.nng_create(C.byref(self.cfg), self.norms.ctypes.data_as(C.c_void_p),
                         table.ctypes.data_as(C.c_void_p), gemv, argmax, C.cast(C.pointer(ctx), C.c_void_p))
        try:
            if self.biases is not None:
                L.nng_set_biases(m, self.biases.ctypes.data_as(C.c_void_p))
            if self.rope_ff is not None:
                L.nng_set_rope_freqs(m, self.rope_ff.ctypes.data_as(C.c_void_p))
            prompt = np.ascontiguousarray(prompt, np.int32)
            out = np.zeros(n_gen, np.int32)
            n_fwd = (len(prompt) + batch - 1) // batch + n_gen
            hashes = np.zeros(n_fwd * self.cfg.n_layer, np.uint64)
            nh, tp, td = C.c_size_t(), C.c_double(), C.c_double()
            if L.nng_generate(m, prompt.ctypes.data_as(C.c_void_p), len(prompt), batch, n_gen,
                              out.ctypes.data_as(C.c_void_p), hashes.ctypes.data_as(C.c_void_p), C.byref(nh),
                              C.byref(tp), C.byref(td)):
                raise RuntimeError(L.nng_error(m).decode())
            kp, vp = C.POINTER(C.c_uint16)(), C.POINTER(C.c_uint16)()
            L.nng_state(m, C.byref(kp), C.byref(vp), None, None, None)
            n = self.cfg.n_layer * self.cfg.n_ctx * self.cfg.n_kv * self.cfg.head_dim
            kc = np.ctypeslib.as_array(kp, shape=(n,)).copy()
            vc = np.ctypeslib.as_array(vp, shape=(n,)).copy()
            return out, hashes[:nh.value], kc, vc
        finally:
            L.nng_free(m)

    def fused_weights(self) -> list:
        """The weight list with [q; k; v] and [gate; up] fused (k, v, up None)."""
        out = list(self.weights)
        for li in range(self.cfg.n_layer):
            b = 7 * li
            out[b] = concat_rows(self.weights[b:b + 3])
            out[b + 1] = out[b + 2] = None
            out[b + 4] = concat_rows(self.weights[b + 4:b + 6])
            out[b + 5] = None
        return out

    def device(self, n_batch: int = 16, act: int = ACT_F32, stream: int = 0, fused: bool = False) -> "DeviceForward":
        w = self.fused_weights() if fused else self.weights
        return DeviceForward(self.cfg, w, self.norms, self.biases, self.embd, n_batch, act, stream, self.rope_ff)


class DeviceForward:
    """The forward resident on the GPU (nngl_*): weights as Model's (k, v None
    for a fused [q; k; v] matrix at q's id, up None for a fused [gate; up] at
    gate's), n_batch the most tokens per forward, act the matmuls' mode."""

    def __init__(self, cfg: NngConfig, weights: list, norms: np.ndarray, biases: np.ndarray | None, embd: Weight,
                 n_batch: int = 16, act: int = ACT_F32, stream: int = 0, rope_ff: np.ndarray | None = None):
        self.cfg = cfg
        self._lib = L = _lib()
        self._w = weights
        self._arr = (C.c_void_p * len(weights))(*[(w.handle if w is not None else None) for w in weights])
        self._norms = np.ascontiguousarray(norms, np.float32)
        self._bias = None if biases is None else np.ascontiguousarray(biases, np.float32)
        self._ff = None if rope_ff is None else np.ascontiguousarray(rope_ff, np.float32)
        self._embd = embd
        self.n_batch = n_batch
        h = C.c_void_p()
        rc = L.nngl_create(C.byref(cfg), self._norms.ctypes.data_as(C.c_void_p),
                           None if self._bias is None else self._bias.ctypes.data_as(C.c_void_p),
                           None if self._ff is None else self._ff.ctypes.data_as(C.c_void_p),
                           self._arr, len(weights), embd.handle, n_batch, act, stream or None, C.byref(h))
        self._h = h
        if rc:
            msg = L.nngl_error(h).decode()
            self.free()
            raise RuntimeError(msg)

    def _check(self, rc: int) -> None:
        if rc:
            raise RuntimeError(self._lib.nngl_error(self._h).decode())

    def forward(self, tokens: np.ndarray) -> None:
        t = np.ascontiguousarray(tokens, np.int32)
        self._check(self._lib.nngl_forward(self._h, t.ctypes.data_as(C.c_void_p), len(t)))

    def forward_dev(self, tokens_ptr: int, n_tok: int, pos0: int) -> None:
        self._check(self._lib.nngl_forward_dev(self._h, tokens_ptr, n_tok, pos0))

    def logits_last_dev(self, n_tok: int, logits_ptr: int) -> None:
        self._check(self._lib.nngl_logits_last_dev(self._h, n_tok, logits_ptr))

    def argmax_last(self, n_tok: int) -> int:
        out = C.c_int32()
        self._check(self._lib.nngl_argmax_last(self._h, n_tok, C.byref(out)))
        return out.value

    def read(self, n_tok: int = 0, caches: bool = False):
        """(final hidden states [n_tok][E], per-layer states [n_layer][E], and
        with `caches` the K and V caches)."""
        c = self.cfg
        hid = np.zeros((n_tok, c.n_embd), np.float32)
        st = np.zeros((c.n_layer, c.n_embd), np.float32)
        n = c.n_layer * c.n_ctx * c.n_kv * c.head_dim
        kc = np.zeros(n, np.uint16) if caches else None
        vc = np.zeros(n, np.uint16) if caches else None
        p = lambda a: None if a is None else a.ctypes.data_as(C.c_void_p)  # noqa: E731
        self._check(self._lib.nngl_read(self._h, n_tok, p(hid) if n_tok else None, p(st), p(kc), p(vc)))
        return (hid, st, kc, vc) if caches else (hid, st)

    def set_fused_quant(self, on: bool) -> None:
        """One-token int8 forwards: the kernels producing each matmul input
        write it quantized (default, same bits), or the matmuls quantize."""
        self._check(self._lib.nngl_set_fused_quant(self._h, int(bool(on))))

    def set_fused_norm(self, on: bool) -> None:
        """One-token f32 forwards with fused matrices: the residual add and
        RMSNorm in the next matmul's prologue (the default) or as a kernel of
        their own (False); the same bits either way."""
        self._check(self._lib.nngl_set_fused_norm(self._h, int(bool(on))))

    def set_pos(self, pos: int) -> None:
        self._check(self._lib.nngl_set_pos(self._h, pos))

    def generate(self, prompt: np.ndarray, n_gen: int, batch: int = 16):
        """cpu_generate's run on the device: (tokens, per-layer hashes of each
        forward, K cache, V cache)."""
        self.set_pos(0)
        prompt = np.ascontiguousarray(prompt, np.int32)
        E, nl = self.cfg.n_embd, self.cfg.n_layer
        hashes = []

        def record():
            _, st = self.read()
            h = np.zeros(nl, np.uint64)
            self._lib.nng_fnv_many(st.ctypes.data_as(C.c_void_p), E, nl, h.ctypes.data_as(C.c_void_p))
            hashes.append(h)

        last = 0
        for p in range(0, len(prompt), batch):
            chunk = prompt[p:p + batch]
            self.forward(chunk)
            record()
            last = len(chunk)
        out = np.zeros(n_gen, np.int32)
        tok = self.argmax_last(last)
        for g in range(n_gen):
            out[g] = tok
            if g + 1 == n_gen:
                break
            self.forward(np.array([tok], np.int32))
            record()
            tok = self.argmax_last(1)
        _, _, kc, vc = self.read(0, caches=True)
        return out, np.concatenate(hashes) if hashes else np.zeros(0, np.uint64), kc, vc

    def generate_graph(self, prompt: np.ndarray, n_gen: int, batch: int = 16, stream=None):
        """The prompt as in `generate`, then the greedy decode with one step
        (nngl_decode_step_dev + nngl_greedy_next_dev: the token, position and
        step counter in device memory) captured in a HIP graph on the model's
        stream (`stream`, the torch stream it was created on) and replayed per
        token. (tokens, decode seconds, K cache, V cache)."""
        import time

        import torch
        self.set_pos(0)
        prompt = np.ascontiguousarray(prompt, np.int32)
        if len(prompt) + n_gen > self.cfg.n_ctx:
            raise ValueError("the prompt and the generated tokens exceed the context")
        last = 0
        for p in range(0, len(prompt), batch):
            chunk = prompt[p:p + batch]
            self.forward(chunk)
            last = len(chunk)
        first = self.argmax_last(last)
        dev = "cuda"
        tok = torch.tensor([first], dtype=torch.int32, device=dev)
        pos = torch.tensor([len(prompt)], dtype=torch.int32, device=dev)
        step = torch.tensor([1], dtype=torch.int32, device=dev)
        out = torch.zeros(n_gen, dtype=torch.int32, device=dev)
        out[0] = first
        torch.cuda.synchronize()
        L = self._lib

        def one():
            self._check(L.nngl_decode_step_dev(self._h, tok.data_ptr(), pos.data_ptr()))
            self._check(L.nngl_greedy_next_dev(self._h, tok.data_ptr(), pos.data_ptr(), out.data_ptr(),
                                               step.data_ptr()))

        secs = 0.0
        if n_gen > 1:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                one()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(n_gen - 1):
                g.replay()
            torch.cuda.synchronize()
            secs = time.perf_counter() - t0
            del g
        toks = out.cpu().numpy()
        _, _, kc, vc = self.read(0, caches=True)
        return toks, secs, kc, vc

    def free(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            self._lib.nngl_free(self._h)
        self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
