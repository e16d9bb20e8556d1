"""Benchmark: nncpu's quantized matmul on one MI355X.

Default workload: the 4-bit GEMV sweep at
Llama-3-8B projection shapes (N x K = 4096x4096, 1024x4096, 14336x4096,
4096x14336), M = 1, weights 0.02*N(0,1) re-encoded to nncpu's Q4 layout,
activations N(0,1) quantized on the device to int8 blocks (nncpu's Q8_0
encoder). One step = one GEMV per shape. Inputs are resident in HBM; each
shape cycles through enough uploaded weight copies (>= 512 MB, twice the
MI355X Infinity Cache) that every launch streams its weights from HBM.

value = algorithmic bytes of the timed steps / wall time between the two
synchronised events (GB/s); bytes per GEMV = N*K/2 + N*K/16 (quants, BF16
scales and biases) + 4K + 4N (f32 x in, f32 y out), the reference's own
byte accounting plus the vectors.

    python bench.py [--gpus 1] [--steps 1000] [--warmup 50] [--workload q4_sweep]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
ROTATE_BYTES = 512 << 20

Q4_SWEEP = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]
# HBM bytes per launch of the sweep's GEMVs, from rocprofv3 --pmc FETCH_SIZE
# (x2.0, the factor a 64 MiB device copy gives) + WRITE_SIZE, in the order of
# Q4_SWEEP; the runs are in profiles/gemv_i8_q4_llama3_8b_sweep.md.
Q4_SWEEP_TRAFFIC = [10_603_212, 2_713_600, 36_853_350, 36_929_126]
Q8_VOCAB = [(262144, 1152), (151936, 3584)]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def weight_bytes(dtype: int, n: int, k: int) -> int:
    """model/mod.rs:391-398: what a gemv streams from the weight."""
    e = n * k
    if dtype == 3:
        return 2 * e
    return e + e // 16 if dtype == 1 else e // 2 + e // 8


def gemv_bytes(dtype: int, n: int, k: int, m: int = 1) -> int:
    return weight_bytes(dtype, n, k) + 4 * k * m + 4 * n * m


def make_weights(N, dtype: int, n: int, k: int, seed: int, copies: int, stream: int = 0):
    """`copies` device weights of 0.02*N(0,1) values (a seeded torch
    generator on the GPU), each re-encoded by the library's device encoder,
    which is nncpu's load-time encoder bit for bit."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    w = torch.randn(n * k, generator=g, device="cuda", dtype=torch.float32).mul_(0.02)
    torch.cuda.synchronize()
    ws = [N.Weight.encode_dev(dtype, w.data_ptr(), n, k, stream) for _ in range(copies)]
    del w
    return ws


def make_x(k: int, m: int, seed: int):
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return torch.randn(m * k, generator=g, device="cuda", dtype=torch.float32)


class Stream:
    def __init__(self):
        import torch
        self.torch = torch
        self.s = torch.cuda.Stream()
        self.handle = self.s.cuda_stream

    def event(self):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record(self.s)
        return e


def time_gemv_set(N, st, launches, steps, warmup):
    """Run `launches` (a list of callables, one step) `warmup` times eagerly,
    then capture `steps` steps in one HIP graph (host launch cost would
    otherwise exceed these microsecond kernels) and time its replay between
    two events on the launch stream, synchronised on both sides."""
    torch = st.torch
    for _ in range(warmup):
        for f in launches:
            f()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st.s):
        for _ in range(steps):
            for f in launches:
                f()
    torch.cuda.synchronize()
    g.replay()  # first replay uploads the graph
    torch.cuda.synchronize()
    e0 = st.event()
    with torch.cuda.stream(st.s):
        g.replay()
    e1 = st.event()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3


def q4_sweep(args, N):
    import torch
    st = Stream()
    shapes = Q4_SWEEP
    per_shape = []
    inputs = []
    all_launch = []
    keep = []
    total_bytes_step = 0
    for i, (n, k) in enumerate(shapes):
        wb = weight_bytes(2, n, k)
        copies = max(2, math.ceil(ROTATE_BYTES / wb))
        ws = make_weights(N, 2, n, k, 0x5EED01 + i, copies)
        x = make_x(k, 1, 0xA11 + i)
        _, _, abytes = N.act_layout(k, 1)
        act = torch.zeros(abytes, dtype=torch.uint8, device="cuda")
        N.quantize_act_dev(x.data_ptr(), k, k, 1, act.data_ptr(), st.handle)
        y = torch.zeros(n, dtype=torch.float32, device="cuda")
        keep += [ws, x, act, y]
        state = {"i": 0}

        def launch(ws=ws, act=act, y=y, state=state):
            w = ws[state["i"] % len(ws)]
            state["i"] += 1
            N.gemv_i8_dev(w, act.data_ptr(), 1, y.data_ptr(), n, st.handle)

        all_launch.append(launch)
        total_bytes_step += gemv_bytes(2, n, k)
        per_shape.append(dict(shape=f"{n}x{k}", copies=copies, bytes=gemv_bytes(2, n, k), launch=launch))
        inputs.append((ws[0], act, k))
        log(f"shape {n}x{k}: {copies} copies of {wb / 1e6:.1f} MB")
    torch.cuda.synchronize()

    # Per-shape timing (each shape alone, back to back).
    for p in per_shape:
        secs = time_gemv_set(N, st, [p["launch"]], args.steps, args.warmup)
        p["us"] = secs / args.steps * 1e6
        p["gbs"] = p["bytes"] / (secs / args.steps) / 1e9
        p["hbm_frac"] = p["gbs"] / HBM_PEAK_GBS
        log(f"{p['shape']}: {p['us']:.2f} us/launch, {p['gbs']:.0f} GB/s ({100 * p['hbm_frac']:.1f}% of HBM)")
        del p["launch"]

    # The sweep: one step = the four GEMVs; barrier + sync on both sides.
    secs = time_gemv_set(N, st, all_launch, args.steps, args.warmup)
    value = total_bytes_step * args.steps / secs / 1e9
    kernel_us = sum(p["us"] for p in per_shape) / len(per_shape)
    bytes_per_launch = total_bytes_step / len(shapes)
    achieved = bytes_per_launch / (kernel_us * 1e-6) / 1e9
    result = dict(
        metric="quantized GEMV GB/s (% HBM peak); int8 GEMM TOPS; batch-1 decode tok/s",
        value=round(value, 1), unit="GB/s", ms_per_step=secs / args.steps * 1e3, dtype="i8",
        config=dict(workload="q4_gemv_llama3_8b_sweep_m1", shapes=[p["shape"] for p in per_shape], m=1,
                    weights="0.02*N(0,1), nncpu Q4 (per-32 BF16 scale+bias)",
                    activations="N(0,1) f32 -> int8 blocks (nncpu Q8_0) on device", parallelism="none",
                    rotate_mb=ROTATE_BYTES >> 20),
        roofline=dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                      frac=round(achieved / HBM_PEAK_GBS, 4),
                      traffic=round(sum(Q4_SWEEP_TRAFFIC) / len(Q4_SWEEP_TRAFFIC)),
                      kernel="gemv_i8_v2_kernel (Q4, M=1)", bytes_per_launch=bytes_per_launch,
                      avg_launch_us=round(kernel_us, 3)),
        per_shape=[{k: (round(v, 4) if isinstance(v, float) else v) for k, v in p.items()} for p in per_shape],
    )
    return result, inputs


QWEN_PREFILL = [(3584, 3584), (512, 3584), (18944, 3584), (3584, 18944)]  # q/o, k/v, gate/up, down
VERIFY_SHAPES = [(6144, 1536), (1536, 6144), (2048, 1536), (1536, 1536)]
GEMMA_DECODE = [(1024, 1152), (256, 1152), (1152, 1024), (6912, 1152), (1152, 6912), (262144, 1152)]
# BF16 weights: the reference's own BF16 test shapes (Gemma E2B/E4B, kernels/tests.rs:435-447) and
# Llama-3-8B projections.
BF16_SHAPES = [(1536, 1536), (2048, 1536), (6144, 1536), (4096, 4096), (14336, 4096)]


def measure_cases(args, N, cases, act_mode, label):
    """Time each (dtype, n, k, m) case alone: `args.steps` launches captured in
    a graph over rotating weight copies (>= 512 MB), inputs resident in HBM.
    act_mode: ACT_I8 / ACT_MXI8 time the int8 matmul on activations
    quantized beforehand (nncpu's Q8_0 encoder / power-of-two MX blocks);
    ACT_F32 times the bit-exact f32 path (block sums included for Q4)."""
    import torch
    st = Stream()
    out = []
    for ci, (dtype, n, k, m) in enumerate(cases):
        wb = weight_bytes(dtype, n, k)
        copies = max(2, math.ceil(ROTATE_BYTES / wb))
        ws = make_weights(N, dtype, n, k, 0x5EED10 + 7 * ci + dtype, copies)
        x = make_x(k, m, 0xA11 + ci)
        y = torch.zeros(m * n, dtype=torch.float32, device="cuda")
        qmode = act_mode if act_mode != N.ACT_F32 else N.ACT_I8
        _, _, abytes = N.act_layout_ex(qmode, k, m)
        act = torch.zeros(abytes, dtype=torch.uint8, device="cuda")
        N.quantize_act_ex_dev(qmode, x.data_ptr(), k, k, m, act.data_ptr(), st.handle)
        state = {"i": 0}

        def launch(ws=ws, state=state, act=act, x=x, y=y, n=n, k=k, m=m):
            w = ws[state["i"] % len(ws)]
            state["i"] += 1
            if act_mode != N.ACT_F32:
                N.gemv_act_dev(w, act_mode, act.data_ptr(), m, y.data_ptr(), n, st.handle)
            else:
                N.gemv_batch_dev(w, x.data_ptr(), k, y.data_ptr(), n, m, N.ACT_F32, st.handle)

        torch.cuda.synchronize()
        steps = max(10, min(args.steps, int(2e5 / max(1.0, wb / 1e6))))  # bound the timed work
        secs = time_gemv_set(N, st, [launch], steps, min(args.warmup, 10))
        us = secs / steps * 1e6
        byts = gemv_bytes(dtype, n, k, m)
        ops = 2.0 * m * n * k
        e = dict(case=f"{ {1: 'Q8', 2: 'Q4', 3: 'BF16'}[dtype]} {n}x{k} M={m}", us=round(us, 3),
                 gbs=round(byts / us / 1e3, 1), hbm_frac=round(byts / us / 1e3 / HBM_PEAK_GBS, 4),
                 tops=round(ops / us / 1e6, 2), int8_frac=round(ops / us / 1e6 / INT8_PEAK_TOPS, 4), steps=steps)
        log(f"{label}: {e}")
        out.append(e)
        del ws
        torch.cuda.synchronize()
    return out


def qwen_prefill(args, N, dtype: int, act: int, n_tok: int = 512, n_layer: int = 28):
    """BASELINE configs[4], end to end: a Qwen2.5-7B-shaped model (d 3584,
    FFN 18944, 28 query / 4 KV heads of 128, RoPE base 1e6, RMSNorm, SwiGLU,
    q/k/v biases) with random weights 0.02*N(0,1) encoded by the library's
    device encoder (nncpu Q8_0 / Q4), prefilling 512 tokens of random
    embeddings through all 28 layers and the last token's lm_head row
    (152064 x 3584). Every weight matmul is the library's int8 path in mode
    `act` (activations quantized on the device: nncpu's Q8_0 encoder and the
    int8 MFMA GEMM, or MX blocks and the BF16-MFMA GEMM); q/k/v and gate/up are
    uploaded as one concatenated matrix each, as serving engines load them.
    The rest of the layer (norms, RoPE, causal GQA attention, SiLU) is torch
    float32 on the GPU: harness, not the measured path. One step = one full
    prefill; returns ms and tokens/s, plus the matmul share from HIP events."""
    import torch
    import torch.nn.functional as F
    d, ff, nh, nkv, hd, vocab = 3584, 18944, 28, 4, 128, 152064
    dev = "cuda"
    st = Stream()
    g = torch.Generator(device=dev)
    g.manual_seed(0x9E11 + dtype)

    def weight(rows, cols):
        w = torch.randn(rows * cols, generator=g, device=dev).mul_(0.02)
        torch.cuda.synchronize()
        out = N.Weight.encode_dev(dtype, w.data_ptr(), rows, cols)
        del w
        return out

    layers = []
    for _ in range(n_layer):
        layers.append(dict(
            qkv=weight(d + 2 * nkv * hd, d), o=weight(d, d), gu=weight(2 * ff, d), down=weight(d, ff),
            bqkv=torch.randn(d + 2 * nkv * hd, generator=g, device=dev).mul_(0.02),
            n1=1.0 + 0.1 * torch.randn(d, generator=g, device=dev),
            n2=1.0 + 0.1 * torch.randn(d, generator=g, device=dev)))
    lm_head = weight(vocab, d)
    norm_f = 1.0 + 0.1 * torch.randn(d, generator=g, device=dev)
    x0 = torch.randn(n_tok, d, generator=g, device=dev)
    pos = torch.arange(n_tok, device=dev, dtype=torch.float32)
    inv = 1.0 / (1e6 ** (torch.arange(0, hd, 2, device=dev, dtype=torch.float32) / hd))
    ang = pos[:, None] * inv[None, :]
    cos, sin = torch.cos(ang), torch.sin(ang)
    mm_events = []

    def mm(w, x, rows):
        y = torch.empty(x.shape[0], rows, device=dev)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(st.s)
        N.gemv_batch_dev(w, x.data_ptr(), x.shape[1], y.data_ptr(), rows, x.shape[0], act, st.handle)
        e1.record(st.s)
        mm_events.append((e0, e1))
        return y

    def rms(x, wgt):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * wgt

    def rope(t):  # t [tokens, heads, hd], NeoX halves
        a, b = t[..., :hd // 2], t[..., hd // 2:]
        c, s_ = cos[:, None, :], sin[:, None, :]
        return torch.cat([a * c - b * s_, b * c + a * s_], dim=-1)

    def forward():
        x = x0.clone()
        for L in layers:
            h = rms(x, L["n1"]).contiguous()
            qkv = mm(L["qkv"], h, d + 2 * nkv * hd) + L["bqkv"]
            q = rope(qkv[:, :d].view(n_tok, nh, hd))
            k = rope(qkv[:, d:d + nkv * hd].view(n_tok, nkv, hd))
            v = qkv[:, d + nkv * hd:].view(n_tok, nkv, hd)
            k = k.repeat_interleave(nh // nkv, dim=1)
            v = v.repeat_interleave(nh // nkv, dim=1)
            a = F.scaled_dot_product_attention(q.transpose(0, 1).contiguous(), k.transpose(0, 1).contiguous(),
                                               v.transpose(0, 1).contiguous(), is_causal=True)
            a = a.transpose(0, 1).reshape(n_tok, d).contiguous()
            x = x + mm(L["o"], a, d)
            h = rms(x, L["n2"]).contiguous()
            gu = mm(L["gu"], h, 2 * ff)
            x = x + mm(L["down"], (F.silu(gu[:, :ff]) * gu[:, ff:]).contiguous(), d)
        last = rms(x[-1:], norm_f).contiguous()
        return mm(lm_head, last, vocab)

    with torch.cuda.stream(st.s):
        for _ in range(2):
            forward()
        torch.cuda.synchronize()
        mm_events.clear()
        steps = max(1, min(args.steps, 5))
        e0 = st.event()
        for _ in range(steps):
            logits = forward()
        e1 = st.event()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    mm_ms = sum(a.elapsed_time(b) for a, b in mm_events) / steps
    per_layer = 2 * n_tok * d * ((d + 2 * nkv * hd) + d + 2 * ff + ff)
    ops = n_layer * per_layer + 2 * d * vocab
    assert torch.isfinite(logits).all()
    res = dict(case=f"{'Q8' if dtype == 1 else 'Q4'} Qwen2.5-7B-shaped prefill, {n_layer} layers, {n_tok} tokens",
               activations="MX int8 blocks (power-of-two scales)" if act == N.ACT_MXI8 else "int8 blocks (nncpu Q8_0)",
               ms=round(ms, 3), tokens_per_s=round(n_tok / ms * 1e3, 1), matmul_ms=round(mm_ms, 3),
               matmul_tops=round(ops / mm_ms / 1e9, 1), steps=steps)
    log(f"qwen_prefill: {res}")
    for L in layers:
        for key in ("qkv", "o", "gu", "down"):
            L[key].free()
    lm_head.free()
    return res


def cpu_baseline_q4(N, O, inputs, budget_s=12.0):
    """nncpu's AVX2 kernels (restated, oracle/avx2.cpp) on this host's cores,
    on the same weights (downloaded from the GPU) and the same quantized
    activations (dequantized: the values nncpu's f32 kernel would be fed),
    rotating >= 256 MB of weight copies as the reference's bench_gemv does;
    best of 3 passes after a warm-up."""
    if not O.avx_available():
        return None
    threads = min(8, os.cpu_count() or 1)
    O.avx_set_threads(threads)
    tot_bytes, tot_secs, sample = 0, 0.0, []
    t_start = time.time()
    for w, act, k in inputs:
        n = w.rows()
        m = O.QMatrix.from_split(2, n, k, w.download())
        copies = max(2, math.ceil((256 << 20) / weight_bytes(2, n, k)))
        mats = [m] + [O.QMatrix(2, n, k, tuple(p.copy() for p in m.parts)) for _ in range(copies - 1)]
        off_s, _, _ = N.act_layout(k, 1)
        a = act.cpu().numpy()
        xd = O.dequant_act(a[:k].view(np.int8), a[off_s:off_s + k // 16].view(np.uint16))
        best = float("inf")
        for rep in range(4):
            t0 = time.perf_counter()
            for mm in mats:
                O.gemv_batch(mm, xd, backend="avx2")
            dt = (time.perf_counter() - t0) / len(mats)
            if rep > 0:
                best = min(best, dt)
        tot_bytes += gemv_bytes(2, n, k)
        tot_secs += best
        sample.append(f"{n}x{k}:{gemv_bytes(2, n, k) / best / 1e9:.1f}GB/s")
        del mats
        if time.time() - t_start > budget_s:
            break
    gbs = tot_bytes / tot_secs / 1e9
    return dict(value=round(gbs, 2), unit="GB/s", cores=threads, kind="port",
                sample="Q4 GEMV M=1 at " + ", ".join(sample) + f"; {threads} threads (nncpu default min(8, CPUs)), "
                "AVX2 restatement of q4_rows_raw on the same weights and dequantized int8 activations, "
                ">=256 MB rotation, best of 3",
                host_stream_gbs_1thread=round(O.avx_stream_gbs(256 << 20, 2), 1))


def gemma_decode(args, N, cpu: bool):
    """Gemma-3-1B-shaped greedy decode of 128 tokens from a
    32-token prompt, on the device-resident step (seeded random Q8_0 weights).
    tok/s counts the 127 decode forwards after the prompt; the timed run is
    the second one (the first captures the step's graph). With `cpu`, the CPU
    baseline leg: the same decode with nncpu's CPU gemv (the oracle's AVX2
    restatement, 8 threads) in the shared C++ forward, timed, and its tokens
    compared with the device run's."""
    import ctypes as C
    from nncpu_amd.gemma import Gemma3, gemma3_1b_config, random_prompt
    t0 = time.perf_counter()
    m = Gemma3(gemma3_1b_config(n_ctx=256))
    log(f"gemma3-1b model built in {time.perf_counter() - t0:.1f}s")
    prompt, n_gen = random_prompt(32, m.cfg.n_vocab), 128
    m.generate_device(prompt, n_gen)
    tg, hg, tp, td = m.generate_device(prompt, n_gen)
    out = dict(config="gemma-3-1b architecture, Q8_0 weights 0.02*N(0,1), 32-token prompt, 128 greedy tokens",
               tok_s=round((n_gen - 1) / td, 1), ms_per_token=round(td / (n_gen - 1) * 1e3, 4),
               prefill_s=round(tp, 4), kernels_per_token=5 * m.cfg.n_layer + 4)
    log(f"gemma3-1b device decode: {out['tok_s']} tok/s")
    if cpu:
        from oracle import oracle as O  # the CPU baseline leg only

        class Table(C.Structure):
            _fields_ = [("n", C.c_int), ("dtype", C.c_int), ("bufs", C.POINTER(C.c_void_p)),
                        ("rows", C.POINTER(C.c_size_t)), ("cols", C.POINTER(C.c_size_t))]
        bufs = [w.download() for w in m.weights]
        arr = (C.c_void_p * len(bufs))(*[b.ctypes.data for b in bufs])
        rows = (C.c_size_t * len(bufs))(*[r for r, _ in m.shapes])
        cols = (C.c_size_t * len(bufs))(*[c for _, c in m.shapes])
        table = Table(n=len(bufs), dtype=1, bufs=C.cast(arr, C.POINTER(C.c_void_p)),
                      rows=C.cast(rows, C.POINTER(C.c_size_t)), cols=C.cast(cols, C.POINTER(C.c_size_t)))
        threads = 8
        O.avx_set_threads(threads)
        gemv = C.cast(O.lib().or_model_gemv_cb, C.c_void_p).value
        tc, hc, _, tdc = m.generate(prompt, n_gen, gemv, None, C.pointer(table))
        out["cpu_baseline"] = dict(tok_s=round((n_gen - 1) / tdc, 1), cores=threads, kind="port",
                                   sample="the same decode, CPU gemv (AVX2 restatement of nncpu's) in the shared "
                                          "C++ forward",
                                   tokens_identical=bool(np.array_equal(tg, tc)),
                                   layer_states_identical=bool(np.array_equal(hg, hc)))
        log(f"gemma3-1b cpu decode: {out['cpu_baseline']}")
    m.free()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default="q4_sweep",
                    choices=["q4_sweep", "prefill", "qwen_prefill", "q8_vocab", "verify", "decode_f32", "gemma_decode",
                             "bf16", "all"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build targets one GPU; --gpus {args.gpus} is not supported "
              "(across GPUs the path shards by rows: each GPU a row slice of every matrix, then an all-gather of y)", file=sys.stderr)
        sys.exit(2)
    import torch
    import nncpu_amd as N
    N.init(0)
    torch.cuda.set_device(0)
    extra = {}
    if args.workload in ("prefill", "all"):
        extra["prefill_m512_mx"] = measure_cases(args, N, [(d, n, k, 512) for d in (1, 2) for n, k in QWEN_PREFILL],
                                                 N.ACT_MXI8, "prefill_mx")
        extra["prefill_m512"] = measure_cases(args, N, [(d, n, k, 512) for d in (1, 2) for n, k in QWEN_PREFILL],
                                              N.ACT_I8, "prefill")
    if args.workload in ("qwen_prefill", "all"):
        extra["qwen_prefill_e2e"] = [qwen_prefill(args, N, d, a) for d in (1, 2) for a in (N.ACT_MXI8, N.ACT_I8)]
    if args.workload in ("q8_vocab", "all"):
        extra["q8_vocab_m1"] = measure_cases(args, N, [(1, n, k, 1) for n, k in Q8_VOCAB], N.ACT_I8, "q8_vocab")
    if args.workload in ("verify", "all"):
        extra["verify"] = measure_cases(args, N, [(d, n, k, m) for d in (1, 2) for n, k in VERIFY_SHAPES[:2]
                                                     for m in (2, 4, 8, 16)], N.ACT_I8, "verify")
    if args.workload in ("decode_f32", "all"):
        extra["decode_f32_bit_exact"] = measure_cases(args, N, [(d, n, k, 1) for d in (1, 2) for n, k in GEMMA_DECODE],
                                                      N.ACT_F32, "decode_f32")
    if args.workload in ("bf16", "all"):
        extra["bf16_bit_exact"] = measure_cases(args, N, [(3, n, k, m) for n, k in BF16_SHAPES for m in (1, 4)],
                                                N.ACT_F32, "bf16")
    if args.workload in ("gemma_decode", "q4_sweep", "all"):
        extra["gemma3_1b_decode"] = gemma_decode(args, N, cpu=not args.no_cpu_baseline)
    if args.workload == "q4_sweep":
        # The metric's GEMM part: M = 512 prefill at the
        # Qwen2.5-7B shapes, MX int8 activations, both weight formats.
        extra["prefill_m512_mx"] = measure_cases(args, N, [(d, n, k, 512) for d in (1, 2) for n, k in QWEN_PREFILL],
                                                 N.ACT_MXI8, "prefill_mx")
    if args.workload not in ("q4_sweep", "all"):
        print(json.dumps(dict(workload=args.workload, results=extra)), flush=True)
        return
    result, inputs = q4_sweep(args, N)
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle as O  # the CPU baseline leg only
        cpu = cpu_baseline_q4(N, O, inputs)
    line = dict(metric=result["metric"], value=result["value"], unit=result["unit"], n_gpus=1, steps=args.steps,
                warmup=args.warmup, ms_per_step=round(result["ms_per_step"], 5), higher_is_better=True,
                scaling="weak", vs_baseline=None, dtype=result["dtype"], data="synthetic (seeded)",
                config=result["config"], roofline=result["roofline"], cpu_baseline=cpu,
                per_shape=result["per_shape"])
    if extra:
        line["extra"] = extra
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
