"""Benchmark: nncpu's quantized matmul on one MI355X.

Default workload: the 4-bit GEMV sweep at
Llama-3-8B projection shapes (N x K = 4096x4096, 1024x4096, 14336x4096,
4096x14336), M = 1, weights 0.02*N(0,1) re-encoded to nncpu's Q4 layout,
activations N(0,1) quantized on the device to int8 blocks (nncpu's Q8_0
encoder). One step = one GEMV per shape. Inputs are resident in HBM; each
shape cycles through enough uploaded weight copies (>= 512 MB, twice the
MI355X Infinity Cache) that every launch streams its weights from HBM.

value = algorithmic bytes of exactly --steps timed steps / the time between
two events on the launch stream, synchronised on both sides (GB/s); bytes
per GEMV = N*K/2 + N*K/16 (quants, BF16 scales and biases) + 4K + 4N (f32 x
in, f32 y out), the reference's own byte accounting plus the vectors.

roofline: the same kernel timed per shape over a HIP graph of
max(copies, 200, steps) launches, so every launch reads a copy no earlier
launch of the graph has left in a cache and the graph's start-up is spread
over many launches; achieved = mean algorithmic bytes / mean per-launch
time. The measured peaks (calibration kernels, include/nncpu_calib.h) go
beside the datasheet's.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--workload q4_sweep]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0
ROTATE_BYTES = 512 << 20
MIN_LAUNCHES = 200

Q4_SWEEP = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]
# Llama-3-8B's gate and up projections as one matrix: what a decode step
# streams in one launch when the two are loaded concatenated.
FUSED_GATE_UP = (28672, 4096)
# HBM bytes per launch of the sweep's GEMVs, in the order of Q4_SWEEP: the
# rocprofv3 --pmc FETCH_SIZE (scaled by 2.0, the factor a 64 MiB device copy
# gives in the same run) + WRITE_SIZE readings of `bench.py --workload traffic`.
TRAFFIC_SOURCE = "profiles/gemv_i8_q4_llama3_8b_sweep.md (rocprofv3 --pmc over bench.py --workload traffic)"
Q4_SWEEP_TRAFFIC = [10_605_568, 2_716_672, 36_854_784, 36_948_992]
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


def time_graph(st, launches, reps, warmup):
    """Run the step `launches` (a list of callables) `warmup` times eagerly,
    capture `reps` steps in one HIP graph (host launch cost would otherwise
    exceed these microsecond kernels), replay it once untimed (the first
    replay uploads the graph) and time a second replay between two events on
    the launch stream, synchronised on both sides. Returns seconds."""
    torch = st.torch
    for _ in range(warmup):
        for f in launches:
            f()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st.s):
        for _ in range(reps):
            for f in launches:
                f()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    e0 = st.event()
    with torch.cuda.stream(st.s):
        g.replay()
    e1 = st.event()
    torch.cuda.synchronize()
    del g
    return e0.elapsed_time(e1) / 1e3


def rotating(N, st, dtype, n, k, m, act, seed, rot_bytes=ROTATE_BYTES):
    """A launch callable over >= rot_bytes of weight copies (each call takes
    the next copy), its inputs resident in HBM. act: ACT_I8 / ACT_MXI8 launch
    the int8 matmul on activations quantized beforehand (nncpu's Q8_0 encoder
    / power-of-two MX blocks); ACT_F32 the bit-exact f32 path (Q4 block sums
    included)."""
    import torch
    wb = weight_bytes(dtype, n, k)
    copies = max(2, math.ceil(rot_bytes / wb))
    ws = make_weights(N, dtype, n, k, seed, copies)
    x = make_x(k, m, seed ^ 0xA11)
    y = torch.zeros(m * n, dtype=torch.float32, device="cuda")
    qmode = act if act != N.ACT_F32 else N.ACT_I8
    _, _, abytes = N.act_layout_ex(qmode, k, m)
    buf = torch.zeros(abytes, dtype=torch.uint8, device="cuda")
    N.quantize_act_ex_dev(qmode, x.data_ptr(), k, k, m, buf.data_ptr(), st.handle)
    for w in ws:
        w.prepare(act, m)
    state = {"i": 0}

    def launch():
        w = ws[state["i"] % len(ws)]
        state["i"] += 1
        if act != N.ACT_F32:
            N.gemv_act_dev(w, act, buf.data_ptr(), m, y.data_ptr(), n, st.handle)
        else:
            N.gemv_batch_dev(w, x.data_ptr(), k, y.data_ptr(), n, m, N.ACT_F32, st.handle)

    launch.keep = (ws, x, y, buf)
    launch.copies = copies
    return launch


def per_launch(st, launch, steps, warmup):
    """Seconds per launch over a graph of max(copies, MIN_LAUNCHES, steps)."""
    reps = max(launch.copies, MIN_LAUNCHES, steps)
    return time_graph(st, [launch], reps, min(warmup, 5)) / reps, reps


def case_name(dtype, n, k, m):
    return f"{ {1: 'Q8', 2: 'Q4', 3: 'BF16'}[dtype]} {n}x{k} M={m}"


def measure_cases(args, N, cases, act, label):
    """Each (dtype, n, k, m) case alone, per launch (see per_launch)."""
    import torch
    st = Stream()
    out = []
    for ci, (dtype, n, k, m) in enumerate(cases):
        launch = rotating(N, st, dtype, n, k, m, act, 0x5EED10 + 7 * ci + dtype)
        torch.cuda.synchronize()
        secs, reps = per_launch(st, launch, args.steps, args.warmup)
        us = secs * 1e6
        byts = gemv_bytes(dtype, n, k, m)
        ops = 2.0 * m * n * k
        e = dict(case=case_name(dtype, n, k, m), us=round(us, 3), gbs=round(byts / us / 1e3, 1),
                 weights_gbs=round(weight_bytes(dtype, n, k) / us / 1e3, 1),
                 hbm_frac=round(byts / us / 1e3 / HBM_PEAK_GBS, 4), tops=round(ops / us / 1e6, 2),
                 int8_frac=round(ops / us / 1e6 / INT8_PEAK_TOPS, 4), launches=reps)
        log(f"{label}: {e}")
        out.append(e)
        del launch
        torch.cuda.synchronize()
    return out


def q4_sweep(args, N):
    """The headline: exactly args.steps timed steps of the four GEMVs, plus
    each shape's per-launch time for the roofline."""
    import torch
    st = Stream()
    per_shape, inputs, launches = [], [], []
    for i, (n, k) in enumerate(Q4_SWEEP):
        launch = rotating(N, st, 2, n, k, 1, N.ACT_I8, 0x5EED01 + i)
        launches.append(launch)
        ws, x, _, buf = launch.keep
        inputs.append((ws[0], buf, k))
        log(f"shape {n}x{k}: {launch.copies} copies of {weight_bytes(2, n, k) / 1e6:.1f} MB")
    torch.cuda.synchronize()
    for (n, k), launch in zip(Q4_SWEEP, launches):
        secs, reps = per_launch(st, launch, args.steps, args.warmup)
        b = gemv_bytes(2, n, k)
        p = dict(shape=f"{n}x{k}", copies=launch.copies, launches=reps, bytes=b, us=round(secs * 1e6, 4),
                 gbs=round(b / secs / 1e9, 1), weights_gbs=round(weight_bytes(2, n, k) / secs / 1e9, 1),
                 hbm_frac=round(b / secs / 1e9 / HBM_PEAK_GBS, 4))
        log(f"{p['shape']}: {p['us']:.2f} us/launch over {reps} launches, {p['gbs']:.0f} GB/s "
            f"({100 * p['hbm_frac']:.1f}% of HBM)")
        per_shape.append(p)
    # The sweep: exactly `steps` steps of the four GEMVs.
    secs = time_graph(st, launches, args.steps, args.warmup)
    step_bytes = sum(gemv_bytes(2, n, k) for n, k in Q4_SWEEP)
    value = step_bytes * args.steps / secs / 1e9
    kernel_us = sum(p["us"] for p in per_shape) / len(per_shape)
    bytes_per_launch = step_bytes / len(Q4_SWEEP)
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
                      traffic=round(sum(Q4_SWEEP_TRAFFIC) / len(Q4_SWEEP_TRAFFIC)), traffic_source=TRAFFIC_SOURCE,
                      kernel="gemv_i8_v2_kernel (Q4, M=1)", bytes_per_launch=bytes_per_launch,
                      avg_launch_us=round(kernel_us, 3),
                      timing=f"HIP events over a graph of max(copies, {MIN_LAUNCHES}, steps) launches per shape"),
        per_shape=per_shape,
    )
    return result, inputs, launches


def traffic_run(N):
    """For `rocprofv3 --pmc FETCH_SIZE` / `--pmc WRITE_SIZE`: a 64 MiB device
    copy (the counter's calibration: 64 MiB read, 64 MiB written), then each
    sweep shape launched eagerly five times over two weight copies, then the
    M = 512 MX GEMM at the Q8 gate and down shapes three times each."""
    import torch
    a = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    st = Stream()
    for i, (n, k) in enumerate(Q4_SWEEP):
        launch = rotating(N, st, 2, n, k, 1, N.ACT_I8, 0x5EED01 + i, rot_bytes=1)
        for _ in range(5):
            launch()
        torch.cuda.synchronize()
        log(f"traffic: {n}x{k} x5")
        del launch
    for i, (n, k) in enumerate([(18944, 3584), (3584, 18944)]):
        launch = rotating(N, st, 1, n, k, 512, N.ACT_MXI8, 0x5EED20 + i, rot_bytes=1)
        for _ in range(3):
            launch()
        torch.cuda.synchronize()
        log(f"traffic: MX Q8 {n}x{k} M=512 x3")
        del launch


# ---- measured peaks (the roofline denominators on this box) ------------------------

def _calib():
    L = C.CDLL(os.path.join(ROOT, "nncpu_amd", "lib", "libnncpu_calib.so"))
    L.nnc_clock_probe.argtypes, L.nnc_clock_probe.restype = [C.c_int, C.c_int, C.c_void_p, C.c_void_p], C.c_int
    L.nnc_read_stream.argtypes, L.nnc_read_stream.restype = [C.c_void_p, C.c_size_t, C.c_int, C.c_void_p, C.c_void_p], C.c_int
    L.nnc_mfma_loop.argtypes, L.nnc_mfma_loop.restype = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p], C.c_int
    L.nnc_mfma_ops.argtypes, L.nnc_mfma_ops.restype = [C.c_int, C.c_int, C.c_int], C.c_longlong
    return L


def shader_clock_mhz():
    """The shader clock now: one wave per CU times a dependent FMA chain with
    the core-clock and the 100 MHz counters (nnc_clock_probe); the median
    over the CUs, in MHz."""
    import torch
    L = _calib()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.zeros(2 * cus, dtype=torch.int64, device="cuda")
    torch.cuda.synchronize()
    assert L.nnc_clock_probe(cus, 200000, out.data_ptr(), None) == 0
    torch.cuda.synchronize()
    v = out.cpu().numpy().reshape(cus, 2).astype(np.float64)
    return round(float(np.median(100.0 * v[:, 0] / np.maximum(v[:, 1], 1))), 1)


def peaks(args):
    """HBM: a read stream over 1 GiB (cold, four times the Infinity Cache)
    and a device copy; per-launch read-stream ceilings at the sweep's weight
    sizes, timed like the sweep (a graph of launches over >= 512 MB of
    rotating slices); the matrix unit: dense int8 and BF16 MFMA loops over
    every CU."""
    import torch
    L = _calib()
    st = Stream()
    out = torch.zeros(256, dtype=torch.int32, device="cuda")
    big = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    big.fill_(1)
    res = {}
    best = {}
    for unroll in (4, 16):
        def f(unroll=unroll):
            assert L.nnc_read_stream(big.data_ptr(), big.numel(), unroll, out.data_ptr(), st.handle) == 0
        secs = time_graph(st, [f], 5, 1) / 5
        best[unroll] = big.numel() / secs / 1e9
    res["hbm_read_1gib_gbs"] = round(max(best.values()), 1)
    dst = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    src = big[:256 << 20]
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0 = st.event()
    with torch.cuda.stream(st.s):
        for _ in range(10):
            dst.copy_(src)
    e1 = st.event()
    torch.cuda.synchronize()
    res["copy_256mib_gbs"] = round(2 * dst.numel() * 10 / (e0.elapsed_time(e1) / 1e3) / 1e9, 1)
    ceil = []
    for size in sorted({weight_bytes(2, n, k) for n, k in Q4_SWEEP + [FUSED_GATE_UP]}):
        sz = (size + 4095) // 4096 * 4096
        slices = max(2, (512 << 20) // sz)
        state = {"i": 0}

        def f(sz=sz, slices=slices, state=state):
            off = (state["i"] % slices) * sz
            state["i"] += 1
            assert L.nnc_read_stream(big.data_ptr() + off, sz, 4, out.data_ptr(), st.handle) == 0
        reps = max(slices, MIN_LAUNCHES)
        secs = time_graph(st, [f], reps, 2) / reps
        ceil.append(dict(bytes=sz, us=round(secs * 1e6, 3), gbs=round(sz / secs / 1e9, 1)))
    res["read_stream_per_launch"] = ceil
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for kind, name, peak in ((1, "mfma_i8_tops", INT8_PEAK_TOPS), (2, "mfma_bf16_tflops", BF16_PEAK_TFLOPS)):
        blocks, iters = cus * 2, 4096

        def f(kind=kind, blocks=blocks, iters=iters):
            assert L.nnc_mfma_loop(kind, iters, blocks, out.data_ptr(), st.handle) == 0
        secs = time_graph(st, [f], 5, 1) / 5
        v = L.nnc_mfma_ops(kind, iters, blocks) / secs / 1e12
        res[name] = round(v, 1)
        res[name.replace("_tops", "_frac").replace("_tflops", "_frac")] = round(v / peak, 4)
    res["datasheet"] = dict(hbm_gbs=HBM_PEAK_GBS, int8_tops=INT8_PEAK_TOPS, bf16_tflops=BF16_PEAK_TFLOPS)
    del big, dst
    # A reference point for the M = 512 GEMMs: the platform library's plain
    # BF16 GEMM (torch.matmul -> hipBLASLt) at the prefill's gate / down
    # shapes, no block scales, four rotating weight copies.
    lib_gemm = []
    for n, k in ((18944, 3584), (3584, 18944)):
        a = torch.randn(512, k, device="cuda", dtype=torch.bfloat16)
        ws = [torch.randn(k, n, device="cuda", dtype=torch.bfloat16) for _ in range(4)]
        for i in range(4):
            torch.matmul(a, ws[i])
        torch.cuda.synchronize()
        e0 = st.event()
        with torch.cuda.stream(st.s):
            for i in range(40):
                torch.matmul(a, ws[i % 4])
        e1 = st.event()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / 40
        lib_gemm.append(dict(case=f"BF16 512x{n}x{k}", us=round(us, 2), tflops=round(2 * 512 * n * k / us / 1e6, 1)))
        del a, ws
    res["hipblaslt_bf16_m512"] = lib_gemm
    torch.cuda.synchronize()
    log(f"peaks: {res}")
    return res


QWEN_PREFILL = [(3584, 3584), (512, 3584), (18944, 3584), (3584, 18944)]  # q/o, k/v, gate/up, down
VERIFY_SHAPES = [(6144, 1536), (1536, 6144), (2048, 1536), (1536, 1536)]
# The bit-exact one-vector kernels' shapes: Qwen2.5-7B's down, q/k/v and o, Llama-3-8B's, and a
# 2560-row case (the streamed kernel's rows-per-workgroup choice at each).
F32_M1_SHAPES = [(3584, 18944), (4096, 14336), (4608, 3584), (4096, 4096), (3584, 3584), (2560, 8192)]
I8_M1_SHAPES = [(4096, 4096), (14336, 4096), (4096, 14336), (28672, 4096), (4608, 3584), (3584, 3584),
                (37888, 3584), (3584, 18944)]
GEMMA_DECODE = [(1024, 1152), (256, 1152), (1152, 1024), (6912, 1152), (1152, 6912), (262144, 1152)]
# BF16 weights: the reference's own BF16 test shapes (Gemma E2B/E4B, kernels/tests.rs:435-447) and
# Llama-3-8B projections.
BF16_SHAPES = [(1536, 1536), (2048, 1536), (6144, 1536), (4096, 4096), (14336, 4096)]


def qwen_prefill(args, N, dtype: int, act: int, n_tok: int = 512, n_layer: int = 28):
    """BASELINE configs[4], end to end: a Qwen2.5-7B-shaped model (d 3584,
    FFN 18944, 28 query / 4 KV heads of 128, RoPE base 1e6, RMSNorm, SwiGLU,
    q/k/v biases) with random weights 0.02*N(0,1) encoded by the library's
    device encoder (nncpu Q8_0 / Q4), prefilling 512 random tokens through
    all 28 layers and the last token's lm_head row (152064 x 3584, tied to
    the embedding table). Every weight matmul is the library's int8 path in
    mode `act` (activations quantized on the device: nncpu's Q8_0 encoder and
    the int8 MFMA GEMM, or MX blocks and the BF16-MFMA GEMM); q/k/v and
    gate/up are one concatenated matrix each, as serving engines load them.
    Everything between the matmuls is the device forward
    (nncpu_amd/host/layers_gpu.hip: embedding rows, RMSNorm, biases, RoPE, the
    BF16 K/V cache, blockwise causal GQA attention, SiLU(gate) * up, with the
    CPU forward's arithmetic). One step = one full prefill, captured in a HIP
    graph; `matmul_ms` is a graph of the same matmul calls alone on the same
    shapes, `layer_ops_ms` the difference."""
    import torch
    from nncpu_amd.models import DeviceForward, norm_stride, qwen25_7b_config
    cfg = qwen25_7b_config(n_ctx=n_tok, n_layer=n_layer, wtype=2 if dtype == 2 else 1)
    d, ff, nkv, hd, vocab = cfg.n_embd, cfg.n_ff, cfg.n_kv, cfg.head_dim, cfg.n_vocab
    qkv = d + 2 * nkv * hd
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

    weights = []
    for _ in range(n_layer):
        weights += [weight(qkv, d), None, None, weight(d, d), weight(2 * ff, d), None, weight(d, ff)]
    lm_head = weight(vocab, d)
    weights.append(lm_head)
    rng = np.random.default_rng(0x9E11 + dtype)
    norms = (1.0 + 0.1 * rng.standard_normal(norm_stride(cfg) * n_layer + d)).astype(np.float32)
    biases = (0.02 * rng.standard_normal(n_layer * qkv)).astype(np.float32)
    fwd = DeviceForward(cfg, weights, norms, biases, lm_head, n_batch=n_tok, act=act, stream=st.handle)
    tok = torch.randint(0, vocab, (n_tok,), generator=g, device=dev, dtype=torch.int32)
    logits = torch.empty(vocab, device=dev)

    def forward():
        fwd.forward_dev(tok.data_ptr(), n_tok, 0)
        fwd.logits_last_dev(n_tok, logits.data_ptr())

    # The matmuls alone, the same calls on buffers of the same shapes.
    xa = torch.randn(n_tok, 2 * ff, device=dev)
    ya = torch.empty(n_tok, 2 * ff, device=dev)

    def matmuls():
        for li in range(n_layer):
            W = weights[7 * li:7 * li + 7]
            N.gemv_batch_dev(W[0], xa.data_ptr(), d, ya.data_ptr(), qkv, n_tok, act, st.handle)
            N.gemv_batch_dev(W[3], xa.data_ptr(), d, ya.data_ptr(), d, n_tok, act, st.handle)
            N.gemv_batch_dev(W[4], xa.data_ptr(), d, ya.data_ptr(), 2 * ff, n_tok, act, st.handle)
            N.gemv_batch_dev(W[6], xa.data_ptr(), 2 * ff, ya.data_ptr(), d, n_tok, act, st.handle)
        N.gemv_batch_dev(lm_head, xa.data_ptr(), d, ya.data_ptr(), vocab, 1, act, st.handle)

    with torch.cuda.stream(st.s):
        for _ in range(2):
            forward()
            matmuls()
        torch.cuda.synchronize()
        steps = max(1, min(args.steps, 5))
        e0 = st.event()
        for _ in range(steps):
            forward()
        e1 = st.event()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    eager_logits = logits.clone()
    assert torch.isfinite(eager_logits).all()
    per_layer = 2 * n_tok * d * (qkv + d + 2 * ff + ff)
    ops = n_layer * per_layer + 2 * d * vocab
    # One prefill captured in a HIP graph and replayed; each replay, with
    # eager work between them, must give the eager logits.
    graph, mgraph = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st.s):
        forward()
    with torch.cuda.graph(mgraph, stream=st.s):
        matmuls()
    for _ in range(3):
        logits.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(logits, eager_logits), "graph replay differs from the eager prefill"
        torch.ones(256, device=dev).sum().item()  # eager work between replays

    def timed(gr):
        with torch.cuda.stream(st.s):
            g0 = st.event()
            for _ in range(steps):
                gr.replay()
            g1 = st.event()
        torch.cuda.synchronize()
        return g0.elapsed_time(g1) / steps

    gms, mm_ms = timed(graph), timed(mgraph)
    del graph, mgraph
    res = dict(case=f"{'Q8' if dtype == 1 else 'Q4'} Qwen2.5-7B-shaped prefill, {n_layer} layers, {n_tok} tokens",
               activations="MX int8 blocks (power-of-two scales)" if act == N.ACT_MXI8 else "int8 blocks (nncpu Q8_0)",
               ms=round(gms, 3), tokens_per_s=round(n_tok / gms * 1e3, 1), eager_ms=round(ms, 3),
               matmul_ms=round(mm_ms, 3), layer_ops_ms=round(gms - mm_ms, 3),
               matmul_tops=round(ops / mm_ms / 1e9, 1), steps=steps,
               timing="ms: one prefill replayed from a HIP graph (embedding, 28 layers of the device forward, "
                      "lm_head row); eager_ms: launched from the host; matmul_ms: a graph of the same matmul calls "
                      "alone; layer_ops_ms = ms - matmul_ms")
    log(f"qwen_prefill: {res}")
    fwd.free()
    for w in weights:
        if w is not None:
            w.free()
    return res


def qwen_decode(args, N, dtype: int, acts, n_prompt: int = 64, n_gen: int = 128, n_layer: int = 28,
                n_check: int = 16):
    """Batch-1 greedy decode of the Qwen2.5-7B shape (config 5's model) on the
    device forward: the prompt in 16-token batches, then one decode step per
    token (nngl_decode_step_dev + nngl_greedy_next_dev, captured once in a
    HIP graph and replayed; no host round trip per token). Random weights as
    qwen_prefill's; every matmul in each activation mode of `acts`. tok/s
    beside the weight bytes a token streams and the matmul-only ceiling at
    the measured HBM read rate."""
    import torch
    from nncpu_amd.models import DeviceForward, Model, norm_stride, qwen25_7b_config
    cfg = qwen25_7b_config(n_ctx=n_prompt + n_gen, n_layer=n_layer, wtype=2 if dtype == 2 else 1)
    d, ff, nkv, hd, vocab = cfg.n_embd, cfg.n_ff, cfg.n_kv, cfg.head_dim, cfg.n_vocab
    qkv = d + 2 * nkv * hd
    g = torch.Generator(device="cuda")
    g.manual_seed(0xDEC0 + dtype)

    def weight(rows, cols):
        w = torch.randn(rows * cols, generator=g, device="cuda").mul_(0.02)
        torch.cuda.synchronize()
        out = N.Weight.encode_dev(dtype, w.data_ptr(), rows, cols)
        del w
        return out

    layers = []
    for _ in range(n_layer):
        layers += [weight(d, d), weight(nkv * hd, d), weight(nkv * hd, d), weight(d, d), weight(ff, d), weight(ff, d),
                   weight(d, ff)]
    lm_head = weight(vocab, d)
    rng = np.random.default_rng(0xDEC0 + dtype)
    norms = (1.0 + 0.1 * rng.standard_normal(norm_stride(cfg) * n_layer + d)).astype(np.float32)
    biases = (0.02 * rng.standard_normal(n_layer * qkv)).astype(np.float32)
    prompt = rng.integers(0, vocab, n_prompt).astype(np.int32)
    # The timed forward reads [q; k; v] and [gate; up] as one matrix each;
    # the CPU forward that checks its tokens takes the seven matrices.
    model = Model(cfg, layers + [lm_head], norms, biases, lm_head)
    weights = model.fused_weights()
    wbytes = sum(w.split_bytes() for w in weights if w is not None)
    out = []
    for act in acts:
        s = torch.cuda.Stream()
        fwd = DeviceForward(cfg, weights, norms, biases, lm_head, n_batch=16, act=act, stream=s.cuda_stream)
        fwd.generate_graph(prompt, 8, stream=s)  # warm-up: layouts, scratch, clocks
        toks, secs, _, _ = fwd.generate_graph(prompt, n_gen, stream=s)
        fwd.free()
        tok_s = (n_gen - 1) / secs
        # The first n_check tokens against the CPU forward (gemma3.cpp's
        # restatement of forward.rs, matmuls through the same library in the
        # same activation mode), outside the timed region.
        t0 = time.perf_counter()
        tc, _, _, _ = model.cpu_generate(prompt, n_check, batch=16, act=act)
        cpu_s = time.perf_counter() - t0
        res = dict(case=f"{'Q8' if dtype == 1 else 'Q4'} Qwen2.5-7B-shaped decode, {n_layer} layers",
                   activations={N.ACT_F32: "f32 (bit-exact drop-in)", N.ACT_I8: "int8 blocks (nncpu Q8_0)",
                                N.ACT_MXI8: "MX int8 blocks"}[act],
                   prompt=n_prompt, generated=n_gen, tok_s=round(tok_s, 1), ms_per_token=round(1e3 / tok_s, 3),
                   weight_bytes_per_token=wbytes, weights_gbs=round(wbytes * tok_s / 1e9, 1),
                   timing="graph replays of one decode step per token, host clock around the replays",
                   tokens_identical=bool(np.array_equal(toks[:n_check], tc)), tokens_checked=n_check,
                   check="the first tokens against the CPU forward with the library's matmuls, same mode")
        res["matmul_ceiling_tok_s"] = round(HBM_PEAK_GBS * 1e9 / wbytes, 1)
        res["frac_of_ceiling"] = round(tok_s / res["matmul_ceiling_tok_s"], 3)
        log(f"qwen_decode: {res} (CPU check {cpu_s:.1f}s)")
        out.append(res)
    for w in weights + layers:
        if w is not None:
            w.free()
    return out


def host_info():
    """nproc, the CPU model and the physical cores this process may use (the
    box's CPU share: OMP_NUM_THREADS when the environment sets it)."""
    model = ""
    try:
        for line in subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
    except Exception:
        pass
    avail = len(os.sched_getaffinity(0))
    try:
        out = subprocess.run(["lscpu", "-p=CORE,SOCKET"], capture_output=True, text=True, timeout=10).stdout
        phys = len({ln for ln in out.splitlines() if ln and not ln.startswith("#")})
    except Exception:
        phys = avail
    share = int(os.environ.get("OMP_NUM_THREADS") or 0) or phys
    return dict(nproc=avail, model=model, physical_cores=phys, all_cores=max(1, min(share, phys, avail)))


def cpu_time(f, budget_s, min_reps=2):
    """Best time of f() over repeats after one warm-up, within a budget."""
    f()
    best, t_end, reps = float("inf"), time.time() + budget_s, 0
    while reps < min_reps or (time.time() < t_end and reps < 3):
        t0 = time.perf_counter()
        f()
        best = min(best, time.perf_counter() - t0)
        reps += 1
    return best


def cpu_inputs(N, O, inputs):
    """The sweep's weights (downloaded from the GPU) and quantized
    activations (dequantized: the values nncpu's f32 kernel would be fed)."""
    out = []
    for w, buf, k in inputs:
        n = w.rows()
        off_s, _, _ = N.act_layout(k, 1)
        a = buf.cpu().numpy()
        xd = O.dequant_act(a[:k].view(np.int8), a[off_s:off_s + k // 16].view(np.uint16))
        out.append((O.QMatrix.from_split(2, n, k, w.download()), xd))
    return out


def cpu_baseline(O, sweep):
    """nncpu's AVX2 kernels (restated, oracle/avx2.cpp) on this host's cores,
    as the reference's bench_gemv (kernels/tests.rs:1295-1416) times them:
    the sweep's own weights and activations (`sweep`, from cpu_inputs),
    >= 256 MB of weight copies rotated so they stream from DRAM, best of
    passes after a warm-up; rows split over threads as pool::for_rows does.
    value: the Q4 sweep at nncpu's default min(8, CPUs) threads; beside it
    the same at 1 thread and at all cores (14336x4096 only), the Q8 vocab
    GEMV, speculative verify at M = 2..16 and the M = 512 prefill as nncpu
    runs it (32 batches of 16 tokens, session/engine.rs:362-380), on seeded
    weights of the reference's test generator."""
    if not O.avx_available():
        return None
    host = host_info()
    threads = min(8, host["nproc"])
    t_start = time.time()
    rot = {}

    def rotation(i):
        if i not in rot:
            m, xd = sweep[i]
            copies = max(2, math.ceil((256 << 20) / weight_bytes(2, m.rows, m.cols)))
            rot[i] = ([m] + [O.QMatrix(2, m.rows, m.cols, tuple(p.copy() for p in m.parts))
                             for _ in range(copies - 1)], xd)
        return rot[i]

    def sweep_rate(th, sel, budget):
        O.avx_set_threads(th)
        tot_b, tot_s, parts = 0, 0.0, []
        for i in sel:
            ms, xd = rotation(i)
            n, k = ms[0].rows, ms[0].cols

            def one_pass(ms=ms, xd=xd):
                for mm in ms:
                    O.gemv_batch(mm, xd, backend="avx2")
            dt = cpu_time(one_pass, budget) / len(ms)
            tot_b += gemv_bytes(2, n, k)
            tot_s += dt
            parts.append(f"{n}x{k}:{gemv_bytes(2, n, k) / dt / 1e9:.1f}GB/s")
        log(f"cpu: {th} threads: {', '.join(parts)}")
        return tot_b / tot_s / 1e9, parts

    gbs, parts = sweep_rate(threads, range(len(sweep)), 2.0)
    g1, _ = sweep_rate(1, [2], 2.0)
    gall, _ = sweep_rate(host["all_cores"], [2], 1.0)
    res = dict(value=round(gbs, 2), unit="GB/s", cores=threads, kind="port",
               sample="Q4 GEMV M=1 at " + ", ".join(parts) + f"; {threads} threads (nncpu default min(8, CPUs)), "
               "AVX2 restatement of q4_rows_raw on the same weights and dequantized int8 activations, "
               ">=256 MB rotation, best of passes",
               host=host, threads_1_gbs=round(g1, 2), threads_all_gbs=round(gall, 2),
               threads_all=host["all_cores"], per_thread_shape="14336x4096",
               host_stream_gbs_1thread=round(O.avx_stream_gbs(256 << 20, 2), 1))
    rot.clear()
    O.avx_set_threads(threads)
    rng = O.Rng(0xC9B)
    other = {}
    # Config 3: Gemma-3 vocab lm_head, Q8, M = 1.
    n, k = Q8_VOCAB[0]
    m = O.QMatrix.from_f32(1, rng.normals(n * k, 0.02).reshape(n, k))
    x = rng.normals(k, 1.0)
    dt = cpu_time(lambda: O.gemv_batch(m, x, backend="avx2"), 1.0)
    other["q8_vocab_262144x1152_m1"] = dict(gbs=round(gemv_bytes(1, n, k) / dt / 1e9, 2), ms=round(dt * 1e3, 3))
    log(f"cpu: vocab {other['q8_vocab_262144x1152_m1']}")
    del m
    # Config 4: verify at M = 2..16, Q8 6144x1536.
    n, k = VERIFY_SHAPES[0]
    m = O.QMatrix.from_f32(1, rng.normals(n * k, 0.02).reshape(n, k))
    ver = {}
    for mt in (2, 4, 8, 16):
        x = rng.normals(mt * k, 1.0)
        dt = cpu_time(lambda: O.gemv_batch(m, x, mt, backend="avx2"), 0.5)
        ver[f"M={mt}"] = dict(us=round(dt * 1e6, 1), gflops=round(2 * mt * n * k / dt / 1e9, 1))
    other["verify_q8_6144x1536"] = ver
    log(f"cpu: verify {ver}")
    # Config 5: the gate projection at M = 512 as 32 calls of 16 tokens.
    n, k = QWEN_PREFILL[2]
    m = O.QMatrix.from_f32(1, rng.normals(n * k, 0.02).reshape(n, k))
    x = rng.normals(16 * k, 1.0)
    dt = cpu_time(lambda: O.gemv_batch(m, x, 16, backend="avx2"), 0.5, min_reps=1)
    other["prefill_q8_18944x3584_m512"] = dict(ms=round(32 * dt * 1e3, 1),
                                               gops=round(2 * 512 * n * k / (32 * dt) / 1e9, 1),
                                               how="32 x gemv_batch(16 tokens), one timed, times 32")
    log(f"cpu: prefill {other['prefill_q8_18944x3584_m512']}")
    del m
    res["configs"] = other
    res["wall_s"] = round(time.time() - t_start, 1)
    return res


def gemma_decode(args, N, cpu: bool):
    """Gemma-3-1B-shaped greedy decode of 128 tokens from a
    32-token prompt, on the device-resident step, the model loaded from the
    seeded random-init GGUF (nncpu_amd.gguf) and re-encoded to Q8_0 (and, in
    `q4`, to nncpu's Q4). tok/s counts the 127 decode forwards after the
    prompt; the timed run is the second one (the first captures the step's
    graph). With `cpu`, the CPU baseline leg: the same decode with nncpu's CPU
    gemv (the oracle's AVX2 restatement, 8 threads) in the shared C++
    forward, timed, and its tokens compared with the device run's."""
    from nncpu_amd.gemma import gemma3_1b_gguf
    t0 = time.perf_counter()
    path = gemma3_1b_gguf()
    log(f"gemma3-1b GGUF written in {time.perf_counter() - t0:.1f}s")
    out = decode_leg(N, path, N.Q8_0, cpu)
    out["q4"] = decode_leg(N, path, N.Q4S, cpu)
    return out


def decode_leg(N, path, dtype, cpu: bool):
    import ctypes as C
    from nncpu_amd.gemma import Gemma3, random_prompt
    fmt = "Q8_0" if dtype == N.Q8_0 else "Q4"
    t1 = time.perf_counter()
    m = Gemma3.from_gguf(path, n_ctx=256, dtype=dtype)
    log(f"gemma3-1b loaded (device decode + {fmt} re-encode) in {time.perf_counter() - t1:.1f}s")
    prompt, n_gen = random_prompt(32, m.cfg.n_vocab), 128
    m.generate_device(prompt, n_gen)
    clk0 = shader_clock_mhz()
    tg, hg, tp, td = m.generate_device(prompt, n_gen)
    clk1 = shader_clock_mhz()
    out = dict(config="gemma-3-1b architecture, random-init GGUF from seed (BF16 matrices 0.02*N(0,1) from the "
                      f"reference's test generator) re-encoded to {fmt} on load, 32-token prompt, 128 greedy tokens",
               tok_s=round((n_gen - 1) / td, 1), ms_per_token=round(td / (n_gen - 1) * 1e3, 4),
               prefill_s=round(tp, 4), kernels_per_token=4, shader_clock_mhz=[clk0, clk1])
    # The matmul-only ceiling: every weight read once per token at the HBM
    # datasheet rate (the layers' matrices and the tied lm_head).
    wpt = sum(weight_bytes(dtype, r, c) for r, c in m.shapes)
    out.update(weight_bytes_per_token=wpt, matmul_ceiling_tok_s=round(HBM_PEAK_GBS * 1e9 / wpt, 1),
               frac_of_ceiling=round(out["tok_s"] * wpt / (HBM_PEAK_GBS * 1e9), 4))
    log(f"gemma3-1b device decode ({fmt}): {out['tok_s']} tok/s")
    if cpu:
        from oracle import oracle as O  # the CPU baseline leg only

        class Table(C.Structure):
            _fields_ = [("n", C.c_int), ("dtype", C.c_int), ("bufs", C.POINTER(C.c_void_p)),
                        ("rows", C.POINTER(C.c_size_t)), ("cols", C.POINTER(C.c_size_t))]
        bufs = [w.download() for w in m.weights]
        arr = (C.c_void_p * len(bufs))(*[b.ctypes.data for b in bufs])
        rows = (C.c_size_t * len(bufs))(*[r for r, _ in m.shapes])
        cols = (C.c_size_t * len(bufs))(*[c for _, c in m.shapes])
        table = Table(n=len(bufs), dtype=dtype, bufs=C.cast(arr, C.POINTER(C.c_void_p)),
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
        log(f"gemma3-1b cpu decode ({fmt}): {out['cpu_baseline']}")
    m.free()
    return out


def fused_norm(args, N):
    """The residual add and RMSNorm fused into the next matmul's prologue
    (nnh_gemv_rmsnorm_act_dev) at the Qwen2.5-7B decode's q / k / v and
    gate / up shapes, per launch beside the plain matmul on an input formed
    beforehand (f32: nnh_gemv_batch_dev; int8: nnh_gemv_act_dev on
    activations quantized beforehand): the difference is what the norm
    costs inside the matmul's launch."""
    import torch
    st = Stream()
    out = []
    for ci, (dtype, n, k) in enumerate((d, n, k) for d in (1, 2) for n, k in ((4608, 3584), (18944 * 2, 3584))):
        for act in (N.ACT_F32, N.ACT_I8):
            launch = rotating(N, st, dtype, n, k, 1, act, 0x5EED40 + 7 * ci + dtype)
            ws, x, y, _ = launch.keep
            r = torch.randn(k, device="cuda")
            g = 1.0 + 0.1 * torch.randn(k, device="cuda")
            xo = torch.zeros(k, device="cuda")
            normed = torch.zeros(k, device="cuda")
            state = {"i": 0}

            def fused(ws=ws, x=x, y=y, r=r, g=g, xo=xo, normed=normed, act=act, state=state):
                w = ws[state["i"] % len(ws)]
                state["i"] += 1
                N.gemv_rmsnorm_dev(w, x.data_ptr(), r.data_ptr(), g.data_ptr(), 1e-6, xo.data_ptr(), 0,
                                   normed.data_ptr(), y.data_ptr(), st.handle, act=act)
            fused.copies = launch.copies
            torch.cuda.synchronize()
            plain, _ = per_launch(st, launch, args.steps, args.warmup)
            both, reps = per_launch(st, fused, args.steps, args.warmup)
            e = dict(case=case_name(dtype, n, k, 1), act="f32" if act == N.ACT_F32 else "i8",
                     plain_us=round(plain * 1e6, 3), fused_us=round(both * 1e6, 3), launches=reps)
            log(f"fused_norm: {e}")
            out.append(e)
            del launch, fused
            torch.cuda.synchronize()
    return out


I8_PROLOGUE_SHAPES = [(4608, 3584), (3584, 3584), (1024, 4096), (14336, 4096), (4096, 8192), (3584, 9216),
                      (4096, 14336), (37888, 3584), (3584, 18944)]


def i8_prologue(args, N):
    """One f32 vector through nnh_gemv_batch_dev(..., NNH_ACT_I8), which
    quantizes x in the int8 GEMV's prologue at rows of 97..384 blocks (not
    tall Q8 matrices of rows that are not whole 64-block groups), per launch
    beside the two launches it replaces (the library quantizer, then
    nnh_gemv_act_dev) and the GEMV alone on activations quantized
    beforehand."""
    import torch
    st = Stream()
    out = []
    for ci, (dtype, n, k) in enumerate((d, n, k) for d in (1, 2) for n, k in I8_PROLOGUE_SHAPES):
        launch = rotating(N, st, dtype, n, k, 1, N.ACT_I8, 0x5EED90 + 7 * ci + dtype)
        ws, x, y, buf = launch.keep
        state = {"i": 0}

        def one(ws=ws, x=x, y=y, n=n, k=k, state=state):
            w = ws[state["i"] % len(ws)]
            state["i"] += 1
            N.gemv_batch_dev(w, x.data_ptr(), k, y.data_ptr(), n, 1, N.ACT_I8, st.handle)

        def two(ws=ws, x=x, y=y, buf=buf, n=n, k=k, state=state):
            w = ws[state["i"] % len(ws)]
            state["i"] += 1
            N.quantize_act_dev(x.data_ptr(), k, k, 1, buf.data_ptr(), st.handle)
            N.gemv_act_dev(w, N.ACT_I8, buf.data_ptr(), 1, y.data_ptr(), n, st.handle)
        one.copies = two.copies = launch.copies
        torch.cuda.synchronize()
        pre, _ = per_launch(st, launch, args.steps, args.warmup)
        t1, _ = per_launch(st, one, args.steps, args.warmup)
        t2, reps = per_launch(st, two, args.steps, args.warmup)
        e = dict(case=case_name(dtype, n, k, 1), prologue=(k // 32) <= 384 and not (dtype == 1 and n >= 16384 and (k // 32) % 64),
                 gemv_batch_dev_us=round(t1 * 1e6, 3), quantizer_then_gemv_us=round(t2 * 1e6, 3),
                 prequantized_gemv_us=round(pre * 1e6, 3), launches=reps)
        log(f"i8_prologue: {e}")
        out.append(e)
        del launch, one, two
        torch.cuda.synchronize()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="q4_sweep",
                    choices=["q4_sweep", "prefill", "qwen_prefill", "qwen_decode", "q8_vocab", "verify", "decode_f32", "gemma_decode",
                             "bf16", "peaks", "traffic", "fused_norm", "i8_m1", "i8_prologue", "f32_m1", "all"])
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
    if args.workload == "traffic":
        traffic_run(N)
        return
    extra = {}
    prefill_cases = [(d, n, k, 512) for d in (1, 2) for n, k in QWEN_PREFILL]
    if args.workload in ("gemma_decode", "q4_sweep", "all"):
        # First, on a GPU that has not yet run the minutes of matrix-unit and
        # streaming work below: the decode step is a chain of dependent
        # hand-offs, so its rate follows the shader clock (recorded beside it).
        extra["gemma3_1b_decode"] = gemma_decode(args, N, cpu=not args.no_cpu_baseline)
    if args.workload in ("peaks", "q4_sweep", "all"):
        extra["peaks"] = peaks(args)
    result = inputs = None
    if args.workload in ("q4_sweep", "all"):
        result, inputs, _ = q4_sweep(args, N)
        # Llama-3-8B's gate and up as one launch (a decode step's largest
        # weight read), and the bit-exact f32 path (the drop-in mode) at the
        # sweep's shapes.
        extra["q4_fused_gate_up_m1"] = measure_cases(args, N, [(2, *FUSED_GATE_UP, 1)], N.ACT_I8, "fused_gate_up")
        extra["q4_sweep_f32_bit_exact"] = measure_cases(args, N, [(2, n, k, 1) for n, k in Q4_SWEEP], N.ACT_F32,
                                                        "q4_f32")
    if args.workload in ("prefill", "q4_sweep", "all"):
        # The metric's GEMM part: M = 512 at the
        # Qwen2.5-7B shapes, both weight formats, both int8 modes (nncpu's
        # Q8_0 activation encoder, and power-of-two MX blocks).
        extra["prefill_m512_i8"] = measure_cases(args, N, prefill_cases, N.ACT_I8, "prefill_i8")
        extra["prefill_m512_mx"] = measure_cases(args, N, prefill_cases, N.ACT_MXI8, "prefill_mx")
    if args.workload in ("qwen_prefill", "all"):
        extra["qwen_prefill_e2e"] = [qwen_prefill(args, N, d, a) for d in (1, 2) for a in (N.ACT_MXI8, N.ACT_I8)]
    elif args.workload == "q4_sweep":
        # Config 5 end to end in the default run: Q8 weights, MX activations;
        # and its model's batch-1 decode, Q8 and Q4 weights, int8 activations.
        extra["qwen_prefill_e2e"] = [qwen_prefill(args, N, 1, N.ACT_MXI8)]
        extra["qwen_decode_e2e"] = [r for d in (1, 2) for r in qwen_decode(args, N, d, (N.ACT_I8,))]
    if args.workload in ("qwen_decode", "all"):
        extra["qwen_decode"] = [r for d in (1, 2) for r in qwen_decode(args, N, d, (N.ACT_F32, N.ACT_I8))]
    if args.workload in ("q8_vocab", "q4_sweep", "all"):
        extra["q8_vocab_m1"] = measure_cases(args, N, [(1, n, k, 1) for n, k in Q8_VOCAB], N.ACT_I8, "q8_vocab")
        extra["q8_vocab_m1_f32_bit_exact"] = measure_cases(args, N, [(1, n, k, 1) for n, k in Q8_VOCAB], N.ACT_F32,
                                                           "q8_vocab_f32")
    if args.workload in ("verify", "q4_sweep", "all"):
        extra["verify"] = measure_cases(args, N, [(d, n, k, m) for d in (1, 2) for n, k in VERIFY_SHAPES[:2]
                                                  for m in (2, 4, 8, 16)], N.ACT_I8, "verify")
    if args.workload in ("decode_f32", "all"):
        extra["decode_f32_bit_exact"] = measure_cases(args, N, [(d, n, k, 1) for d in (1, 2) for n, k in GEMMA_DECODE],
                                                      N.ACT_F32, "decode_f32")
    if args.workload in ("fused_norm", "all"):
        extra["fused_norm"] = fused_norm(args, N)
    if args.workload in ("i8_m1", "all"):
        # The one-vector int8 GEMV at Llama-3-8B's and Qwen2.5-7B's matrices,
        # both formats (the staged grid-stride kernel takes the Q8 4096- and
        # 14336-column shapes and both 18944-column ones).
        extra["i8_m1"] = measure_cases(args, N, [(d, n, k, 1) for d in (1, 2) for n, k in I8_M1_SHAPES], N.ACT_I8,
                                       "i8_m1")
    if args.workload in ("f32_m1", "all"):
        # The bit-exact one-vector GEMV (the drop-in mode) at the streamed
        # kernel's shapes, both formats.
        extra["f32_m1"] = measure_cases(args, N, [(d, n, k, 1) for d in (1, 2) for n, k in F32_M1_SHAPES],
                                        N.ACT_F32, "f32_m1")
    if args.workload in ("i8_prologue", "all"):
        extra["i8_prologue"] = i8_prologue(args, N)
    if args.workload in ("bf16", "all"):
        extra["bf16_bit_exact"] = measure_cases(args, N, [(3, n, k, m) for n, k in BF16_SHAPES for m in (1, 4)],
                                                N.ACT_F32, "bf16")
    if args.workload in ("q4_sweep", "all"):
        # The same decode again after everything above (device only), with
        # the shader clock it ran at.
        extra["gemma3_1b_decode_late"] = gemma_decode(args, N, cpu=False)
    if result is None:
        print(json.dumps(dict(workload=args.workload, results=extra)), flush=True)
        return
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle as O  # the CPU baseline leg only
        cpu = cpu_baseline(O, cpu_inputs(N, O, inputs))
    line = dict(metric=result["metric"], value=result["value"], unit=result["unit"], n_gpus=1, steps=args.steps,
                warmup=args.warmup, ms_per_step=round(result["ms_per_step"], 5), higher_is_better=True,
                scaling="weak", vs_baseline=None, dtype=result["dtype"], data="synthetic (seeded)",
                config=result["config"], roofline=result["roofline"], cpu_baseline=cpu,
                per_shape=result["per_shape"])
    pk = extra.get("peaks")
    if pk:
        line["roofline"]["measured_peak"] = pk["hbm_read_1gib_gbs"]
        line["roofline"]["frac_of_measured"] = round(result["roofline"]["achieved"] / pk["hbm_read_1gib_gbs"], 4)
    if extra:
        line["extra"] = extra
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
