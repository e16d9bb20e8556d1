"""Gemma-3-1B-architecture greedy decode with the GPU matmul
is token-identical to the same decode with nncpu's CPU gemv.

The model is the random-init GGUF from a seed (nncpu_amd.gguf.write_gemma3:
26 layers, d 1152, FFN 6912, 4 / 1 heads, head_dim 256, vocab 262144, BF16
matrices drawn from the reference's test generator), loaded as nncpu loads
it: each matrix decoded and re-encoded to Q8_0 (on the device, through
nnh_upload_gguf; checked bit for bit against the oracle's encoder below); a
32-token uniform-random prompt evaluated in 16-token batches, then 128
greedy tokens. The CPU run
uses the AVX2 restatement of nncpu's gemv (bit-equal to the scalar oracle,
tests/test_oracle.py) on the same weight bytes; both runs share the CPU
forward (nncpu_amd/host/gemma3.cpp). Tokens and the per-layer residual
hashes of every forward call must match exactly.
"""
import ctypes as C
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class OrModelTable(C.Structure):
    _fields_ = [("n", C.c_int), ("dtype", C.c_int), ("bufs", C.POINTER(C.c_void_p)),
                ("rows", C.POINTER(C.c_size_t)), ("cols", C.POINTER(C.c_size_t))]


@pytest.fixture(scope="module")
def model():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import nncpu_amd as N
    from nncpu_amd.gemma import Gemma3, gemma3_1b_gguf
    N.init(0)
    print("writing / loading the GGUF", flush=True)
    return Gemma3.from_gguf(gemma3_1b_gguf(), n_ctx=256)


def test_gguf_load_reencodes_like_nncpu(oracle, model):
    # The device decode + re-encode of a BF16 GGUF matrix (load.rs:182-243)
    # gives the oracle encoder's bytes for the same decoded values.
    from nncpu_amd.gemma import gemma3_1b_gguf
    from nncpu_amd.gguf import GgufFile
    f = GgufFile(gemma3_1b_gguf())
    for idx, name in ((0, "blk.0.attn_q.weight"), (7 * 3 + 6, "blk.3.ffn_down.weight")):
        t = f.tensors[name]
        vals = oracle.bf16_array_to_f32(np.asarray(t.data).view(np.uint16)).reshape(t.rows, t.cols)
        want = oracle.QMatrix.from_f32(1, vals).buf
        assert np.array_equal(model.weights[idx].download(), want), name


def cpu_generate(oracle, model, prompt, n_gen):
    bufs = [w.download() for w in model.weights]
    arr = (C.c_void_p * len(bufs))(*[b.ctypes.data for b in bufs])
    rows = (C.c_size_t * len(bufs))(*[r for r, _ in model.shapes])
    cols = (C.c_size_t * len(bufs))(*[c for _, c in model.shapes])
    table = OrModelTable(n=len(bufs), dtype=model.cfg.wtype, bufs=C.cast(arr, C.POINTER(C.c_void_p)),
                         rows=C.cast(rows, C.POINTER(C.c_size_t)), cols=C.cast(cols, C.POINTER(C.c_size_t)))
    oracle.avx_set_threads(8)
    gemv = C.cast(oracle.lib().or_model_gemv_cb, C.c_void_p).value
    out = model.generate(prompt, n_gen, gemv, None, C.pointer(table))
    del bufs
    return out


PROMPT_LEN, N_GEN = 32, 128


@pytest.fixture(scope="module")
def cpu_run(oracle, model):
    from nncpu_amd.gemma import random_prompt
    prompt = random_prompt(PROMPT_LEN, model.cfg.n_vocab)
    print("cpu decode", flush=True)
    tc, hc, tpc, tdc = cpu_generate(oracle, model, prompt, N_GEN)
    print(f"cpu: prefill {tpc:.3f}s decode {tdc:.3f}s ({(N_GEN - 1) / tdc:.1f} tok/s)", flush=True)
    return prompt, tc, hc


def check_same(model, tg, hg, tc, hc, n_fwd=2 + N_GEN - 1):
    assert len(hg) == len(hc) == n_fwd * model.cfg.n_layer
    assert np.array_equal(tg, tc), np.nonzero(tg != tc)[0][:5]
    assert np.array_equal(hg, hc), np.nonzero(hg != hc)[0][:5]
    # Random weights settle greedy decoding on few tokens, but every step's
    # hidden state is new: the last layer's hashes are all distinct.
    last = hg[model.cfg.n_layer - 1::model.cfg.n_layer]
    assert len(set(last.tolist())) == len(last)


def test_gemma3_1b_decode_token_identical(model, cpu_run):
    prompt, tc, hc = cpu_run
    print("gpu decode (matmuls on the GPU)", flush=True)
    tg, hg, tpg, tdg = model.generate_gpu(prompt, N_GEN)
    print(f"gpu: prefill {tpg:.3f}s decode {tdg:.3f}s ({(N_GEN - 1) / tdg:.1f} tok/s)", flush=True)
    check_same(model, tg, hg, tc, hc)
    sys.stdout.flush()


def test_gemma3_1b_device_decode_token_identical(model, cpu_run):
    # The decode step resident on the GPU (norms, RoPE, attention, GELU as
    # HIP kernels; one step captured in a HIP graph and replayed per token):
    # the same tokens and per-layer hidden states as the CPU run, including
    # every graph replay.
    prompt, tc, hc = cpu_run
    print("device-resident decode", flush=True)
    tg, hg, tpg, tdg = model.generate_device(prompt, N_GEN)
    print(f"device: prefill {tpg:.3f}s decode {tdg:.3f}s ({(N_GEN - 1) / tdg:.1f} tok/s)", flush=True)
    check_same(model, tg, hg, tc, hc)
    # A second run replays the captured graph from a fresh prefill.
    tg2, hg2, _, tdg2 = model.generate_device(prompt, N_GEN)
    print(f"device (graph reused): decode {tdg2:.3f}s ({(N_GEN - 1) / tdg2:.1f} tok/s)", flush=True)
    check_same(model, tg2, hg2, tc, hc)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def long_model():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import nncpu_amd as N
    from nncpu_amd.gemma import Gemma3, gemma3_1b_gguf
    N.init(0)
    return Gemma3.from_gguf(gemma3_1b_gguf(), n_ctx=768)


def test_device_decode_past_one_block_and_the_window(oracle, long_model):
    # A 500-token prompt, then 40 tokens: positions 500..539. Every layer
    # attends over two or three 256-key blocks, merged as attn_merge does
    # (kernels/mod.rs:765-800, forward.rs:387-414), and from position 512 on
    # the sliding layers' 512-key window starts past key 0, so their first
    # block is partial (model/embed.rs:14-30).
    from nncpu_amd.gemma import random_prompt
    n_prompt, n_gen = 500, 40
    prompt = random_prompt(n_prompt, long_model.cfg.n_vocab, seed=0x1B0C)
    print("cpu decode, long context", flush=True)
    tc, hc, _, _ = cpu_generate(oracle, long_model, prompt, n_gen)
    print("device decode, long context", flush=True)
    tg, hg, _, tdg = long_model.generate_device(prompt, n_gen)
    print(f"device: {(n_gen - 1) / tdg:.1f} tok/s at positions {n_prompt}..{n_prompt + n_gen - 1}", flush=True)
    check_same(long_model, tg, hg, tc, hc, n_fwd=(n_prompt + 15) // 16 + n_gen - 1)


@pytest.fixture(scope="module")
def q4_model():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import nncpu_amd as N
    from nncpu_amd.gemma import Gemma3, gemma3_1b_gguf
    N.init(0)
    return Gemma3.from_gguf(gemma3_1b_gguf(), n_ctx=256, dtype=N.Q4S)


def test_gemma3_1b_q4_device_decode_token_identical(oracle, q4_model):
    # The same GGUF re-encoded to nncpu's Q4 (every matrix and the tied
    # embedding, as load.rs:186-197 does for WeightFormat::Q4): the embedding
    # row is embed_row_q4 (kernels/mod.rs:934-954), every matmul q4_row plus
    # the bias term (scalar.rs:654-674, 708-740). The device decode against
    # the CPU forward with the AVX2 restatement of nncpu's Q4 gemv.
    from nncpu_amd.gemma import random_prompt
    n_gen = 64
    prompt = random_prompt(PROMPT_LEN, q4_model.cfg.n_vocab, seed=0x4B17)
    print("cpu decode, Q4", flush=True)
    tc, hc, _, _ = cpu_generate(oracle, q4_model, prompt, n_gen)
    print("device decode, Q4", flush=True)
    tg, hg, _, tdg = q4_model.generate_device(prompt, n_gen)
    print(f"device, Q4: {(n_gen - 1) / tdg:.1f} tok/s", flush=True)
    check_same(q4_model, tg, hg, tc, hc, n_fwd=2 + n_gen - 1)
    # The matmuls through the library's Q4 path (host round trips) agree too.
    tg2, hg2, _, _ = q4_model.generate_gpu(prompt, n_gen)
    check_same(q4_model, tg2, hg2, tc, hc, n_fwd=2 + n_gen - 1)
