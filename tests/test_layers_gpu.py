"""The device forward (nncpu_amd/host/layers_gpu.hip) against the CPU forward
(nncpu_amd/host/gemma3.cpp, crates/nncpu/src/model/forward.rs restated) for
Qwen2, Llama and Gemma-3 layers.

Both runs use the library's bit-exact f32 matmul (nncpu's own kernel, bit for
bit), so everything between the matmuls on the device must reproduce the CPU
forward exactly: the greedy tokens, the last token's residual after every
layer of every forward (hashed), and the whole BF16 K/V cache. Prompts run in
16-token batches (session/engine.rs:362-380), then one token per forward;
contexts past 256 keys exercise the blockwise attention merge
(kernels/mod.rs:765-800), a short sliding window a partial first block
(model/embed.rs:14-30).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def N():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import nncpu_amd as N
    N.init(0)
    return N


def run_both(model, prompt, n_gen, fused=False, batch=16):
    print(f"arch {model.cfg.arch} dtype {model.cfg.wtype} prompt {len(prompt)} gen {n_gen} fused {fused}", flush=True)
    tc, hc, kc, vc = model.cpu_generate(prompt, n_gen, batch=batch)
    dev = model.device(n_batch=batch, fused=fused)
    try:
        tg, hg, kg, vg = dev.generate(prompt, n_gen, batch=batch)
    finally:
        dev.free()
    assert np.array_equal(tg, tc), (tg, tc)
    assert np.array_equal(hg, hc), np.argwhere(hg != hc)[:5]
    assert np.array_equal(kg, kc), np.argwhere(kg != kc)[:5]
    assert np.array_equal(vg, vc), np.argwhere(vg != vc)[:5]
    return tc


def test_qwen2_layers_match_cpu_forward(N):
    # Qwen2: q / k / v biases, NeoX RoPE, SiLU(gate) * up, GQA 2 query heads
    # per KV head; 270 prompt tokens, so the later tokens attend over two
    # 256-key blocks merged with glibc's expf.
    from nncpu_amd.models import Model, qwen2_config
    cfg = qwen2_config(n_layer=2, n_embd=256, n_head=4, n_kv=2, n_ff=512, n_vocab=1024, n_ctx=320)
    model = Model.random(cfg, seed=0x0E2)
    prompt = np.random.default_rng(1).integers(0, cfg.n_vocab, 270).astype(np.int32)
    run_both(model, prompt, 6)


def test_llama_layers_match_cpu_forward(N):
    # Llama: adjacent-pair RoPE, no biases, 3 query heads per KV head, an
    # untied embedding table.
    from nncpu_amd.models import Model, llama_config
    cfg = llama_config(n_layer=2, n_embd=384, n_head=6, n_kv=2, n_ff=1024, n_vocab=2048, n_ctx=64)
    model = Model.random(cfg, seed=0x11A, tied=False)
    prompt = np.random.default_rng(2).integers(0, cfg.n_vocab, 21).astype(np.int32)
    run_both(model, prompt, 8)


def test_qwen3_layers_match_cpu_forward(N):
    # Qwen3: per-head q / k RMSNorm (forward.rs:274-290) with NeoX RoPE, no
    # biases, head_dim 128 (past n_embd / n_head).
    from nncpu_amd.models import Model, qwen3_config
    cfg = qwen3_config(n_layer=2, n_embd=256, n_head=4, n_kv=2, n_ff=512, n_vocab=768, n_ctx=48, head_dim=128)
    model = Model.random(cfg, seed=0x03)
    prompt = np.random.default_rng(6).integers(0, cfg.n_vocab, 18).astype(np.int32)
    run_both(model, prompt, 5)


def test_llama_rope_frequency_factors(N):
    # Llama 3's RoPE frequency factors divide each pair's angle (kernels/mod.rs
    # 712-716), in both forwards' tables.
    from nncpu_amd.models import Model, llama_config
    cfg = llama_config(n_layer=1, n_embd=256, n_head=4, n_kv=4, n_ff=512, n_vocab=512, n_ctx=48)
    model = Model.random(cfg, seed=0x3F)
    model.rope_ff = np.linspace(1.0, 8.0, cfg.head_dim // 2).astype(np.float32)
    prompt = np.random.default_rng(3).integers(0, cfg.n_vocab, 17).astype(np.int32)
    run_both(model, prompt, 4)


def test_gemma3_layers_match_cpu_forward(N):
    # Gemma-3 through the generic kernels: embedding scale, per-head q / k
    # RMSNorm, post-attention and post-FFW norms, GELU(gate) * up, head_dim 256,
    # and a 24-key sliding window on every layer but each second one, so
    # from position 24 the sliding layers' spans start past key 0.
    from nncpu_amd.gemma import gemma3_1b_config
    from nncpu_amd.models import Model
    cfg = gemma3_1b_config(n_ctx=64, n_layer=2, n_vocab=1024)
    cfg.window, cfg.swa_period = 24, 2
    model = Model.random(cfg, seed=0x6E3)
    prompt = np.random.default_rng(4).integers(0, cfg.n_vocab, 40).astype(np.int32)
    run_both(model, prompt, 6)


def test_qwen2_q4_and_fused_matrices(N):
    # Q4 weights and embedding table; q / k / v and gate / up uploaded as one
    # matrix each (concat_rows): the same rows, so the same bits.
    from nncpu_amd import Q4S
    from nncpu_amd.models import Model, qwen2_config
    cfg = qwen2_config(n_layer=2, n_embd=256, n_head=4, n_kv=1, n_ff=768, n_vocab=640, n_ctx=48)
    model = Model.random(cfg, seed=0x44, dtype=Q4S)
    prompt = np.random.default_rng(5).integers(0, cfg.n_vocab, 19).astype(np.int32)
    t = run_both(model, prompt, 5)
    t2 = run_both(model, prompt, 5, fused=True)
    assert np.array_equal(t, t2)


@pytest.mark.parametrize("size", ["small", "wide"])
def test_fused_norm_decode(N, size):
    # One-token f32 forwards with fused q / k / v and gate / up: each
    # residual add and RMSNorm runs in the next matmul's prologue
    # (nnh_gemv_rmsnorm_dev; the residual stream alternates between two
    # buffers). Tokens, per-layer states and K/V caches equal the CPU
    # forward's, eagerly and from decode-graph replays, and the unfused
    # run's. "wide": d 2048 and FFN 6144, so q / k / v takes the streamed
    # kernel's prologue and gate / up (12288 rows) the tall kernel's;
    # "small": the norm kernel before the plain gemv.
    import torch
    from nncpu_amd.models import Model, llama_config, qwen2_config
    if size == "wide":
        cfg = qwen2_config(n_layer=2, n_embd=2048, n_head=16, n_kv=2, n_ff=6144, n_vocab=1024, n_ctx=64,
                           head_dim=128)
        model = Model.random(cfg, seed=0x7E1)
    else:
        cfg = llama_config(n_layer=2, n_embd=384, n_head=6, n_kv=2, n_ff=1024, n_vocab=1024, n_ctx=64)
        model = Model.random(cfg, seed=0x7E2, tied=False)
    prompt = np.random.default_rng(11).integers(0, cfg.n_vocab, 21).astype(np.int32)
    n_gen = 8
    tc = run_both(model, prompt, n_gen, fused=True)
    s = torch.cuda.Stream()
    dev = model.device(n_batch=16, stream=s.cuda_stream, fused=True)
    try:
        tg, _, kg, vg = dev.generate_graph(prompt, n_gen, stream=s)
        dev.set_fused_norm(False)
        tu, hu, ku, vu = dev.generate(prompt, n_gen)
        dev.set_fused_norm(True)
        tf, hf, kf, vf = dev.generate(prompt, n_gen)
    finally:
        dev.free()
    assert np.array_equal(tg, tc) and np.array_equal(tu, tc) and np.array_equal(tf, tc)
    assert np.array_equal(hf, hu), np.argwhere(hf != hu)[:5]
    assert np.array_equal(kf, ku) and np.array_equal(vf, vu) and np.array_equal(kg, kf) and np.array_equal(vg, vf)


@pytest.mark.parametrize("dtype", [1, 2])
def test_fused_norm_decode_i8(N, dtype):
    # One-token int8 forwards with fused q / k / v and gate / up at a width
    # whose rows take the fused int8 kernel (d 3200: 100 blocks, the xor lane
    # tree): each residual add, RMSNorm and Q8_0 quantizer runs in the next
    # matmul's prologue (nnh_gemv_rmsnorm_act_dev). Tokens, per-layer states
    # and K/V caches equal the run with the norm kernels, eagerly and from
    # decode-graph replays, and the tokens and caches equal the CPU forward's
    # in the int8 mode.
    import torch
    from nncpu_amd import ACT_I8, Q4S, Q8_0
    from nncpu_amd.models import Model, qwen2_config
    cfg = qwen2_config(n_layer=2, n_embd=3200, n_head=25, n_kv=5, n_ff=3200, n_vocab=1024, n_ctx=64, head_dim=128)
    model = Model.random(cfg, seed=0x7E3 + dtype, dtype=Q8_0 if dtype == 1 else Q4S)
    prompt = np.random.default_rng(12).integers(0, cfg.n_vocab, 21).astype(np.int32)
    n_gen = 8
    print(f"fused norm i8 dtype {dtype}", flush=True)
    tc, _, kc, vc = model.cpu_generate(prompt, n_gen, act=ACT_I8)
    s = torch.cuda.Stream()
    dev = model.device(n_batch=16, act=ACT_I8, stream=s.cuda_stream, fused=True)
    try:
        tg, _, kg, vg = dev.generate_graph(prompt, n_gen, stream=s)
        dev.set_fused_norm(False)
        tu, hu, ku, vu = dev.generate(prompt, n_gen)
        dev.set_fused_norm(True)
        tf, hf, kf, vf = dev.generate(prompt, n_gen)
    finally:
        dev.free()
    assert np.array_equal(tu, tc) and np.array_equal(tf, tc) and np.array_equal(tg, tc), (tf, tc)
    assert np.array_equal(hf, hu), np.argwhere(hf != hu)[:5]
    assert np.array_equal(kf, ku) and np.array_equal(vf, vu) and np.array_equal(kg, kf) and np.array_equal(vg, vf)
    assert np.array_equal(kf, kc) and np.array_equal(vf, vc)


def test_forward_dev_graph_replay(N):
    # nngl_forward_dev allocates nothing: one prefill captured in a HIP graph
    # and replayed (eager work between replays) gives the eager hidden states.
    import torch
    from nncpu_amd.models import Model, qwen2_config
    cfg = qwen2_config(n_layer=2, n_embd=256, n_head=4, n_kv=2, n_ff=512, n_vocab=512, n_ctx=64)
    model = Model.random(cfg, seed=0x6A)
    s = torch.cuda.Stream()
    dev = model.device(n_batch=32, stream=s.cuda_stream)
    try:
        tok = torch.randint(0, cfg.n_vocab, (32,), dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        dev.forward_dev(tok.data_ptr(), 32, 0)
        want, want_st = dev.read(32)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            dev.forward_dev(tok.data_ptr(), 32, 0)
        for i in range(3):
            junk = torch.randn(1 << 20, device="cuda")
            (junk * 2).sum().item()
            g.replay()
            torch.cuda.synchronize()
            got, got_st = dev.read(32)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), i
            assert np.array_equal(got_st.view(np.uint32), want_st.view(np.uint32)), i
    finally:
        dev.free()


def test_decode_graph_matches_eager(N):
    # One decode step (the token, position and step counter in device memory)
    # captured in a HIP graph and replayed per token: the same tokens and the
    # same K/V cache as the eager decode, across a 256-key block boundary.
    import torch
    from nncpu_amd.models import Model, qwen2_config
    cfg = qwen2_config(n_layer=2, n_embd=256, n_head=4, n_kv=2, n_ff=512, n_vocab=1024, n_ctx=300)
    model = Model.random(cfg, seed=0x5D)
    prompt = np.random.default_rng(7).integers(0, cfg.n_vocab, 250).astype(np.int32)
    n_gen = 20
    print("decode graph vs eager", flush=True)
    tc, _, kc, vc = model.cpu_generate(prompt, n_gen)
    s = torch.cuda.Stream()
    dev = model.device(n_batch=16, stream=s.cuda_stream)
    try:
        tg, _, kg, vg = dev.generate_graph(prompt, n_gen, stream=s)
        te, _, ke, ve = dev.generate(prompt, n_gen)
    finally:
        dev.free()
    assert np.array_equal(te, tc) and np.array_equal(ke, kc) and np.array_equal(ve, vc)
    assert np.array_equal(tg, tc), (tg, tc)
    assert np.array_equal(kg, kc) and np.array_equal(vg, vc)


@pytest.mark.parametrize("case", ["qwen2_q4", "llama_q8", "gemma3_q8"])
def test_i8_producer_quantization_matches_library_quantizer(N, case):
    # One-token forwards in the int8 mode: the norm, attention-merge and
    # activation kernels write each matmul's int8 input themselves
    # (nngl_set_fused_quant). The library's quantizer on the same f32 rows
    # gives the same bits, so the tokens, per-layer states and K/V caches
    # equal the unfused run's, eagerly and from decode-graph replays (whose
    # lm_head reads the final norm's int8 row). The 17- and 33-token prompts
    # end in a one-token prompt batch.
    import torch
    from nncpu_amd import ACT_I8, Q4S
    from nncpu_amd.gemma import gemma3_1b_config
    from nncpu_amd.models import Model, llama_config, qwen2_config
    if case == "qwen2_q4":
        cfg = qwen2_config(n_layer=2, n_embd=256, n_head=4, n_kv=2, n_ff=512, n_vocab=768, n_ctx=300)
        model, n_prompt = Model.random(cfg, seed=0x7A, dtype=Q4S), 257
    elif case == "llama_q8":
        cfg = llama_config(n_layer=2, n_embd=384, n_head=6, n_kv=2, n_ff=1024, n_vocab=1024, n_ctx=64)
        model, n_prompt = Model.random(cfg, seed=0x7B, tied=False), 17
    else:
        cfg = gemma3_1b_config(n_ctx=64, n_layer=2, n_vocab=1024)
        cfg.window, cfg.swa_period = 24, 2
        model, n_prompt = Model.random(cfg, seed=0x7C), 33
    prompt = np.random.default_rng(8).integers(0, cfg.n_vocab, n_prompt).astype(np.int32)
    n_gen = 12
    print(f"{case}: prompt {n_prompt} gen {n_gen}", flush=True)
    s = torch.cuda.Stream()
    dev = model.device(n_batch=16, act=ACT_I8, stream=s.cuda_stream, fused=case == "qwen2_q4")
    try:
        dev.set_fused_quant(False)
        t0, h0, k0, v0 = dev.generate(prompt, n_gen)
        g0, _, gk0, gv0 = dev.generate_graph(prompt, n_gen, stream=s)
        dev.set_fused_quant(True)
        t1, h1, k1, v1 = dev.generate(prompt, n_gen)
        g1, _, gk1, gv1 = dev.generate_graph(prompt, n_gen, stream=s)
    finally:
        dev.free()
    assert np.array_equal(t1, t0), (t1, t0)
    assert np.array_equal(h1, h0), np.argwhere(h1 != h0)[:5]
    assert np.array_equal(k1, k0) and np.array_equal(v1, v0)
    assert np.array_equal(g0, t0) and np.array_equal(gk0, k0) and np.array_equal(gv0, v0)
    assert np.array_equal(g1, t0), (g1, t0)
    assert np.array_equal(gk1, k0) and np.array_equal(gv1, v0)


def test_qwen25_7b_width_layer_prefill_512(N):
    # One layer at Qwen2.5-7B's full width (d 3584, 28 query / 4 KV heads of
    # 128 = 7 per KV head, FFN 18944, q/k/v biases, NeoX RoPE base 1e6), the
    # 512-token prompt in one forward as the timed prefill runs it, then
    # greedy tokens: hidden states and K/V cache identical to the CPU forward
    # (forward.rs:197-439,719-841 restated), matmuls bit-exact in both.
    from nncpu_amd.models import Model, qwen25_7b_config
    cfg = qwen25_7b_config(n_ctx=520, n_layer=1)
    cfg.n_vocab = 2048
    model = Model.random(cfg, seed=0x7B7)
    prompt = np.random.default_rng(9).integers(0, cfg.n_vocab, 512).astype(np.int32)
    run_both(model, prompt, 4, batch=512)


def test_qwen2_seven_query_heads_per_kv_head(N):
    # Qwen2.5-7B's grouping, 7 query heads per KV head at head_dim 128 (4
    # tokens per attention tile, 28 of its 32 query rows used), over more
    # than one 256-key block, in 16-token prompt batches, one-token decodes
    # and decode-graph replays.
    import torch
    from nncpu_amd.models import Model, qwen2_config
    cfg = qwen2_config(n_layer=2, n_embd=896, n_head=7, n_kv=1, n_ff=1024, n_vocab=1024, n_ctx=300, head_dim=128)
    model = Model.random(cfg, seed=0x77)
    prompt = np.random.default_rng(10).integers(0, cfg.n_vocab, 270).astype(np.int32)
    tc = run_both(model, prompt, 8)
    _, _, kc, vc = model.cpu_generate(prompt, 8)
    s = torch.cuda.Stream()
    dev = model.device(n_batch=16, stream=s.cuda_stream)
    try:
        tg, _, kg, vg = dev.generate_graph(prompt, 8, stream=s)
    finally:
        dev.free()
    assert np.array_equal(tg, tc), (tg, tc)
    assert np.array_equal(kg, kc) and np.array_equal(vg, vc)
