"""The GGUF writer and reader of nncpu_amd.gguf and the seeded generator of
the config-1 model file (CPU only).

The writer mirrors the reference's test writer (crates/nncpu/src/gguf.rs:
656-778); its round trip restates gguf.rs:784-807. The generator is the
reference's test Rng (kernels/tests.rs:9-50), checked bit for bit against
the oracle's restatement of it.
"""
import os
import struct

import numpy as np
import pytest

from nncpu_amd import gguf as G


def test_round_trip(tmp_path):
    # gguf.rs:784-807
    w = G.GgufWriter()
    w.str("general.architecture", "llama").u32("llama.block_count", 2).f32("llama.rope.freq_base", 10000.0)
    w.strs("tokenizer.ggml.tokens", ["a", "b"])
    data = np.arange(1, 9, dtype=np.float32)
    w.tensor("w", [4, 2], G.GGML_F32, data.nbytes, data.tobytes())
    path = str(tmp_path / "round_trip.gguf")
    w.write(path)
    f = G.GgufFile(path)
    assert f.kv["general.architecture"] == "llama"
    assert f.kv["llama.block_count"] == 2
    assert f.kv["llama.rope.freq_base"] == 10000.0
    assert f.kv["tokenizer.ggml.tokens"] == ["a", "b"]
    t = f.tensors["w"]
    assert t.data.size == 32 and (t.rows, t.cols) == (2, 4)
    assert struct.unpack("<f", bytes(t.data[4:8]))[0] == 2.0


def test_layout_matches_the_reference_writer(tmp_path):
    # Offsets are each tensor's bytes rounded up to 32; the data section
    # starts at the next multiple of 32 after the tensor infos (gguf.rs:748-767).
    w = G.GgufWriter().u32("k", 7)
    a = np.arange(5, dtype=np.float32)  # 20 bytes: the next tensor starts 32 later
    b = np.arange(3, dtype=np.float32)
    w.tensor("a", [5], G.GGML_F32, a.nbytes, a.tobytes()).tensor("b", [3], G.GGML_F32, b.nbytes, b.tobytes())
    path = str(tmp_path / "t.gguf")
    w.write(path)
    raw = open(path, "rb").read()
    magic, ver, nt, nkv = struct.unpack_from("<IIQQ", raw, 0)
    assert (magic, ver, nt, nkv) == (G.GGUF_MAGIC, 3, 2, 1)
    f = G.GgufFile(path)
    base = len(raw) - 32 - 12  # b starts at offset 32 of the data section and holds 12 bytes
    assert base % 32 == 0
    assert np.array_equal(np.frombuffer(raw[base:base + 20], np.float32), a)
    assert np.array_equal(np.asarray(f.tensors["b"].data).view(np.float32), b)


def test_rejects_bad_input(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGUX\x03\0\0\0" + b"\0" * 16)
    with pytest.raises(ValueError):
        G.GgufFile(str(p))


def test_generator_is_the_reference_rng(oracle):
    # Chunk c of a tensor is the reference's Rng(seed + c).normals (tests.rs:9-50).
    seed, n = 0x6E33A, 3 * G.RNG_CHUNK + 12345
    got = G.normals(seed, n, 0.0, 0.02, threads=3)
    for c in range(4):
        want = oracle.Rng(seed + c).normals(min(G.RNG_CHUNK, n - c * G.RNG_CHUNK), 0.02)
        assert np.array_equal(got[c * G.RNG_CHUNK:c * G.RNG_CHUNK + want.size].view(np.uint32), want.view(np.uint32))
    assert np.array_equal(G.normals(seed, n, 0.0, 0.02, threads=1).view(np.uint32), got.view(np.uint32))
    one = G.normals(seed, 1000, 1.0, 0.1)
    z = oracle.Rng(seed).normals(1000, 0.1)
    assert np.array_equal(one, (np.float32(1.0) + z).astype(np.float32))


def test_bf16_bits_round_to_nearest_even(oracle):
    x = np.array([1.0, 1.00390625, 1.01171875, -2.5, 3e38], np.float32)
    x = np.concatenate([x, oracle.Rng(9).normals(1000, 3.0)])
    assert np.array_equal(G.bf16_bits(x), oracle.f32_array_to_bf16(x))


def test_write_gemma3_small(tmp_path, oracle):
    from nncpu_amd.gemma import gemma3_1b_config
    cfg = gemma3_1b_config(n_ctx=64, n_layer=2, n_vocab=512)
    path = str(tmp_path / "g.gguf")
    G.write_gemma3(path, cfg, seed=5)
    f = G.GgufFile(path)
    assert f.kv["general.architecture"] == "gemma3"
    assert f.kv["gemma3.block_count"] == 2 and f.kv["gemma3.embedding_length"] == 1152
    assert len(f.kv["tokenizer.ggml.tokens"]) == 512
    names = G.gemma3_tensors(cfg)
    assert set(f.tensors) == {n for n, *_ in names}
    for i, (name, rows, cols, role) in enumerate(names):
        t = f.tensors[name]
        assert (t.rows, t.cols) == (rows, cols), name
        if role == "norm":
            assert t.ggml_type == G.GGML_F32
        else:
            assert t.ggml_type == G.GGML_BF16
            if i < 3:  # token_embd, the first norm, blk.0.attn_q: the seeds' values
                want = G.bf16_bits(G.normals((5 << 32) + (i << 24), rows * cols, 0.0, 0.02))
                assert np.array_equal(np.asarray(t.data).view(np.uint16), want), name
    os.remove(path)


def _gemma_kv(**extra):
    kv = {"gemma3.embedding_length": 1152, "gemma3.attention.head_count": 4, "gemma3.attention.head_count_kv": 1,
          "gemma3.attention.key_length": 256, "gemma3.block_count": 12, "gemma3.feed_forward_length": 6912,
          "gemma3.rope.freq_base": 1e6, "gemma3.attention.sliding_window": 512,
          "tokenizer.ggml.tokens": ["a"] * 64}
    kv.update({"gemma3." + k: v for k, v in extra.items()})
    return kv


def test_gemma3_hyperparameters_follow_the_loader():
    # model/load.rs:486-493, 550-554, 1147-1165: the local RoPE base (stored
    # or gemma3's 10000), the sliding pattern (every 6th layer global by
    # default, a period or a per-layer array), no sliding layer when the
    # window is 0, and the models these forwards cannot run are refused.
    from nncpu_amd.gemma import gemma3_config_from_kv
    c = gemma3_config_from_kv(_gemma_kv(), 256, 1)
    assert (c.swa_period, c.window, c.rope_base, c.rope_base_swa) == (6, 512, 1e6, 10000.0)
    c = gemma3_config_from_kv(_gemma_kv(**{"rope.freq_base_swa": 5e4, "attention.sliding_window_pattern": 4}), 256, 1)
    assert (c.swa_period, c.rope_base_swa) == (4, 5e4)
    pat = np.array([(i + 1) % 3 != 0 for i in range(12)], np.int32)
    assert gemma3_config_from_kv(_gemma_kv(**{"attention.sliding_window_pattern": pat}), 256, 1).swa_period == 3
    c = gemma3_config_from_kv(_gemma_kv(**{"attention.sliding_window": 0}), 256, 1)
    assert c.swa_period == 0  # no layer slides: every layer keeps the global base
    bad = [{"rope.scaling.type": "linear", "rope.scaling.factor": 8.0},
           {"attention.sliding_window_pattern": np.array([1, 0] + [1] * 10, np.int32)},
           {"attention.sliding_window_pattern": 0}]
    for extra in bad:
        with pytest.raises(ValueError):
            gemma3_config_from_kv(_gemma_kv(**extra), 256, 1)
