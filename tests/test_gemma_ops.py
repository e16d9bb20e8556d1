"""The model harness's non-matmul ops against the reference's own op tests
(CPU only).

nncpu_amd/host/gemma3.cpp restates the forward's non-matmul kernels of
crates/nncpu/src/kernels/scalar.rs and kernels/mod.rs; the device decode
step repeats them operation for operation and is checked bit for bit against
this forward (tests/test_gemma_decode_gpu.py). Here the same functions, as the
harness library exports them, meet the checks kernels/tests.rs applies to
the reference's kernels: known values, a direct f64 (or libm) evaluation at
the reference's tolerance, and the invariants. Data comes from the
reference's test generator (xorshift64*, kernels/tests.rs:9-50, restated in
the oracle) with the reference's seeds.
"""
import ctypes as C
import math
import os

import numpy as np
import pytest

from conftest import bits, close

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GEMMA_LIB = os.path.join(ROOT, "nncpu_amd", "lib", "libnncpu_gemma.so")


@pytest.fixture(scope="module")
def ops():
    if not os.path.exists(GEMMA_LIB):
        pytest.fail(f"{GEMMA_LIB} is not built")
    L = C.CDLL(GEMMA_LIB)
    vp, sz, f = C.c_void_p, C.c_size_t, C.c_float
    L.nng_op_exp.argtypes = [vp, vp, sz]
    L.nng_op_gelu.argtypes = [vp, sz]
    L.nng_op_gelu_mul.argtypes = [vp, vp, sz]
    L.nng_op_rmsnorm_gamma.argtypes = [vp, vp, sz, sz, vp, f]
    L.nng_op_rope_neox.argtypes = [vp, sz, sz, sz, f, f]
    L.nng_op_rope.argtypes = [vp, sz, sz, sz, f, f, C.c_int, vp]
    L.nng_op_swiglu.argtypes = [vp, vp, sz]
    L.nng_op_attn_block.argtypes = [vp, sz, vp, vp, sz, sz, sz, sz, f, vp, vp]
    L.nng_op_attn_merge.argtypes = [vp, vp, sz, sz]
    L.nng_op_attn_finish.argtypes = [vp, sz, vp, sz, sz]
    for fn in (L.nng_op_exp, L.nng_op_gelu, L.nng_op_gelu_mul, L.nng_op_rmsnorm_gamma, L.nng_op_rope_neox,
               L.nng_op_rope, L.nng_op_swiglu, L.nng_op_attn_block, L.nng_op_attn_merge, L.nng_op_attn_finish):
        fn.restype = None
    return L


def p(a):
    return a.ctypes.data_as(C.c_void_p)


def f32(a):
    return np.ascontiguousarray(a, np.float32)


def assert_close(got, want, rel, what):
    ok = close(got, want, rel)
    assert ok.all(), (what, np.argwhere(~ok)[:5], np.asarray(got)[~ok][:5], np.asarray(want)[~ok][:5])


# ---- exp (kernels/tests.rs:1261-1271) -------------------------------------------------------

def test_exp_lane_is_accurate(ops):
    x = f32(-87.0 + 175.0 * np.arange(20001, dtype=np.float32) / np.float32(20000.0))
    y = np.empty_like(x)
    ops.nng_op_exp(p(x), p(y), x.size)
    worst = np.max(np.abs(y.astype(np.float64) / np.exp(x.astype(np.float64)) - 1.0))
    assert worst < 1e-6, worst


# ---- GELU (kernels/tests.rs:103-147) ---------------------------------------------------------

GELU_C, GELU_A = np.float32(0.79788456080286535), np.float32(0.044715)


def gelu_ref(v):
    """kernels/tests.rs:73-76 in f32 with libm's tanh."""
    v = f32(v)
    u = GELU_C * (v + GELU_A * v * v * v)
    return f32(np.float32(0.5) * v * (np.float32(1.0) + np.tanh(u)))


def test_gelu_matches_reference(ops, oracle):
    rng = oracle.Rng(0xdead)
    for n in (1024, 1, 7, 13, 1031):
        x = rng.vec(n, -5.0, 5.0)
        y = x.copy()
        ops.nng_op_gelu(p(y), n)
        assert_close(y, gelu_ref(x), 5e-4, f"gelu n={n}")
    out = f32([0.0, 1.0, -1.0, 3.0, -3.0, 6.0, -6.0, 100.0, -100.0])
    ops.nng_op_gelu(p(out), out.size)
    assert close(out[0], 0.0, 1e-6)
    assert close(out[1], 0.841192, 1e-4), out[1]
    assert close(out[2], -0.158808, 1e-4), out[2]
    assert out[7] == 100.0
    assert out[8] == 0.0 and np.signbit(out[8])  # -0.0


def test_gelu_mul_matches_reference(ops, oracle):
    # The gated form of kernels/tests.rs:125-147 that Gemma's MLP uses.
    rng = oracle.Rng(0x5167)
    for n in (257, 8, 5):
        g, u = rng.vec(n, -3.0, 3.0), rng.vec(n, -3.0, 3.0)
        y = g.copy()
        ops.nng_op_gelu_mul(p(y), p(u), n)
        assert_close(y, gelu_ref(g) * u, 5e-4, f"gelu_mul n={n}")
        # the same bits as GELU then a product
        z = g.copy()
        ops.nng_op_gelu(p(z), n)
        assert np.array_equal(bits(y), bits(f32(z * u)))


# ---- RMSNorm (kernels/tests.rs:242-293) -------------------------------------------------------

def dot_f64(a, b):
    return float(np.dot(np.asarray(a, np.float64), np.asarray(b, np.float64)))


def test_rmsnorm_matches_reference(ops, oracle):
    # Plain RMSNorm is the gamma form with gamma = 1 (x * scale * 1.0 is x * scale exactly).
    rng = oracle.Rng(0xcafe)
    for n in (1536, 2560, 256, 13):
        x = rng.vec(n, -3.0, 3.0)
        y = np.zeros(n, np.float32)
        one = np.ones(n, np.float32)
        ops.nng_op_rmsnorm_gamma(p(y), p(x), n, n, p(one), 1e-6)
        scale = np.float32(1.0 / math.sqrt(dot_f64(x, x) / n + 1e-6))
        assert_close(y, f32(x * scale), 1e-5, f"rmsnorm n={n}")
        assert abs(math.sqrt(dot_f64(y, y) / n) - 1.0) < 1e-3
        z = x.copy()
        ops.nng_op_rmsnorm_gamma(p(z), p(z), n, n, p(one), 1e-6)
        assert np.array_equal(bits(z), bits(y))


def test_rmsnorm_gamma_multi_matches_reference(ops, oracle):
    rng = oracle.Rng(0x9a11)
    for groups, dim in ((3, 256), (5, 37), (4, 8), (2, 3)):
        x = rng.vec(groups * dim, -3.0, 3.0)
        gamma = rng.vec(dim, 0.5, 1.5)
        y = np.zeros(groups * dim, np.float32)
        ops.nng_op_rmsnorm_gamma(p(y), p(x), groups * dim, dim, p(gamma), 1e-6)
        for g in range(groups):
            xg = x[g * dim:(g + 1) * dim]
            scale = 1.0 / math.sqrt(dot_f64(xg, xg) / dim + 1e-6)
            want = f32((xg.astype(np.float64) * scale).astype(np.float32) * gamma)
            assert_close(y[g * dim:(g + 1) * dim], want, 1e-5, f"rmsnorm_gamma {groups}x{dim}")
        z = x.copy()
        ops.nng_op_rmsnorm_gamma(p(z), p(z), groups * dim, dim, p(gamma), 1e-6)
        assert np.array_equal(bits(z), bits(y))


# ---- RoPE (kernels/tests.rs:936-992; the NeoX pairing Gemma uses, no frequency factors) ---------

def test_rope_matches_reference(ops, oracle):
    rng = oracle.Rng(0x5051)
    x0 = rng.vec(8 * 64, -1.0, 1.0)
    x = x0.copy()
    ops.nng_op_rope_neox(p(x), 8, 64, 64, 0.0, 10000.0)
    assert_close(x, x0, 1e-6, "rope pos 0")
    h, d, r, pos, base = 4, 64, 32, 17.0, 1e6
    half = r // 2
    x0 = rng.vec(h * d, -1.0, 1.0)
    want = x0.copy().reshape(h, d)
    for i in range(half):
        inv = np.float32(base) ** np.float32(-(2 * i) / r)
        theta = np.float32(pos) * inv
        c, s = np.cos(theta, dtype=np.float32), np.sin(theta, dtype=np.float32)
        a, b = want[:, i].copy(), want[:, i + half].copy()
        want[:, i] = c * a - s * b
        want[:, i + half] = s * a + c * b
    x = x0.copy()
    ops.nng_op_rope_neox(p(x), h, d, r, pos, base)
    assert_close(x, want.ravel(), 1e-5, "rope neox")
    xr, x0r = x.reshape(h, d), x0.reshape(h, d)
    assert np.array_equal(bits(xr[:, r:]), bits(x0r[:, r:])), "pass-through lanes"
    x0 = rng.vec(2 * 16, -1.0, 1.0)
    x = x0.copy()
    ops.nng_op_rope_neox(p(x), 2, 16, 16, 42.0, 10000.0)
    for a, b in zip(x0.reshape(2, 16), x.reshape(2, 16)):
        for i in range(8):
            m0 = a[i] * a[i] + a[i + 8] * a[i + 8]
            m1 = b[i] * b[i] + b[i + 8] * b[i + 8]
            assert abs(m0 - m1) <= 1e-4 * max(m0, 1e-6)


def test_rope_both_pairings_and_frequency_factors(ops, oracle):
    # kernels/tests.rs:947-983: NeoX (Gemma, Qwen) and Norm (Llama's
    # adjacent pairs), n_rot < head_dim, with and without frequency factors
    # (1e30 switches a pair off), against a direct evaluation; the lanes past
    # n_rot pass through unchanged. The generator continues as the
    # reference's does after its pos-0 vector.
    rng = oracle.Rng(0x5051)
    rng.vec(8 * 64, -1.0, 1.0)
    h, d, r, pos, base = 4, 64, 32, 17.0, 1e6
    half = r // 2
    ff = f32([1e30 if i == 3 else 1.0 + i * 0.25 for i in range(half)])
    for mode in (0, 1):  # NNG_ROPE_NEOX, NNG_ROPE_NORM
        for factors in (None, ff):
            x0 = rng.vec(h * d, -1.0, 1.0)
            want = x0.copy().reshape(h, d)
            for i in range(half):
                inv = np.float32(base) ** np.float32(-(2 * i) / r)
                theta = np.float32(pos) * inv / (np.float32(1.0) if factors is None else factors[i])
                c, s = np.cos(theta, dtype=np.float32), np.sin(theta, dtype=np.float32)
                pa, pb = (i, i + half) if mode == 0 else (2 * i, 2 * i + 1)
                a, b = want[:, pa].copy(), want[:, pb].copy()
                want[:, pa] = c * a - s * b
                want[:, pb] = s * a + c * b
            x = x0.copy()
            ops.nng_op_rope(p(x), h, d, r, pos, base, mode, None if factors is None else p(factors))
            assert_close(x, want.ravel(), 1e-5, f"rope mode {mode} factors {factors is not None}")
            xr, x0r = x.reshape(h, d), x0.reshape(h, d)
            assert np.array_equal(bits(xr[:, r:]), bits(x0r[:, r:])), "pass-through lanes"
    # A switched-off pair (factor 1e30: theta 0) is unchanged; the Norm
    # pairing rotates lanes 2i, 2i + 1 and leaves the half-split partner alone.
    x0 = rng.vec(d, -1.0, 1.0)
    x = x0.copy()
    ops.nng_op_rope(p(x), 1, d, r, pos, base, 0, p(ff))
    assert x[3] == x0[3] and x[3 + half] == x0[3 + half]
    x = x0.copy()
    ops.nng_op_rope(p(x), 1, d, r, 0.0, base, 1, None)
    assert np.array_equal(bits(x), bits(x0)), "pos 0 is the identity in the Norm pairing too"


# ---- gated activations (kernels/tests.rs:120-146): SiLU(gate) * up ---------------------------

def test_swiglu_matches_reference(ops, oracle):
    rng = oracle.Rng(0x5167)
    for n in (257, 8, 5):
        g, u = rng.vec(n, -3.0, 3.0), rng.vec(n, -3.0, 3.0)
        sig = np.float32(1.0) / (np.float32(1.0) + np.exp(-g.astype(np.float64)).astype(np.float32))
        want = (g * sig * u).astype(np.float32)
        y = g.copy()
        ops.nng_op_swiglu(p(y), p(f32(u)), n)
        assert_close(y, want, 1e-5, f"swiglu n={n}")
    # Known values: silu(0) = 0, silu(x) -> x for large x, -> -0 for very negative x.
    g = f32([0.0, 20.0, -100.0, 1.0])
    u = f32([1.0, 1.0, 1.0, 2.0])
    ops.nng_op_swiglu(p(g), p(u), 4)
    assert g[0] == 0.0 and abs(g[1] - 20.0) < 1e-5 and g[2] == 0.0
    assert abs(g[3] - 2.0 * 0.7310585786) < 1e-6


# ---- attention blocks (kernels/tests.rs:1099-1217), BF16 K/V as Gemma's cache ----------------

def ref_attention(q, k, v, kv_stride, n_keys, hd, group, scale):
    out = np.zeros(group * hd, np.float32)
    K = np.stack([k[t * kv_stride:t * kv_stride + hd] for t in range(n_keys)]).astype(np.float64)
    V = np.stack([v[t * kv_stride:t * kv_stride + hd] for t in range(n_keys)]).astype(np.float64)
    for h in range(group):
        s = K @ q[h * hd:(h + 1) * hd].astype(np.float64) * float(scale)
        e = np.exp(s - s.max())
        out[h * hd:(h + 1) * hd] = (e @ V / e.sum()).astype(np.float32)
    return out


def test_attn_blocks_match_softmax_attention(ops, oracle):
    rng = oracle.Rng(7)
    for hd, group in ((64, 3), (36, 3), (64, 5), (40, 4)):
        n_kv, n_keys = 2, 600
        kv_stride = n_kv * hd
        scale = np.float32(1.0 / math.sqrt(hd))
        q = rng.normals(group * hd, 1.0)
        kf = rng.normals(n_keys * kv_stride, 2.0)
        vf = rng.normals(n_keys * kv_stride, 1.0)
        kb = oracle.f32_array_to_bf16(kf)
        vb = oracle.f32_array_to_bf16(vf)
        kf = oracle.bf16_array_to_f32(kb)
        vf = oracle.bf16_array_to_f32(vb)
        want = ref_attention(q, kf[hd:], vf[hd:], kv_stride, n_keys, hd, group, scale)
        pw = group * (hd + 2)
        blocks = ((0, 100), (100, 256), (356, 244))
        scores = np.zeros(group * 256, np.float32)
        acc, part = np.zeros(pw, np.float32), np.zeros(pw, np.float32)
        parts = []
        for i, (k0, n) in enumerate(blocks):
            off = k0 * kv_stride + hd  # KV head 1
            dst = acc if i == 0 else part
            ops.nng_op_attn_block(p(q), hd, p(kb[off:]), p(vb[off:]), kv_stride, n, hd, group, scale, p(scores),
                                  p(dst))
            parts.append(dst.copy())
            if i > 0:
                ops.nng_op_attn_merge(p(acc), p(part), hd, group)
        out = np.zeros(group * hd, np.float32)
        ops.nng_op_attn_finish(p(out), hd, p(acc), hd, group)
        err = np.abs(out - want)
        assert np.all(err <= 1e-4 * (1.0 + np.abs(want))), (hd, group, err.max())
        # Blocks computed separately, then merged in order: the same bits.
        acc2 = parts[0].copy()
        for pt in parts[1:]:
            ops.nng_op_attn_merge(p(acc2), p(pt), hd, group)
        assert np.array_equal(bits(acc2), bits(acc))


def test_attn_block_softmax_known_values(ops, oracle):
    # The block's softmax (kernels/tests.rs:192-240's checks): with one-hot
    # value rows the output is the softmax of the scores. Scores 1..4, and
    # 256 random scores in [-10, 10) (BF16 keys: the scores are the BF16
    # values), against the f64 softmax.
    hd = 256
    for scores in (f32([1.0, 2.0, 3.0, 4.0]), None):
        if scores is None:
            rng = oracle.Rng(0xc0ffee)
            scores = oracle.bf16_array_to_f32(oracle.f32_array_to_bf16(rng.vec(256, -10.0, 10.0)))
        n = scores.size
        q = np.zeros(hd, np.float32)
        q[0] = 1.0
        k = np.zeros((n, hd), np.float32)
        k[:, 0] = scores
        v = np.zeros((n, hd), np.float32)
        v[np.arange(n), np.arange(n)] = 1.0
        kb, vb = oracle.f32_array_to_bf16(k.ravel()), oracle.f32_array_to_bf16(v.ravel())
        sc = np.zeros(n, np.float32)
        part = np.zeros(hd + 2, np.float32)
        ops.nng_op_attn_block(p(q), hd, p(kb), p(vb), hd, n, hd, 1, 1.0, p(sc), p(part))
        out = np.zeros(hd, np.float32)
        ops.nng_op_attn_finish(p(out), hd, p(part), hd, 1)
        e = np.exp(scores.astype(np.float64) - scores.max())
        want = e / e.sum()
        got = out[:n].astype(np.float64)
        assert np.all(got >= 0.0)
        assert abs(got.sum() - 1.0) < 1e-5
        if n == 4:
            assert np.all(close(out[:4], want, 1e-6))
        else:
            assert np.all(np.abs(got - want) <= 2e-6 * want + 1e-12), np.max(np.abs(got - want) / want)
        assert np.all(out[n:] == 0.0)


def test_merge_expf_restatement_is_glibc_expf(ops):
    # attn_merge scales the block partials by std::exp of a float (scalar.rs:
    # 521-537, the platform's expf). The device step restates glibc's expf
    # (glibc_expf in gemma3_gpu.hip); every one of the 2^32 float inputs
    # gives the same bits as the harness's own std::exp.
    from concurrent.futures import ThreadPoolExecutor
    L = ops
    L.nng_op_libm_expf.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
    L.nngd_expf_batch.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
    chunk = 1 << 24

    def run(c):
        x = (np.arange(chunk, dtype=np.uint64) + c * chunk).astype(np.uint32).view(np.float32)
        a = np.empty_like(x)
        b = np.empty_like(x)
        L.nng_op_libm_expf(x.ctypes.data, a.ctypes.data, chunk)
        L.nngd_expf_batch(x.ctypes.data, b.ctypes.data, chunk)
        same = (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))
        return int(chunk - np.count_nonzero(same))

    with ThreadPoolExecutor(8) as pool:
        bad = sum(pool.map(run, range((1 << 32) // chunk)))
    assert bad == 0


# ---- embedding rows (kernels/tests.rs:992-1032) ------------------------------------------------

def embed(ops, wtype, table, n_vocab, n_embd, tok, scale):
    ops.nng_op_embed_row.argtypes = [C.c_int, C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_float, C.c_void_p]
    ops.nng_op_embed_row.restype = None
    y = np.zeros(n_embd, np.float32)
    ops.nng_op_embed_row(wtype, p(table), n_vocab, n_embd, tok, scale, p(y))
    return y


def test_embed_rows_match_dequantized_tables(ops, oracle):
    # The scaled dequantized row, within quantization error of the source.
    rng = oracle.Rng(0xE3B0)
    rng.vec(17 * 5, -2.0, 2.0)  # the reference's BF16 case draws first (no BF16 tables here)
    n_embd, n_vocab, tok, scale = 64, 7, 5, 0.75
    src = rng.vec(n_vocab * n_embd, -2.0, 2.0)
    row = tok * n_embd
    qs, sc = oracle.quantize_q8_0(src)
    y = embed(ops, 1, oracle.pack_q8(qs, sc), n_vocab, n_embd, tok, scale)
    want = np.array([float(np.float32(qs[row + i]) * np.float32(oracle.bf16_to_f32(int(sc[(row + i) // 32])))
                           * np.float32(scale)) for i in range(n_embd)])
    assert close(y, want, 1e-5).all()
    assert (np.abs(y - src[row:row + n_embd] * scale) <= 0.05).all()
    q4, s4, b4 = oracle.quantize_q4(src)
    y = embed(ops, 2, oracle.pack_q4(q4, s4, b4), n_vocab, n_embd, tok, scale)
    # q4_dequant (kernels/tests.rs:387-397): sc * q + bi per element.
    want = np.zeros(n_embd, np.float32)
    for b in range(n_embd // 32):
        s_ = np.float32(oracle.bf16_to_f32(int(s4[row // 32 + b])))
        b_ = np.float32(oracle.bf16_to_f32(int(b4[row // 32 + b])))
        for k in range(16):
            byte = int(q4[row // 2 + 16 * b + k])
            want[32 * b + k] = s_ * np.float32(byte & 15) + b_
            want[32 * b + k + 16] = s_ * np.float32(byte >> 4) + b_
    assert close(y, want * np.float32(scale), 1e-5).all()
    assert (np.abs(y - src[row:row + n_embd] * scale) <= 0.2).all()


def test_embed_row_q4_nibble_order(ops):
    # Known answers: byte k of a block holds element k in its low nibble and
    # element k + 16 in its high one (kernels/mod.rs:948-951); scale 1 and
    # bias 0 make every output the nibble itself, times the row scale.
    n_vocab, n_embd = 2, 64
    q = np.zeros(n_vocab * n_embd // 2, np.uint8)
    for t in range(n_vocab):
        for b in range(2):
            for k in range(16):
                q[t * 32 + 16 * b + k] = ((k + b + t) & 15) | (((15 - k) & 15) << 4)
    one = 0x3F80
    table = np.concatenate([q, np.full(n_vocab * 2, one, np.uint16).view(np.uint8),
                            np.zeros(n_vocab * 2, np.uint16).view(np.uint8)])
    for t in range(n_vocab):
        y = embed(ops, 2, table, n_vocab, n_embd, t, 2.0)
        for b in range(2):
            for k in range(16):
                assert y[32 * b + k] == 2.0 * ((k + b + t) & 15)
                assert y[32 * b + k + 16] == 2.0 * (15 - k)
