"""Pins the CPU oracle (oracle/oracle.cpp, oracle/avx2.cpp) before it is trusted.

Each check comes from the reference's own tests or from what the mathematics
fixes, chosen so a plausible restatement mistake fails one of them:
  * known answers from crates/nncpu/src/kernels/tests.rs, runtime.rs and
    model/tests.rs;
  * f64 brute force with the reference's tolerance;
  * exactness of the weight products (closed form);
  * batch == single and thread-count invariance, bit for bit;
  * the scalar restatement == the AVX2-intrinsics restatement, bit for bit
    (two independent writings of the same reduction trees);
  * known answers of the row kernels, the Q4 bias dot and block_sums whose
    inputs tell the candidate reduction orders apart, derived by exact
    rational arithmetic rounded per operation (tests/row_kats.py,
    tests/f32_exact.py);
  * the committed golden vectors (tests/golden/).
"""
import json
import os

import numpy as np
import pytest

from conftest import bits, close
from f32_exact import Lcg, bf16_value, block_sums_ref, dot_bf16_ref, f32_bits, row_candidates, row_ref
from row_kats import (DOT_KATS, Q4_BIAS_DISCRIMINATED, Q4_KATS, Q8_KATS, dot_candidates, dot_inputs,
                      q4_candidates, q4_inputs, q4_ref, q4_split, q8_inputs, q8_split)

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def f32_from_bits(u):
    return float(np.array([u], np.uint32).view(np.float32)[0])


# ---- runtime.rs:225-241 ---------------------------------------------------------

def test_bf16_round_trip_and_rne(oracle):
    for f in [0.0, 1.0, -2.5, 3.140625, 2.0 ** -100, -(2.0 ** 100)]:
        assert oracle.bf16_to_f32(oracle.f32_to_bf16(f)) == np.float32(f)
    assert oracle.f32_to_bf16(f32_from_bits(0x3F808000)) == 0x3F80
    assert oracle.f32_to_bf16(f32_from_bits(0x3F818000)) == 0x3F82


# ---- kernels/tests.rs:531-553 ---------------------------------------------------

def test_rint_rounds_half_to_even(oracle):
    for v in [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5, 0.49999997, 3.7, -3.7, 1e9, -1e9,
              4_194_304.5, 8e6 + 0.5]:
        v32 = np.float32(v)
        assert oracle.rint(float(v32)) == int(np.rint(v32)), v
    assert oracle.rint(float("nan")) == 0
    assert oracle.rint(3e10) == 2**31 - 1 and oracle.rint(-3e10) == -(2**31)


# ---- kernels/tests.rs:502-529 ---------------------------------------------------

def test_q8_0_quantize_roundtrip(oracle):
    rng = oracle.Rng(0xC0FFEE)
    w = rng.vec(3 * 64, -2.5, 2.5)
    wb = oracle.bf16_array_to_f32(np.array([oracle.f32_to_bf16(float(v)) for v in w], np.uint16))
    qs, sc = oracle.quantize_q8_0(wb)
    s = oracle.bf16_array_to_f32(sc).repeat(32)
    assert np.all(np.abs(s * qs.astype(np.float32) - wb) <= s + 1e-6)
    assert qs.min() >= -127 and qs.max() <= 127
    src = np.zeros(32, np.float32)
    src[5], src[9] = -3.0, 1.5
    q, s1 = oracle.quantize_q8_0(src)
    assert oracle.bf16_to_f32(int(s1[0])) == oracle.bf16_to_f32(oracle.f32_to_bf16(3.0 / 127.0))
    assert (q[5], q[0]) == (-127, 0)
    q, s1 = oracle.quantize_q8_0(np.zeros(32, np.float32))
    assert s1[0] == 0 and not q.any()


def test_scales_are_times_reciprocal(oracle):
    # quant.rs:49-53,86-88: amax * (1/127) and (hi - lo) * (1/15), not a
    # division. These inputs (found by scanning every f32 in [1, 2)) are
    # ones where the two round to different BF16 scales.
    def bf(v):
        return oracle.f32_to_bf16(float(v))

    amax = np.float32(f32_from_bits(0x3FFEFE01))
    prod, quot = amax * np.float32(1.0 / 127.0), amax / np.float32(127.0)
    assert bf(prod) != bf(quot)
    src = np.zeros(32, np.float32)
    src[3] = amax
    assert oracle.quantize_q8_0(src)[1][0] == bf(prod)
    span = np.float32(f32_from_bits(0x3F895800))
    prod, quot = span * np.float32(1.0 / 15.0), span / np.float32(15.0)
    assert bf(prod) != bf(quot)
    src = np.zeros(32, np.float32)
    src[7] = span
    assert oracle.quantize_q4(src)[1][0] == bf(prod)


# ---- kernels/tests.rs:578-614 ---------------------------------------------------

def test_q4_quantize_roundtrip(oracle):
    src = np.zeros(64, np.float32)
    for i in range(32):
        src[i] = -2.0 + (i % 16) * 0.25
        src[32 + i] = 4.0 + (i % 16) * 0.5
    qs, sc, bi = oracle.quantize_q4(src)
    for b, (s, bias) in enumerate([(0.25, -2.0), (0.5, 4.0)]):
        assert (oracle.bf16_to_f32(int(sc[b])), oracle.bf16_to_f32(int(bi[b]))) == (s, bias)
        for k in range(16):
            byte = int(qs[16 * b + k])
            assert s * (byte & 15) + bias == src[32 * b + k]
            assert s * (byte >> 4) + bias == src[32 * b + k + 16]
    rng = oracle.Rng(0x4B15)
    src = rng.vec(32, -3.0, 7.0)
    qs, sc, bi = oracle.quantize_q4(src)
    s, bias = oracle.bf16_to_f32(int(sc[0])), oracle.bf16_to_f32(int(bi[0]))
    tol = 0.5 * s + (15.0 * s + abs(bias)) * 0.00391 + 1e-6
    for k in range(16):
        assert abs(s * (qs[k] & 15) + bias - src[k]) <= tol
        assert abs(s * (qs[k] >> 4) + bias - src[k + 16]) <= tol
    qs, sc, bi = oracle.quantize_q4(np.full(32, 3.5, np.float32))
    assert (oracle.bf16_to_f32(int(sc[0])), oracle.bf16_to_f32(int(bi[0]))) == (0.0, 3.5)
    assert not qs.any()


# ---- kernels/tests.rs:360-372 ---------------------------------------------------

def test_block_sums_match_reference(oracle):
    rng = oracle.Rng(0xB10C)
    x = rng.vec(128, -4.0, 4.0)
    out = oracle.block_sums(x)
    want = x.astype(np.float64).reshape(4, 32).sum(1)
    assert close(out, want, 1e-5).all()


def test_block_sums_order(oracle):
    # Values whose f32 sum depends on the order: the tree is
    # hsum8(((c[l]+c[8+l])+c[16+l])+c[24+l]); a sequential sum gives 0 here.
    c = np.zeros(32, np.float32)
    c[0], c[8], c[1] = 2.0 ** 24, 1.0, 1.0
    out = oracle.block_sums(c)[0]
    # lane 0: (2^24 + 1) -> 2^24; lane 1: 1; hsum8: (v0+v4)+(v1+v5) = 2^24 + 1 -> 2^24 (tie to even)
    assert out == np.float32(2.0 ** 24)
    c[:] = 0
    c[0], c[1], c[4] = 2.0 ** 24, 1.0, 1.0
    # (v0+v4) = 2^24+1 -> 2^24 (tie, even); (v1+v5) = 1 -> total 2^24+1 -> 2^24
    assert oracle.block_sums(c)[0] == np.float32(2.0 ** 24)
    c[:] = 0
    c[1], c[5], c[0] = 1.0, 1.0, 2.0 ** 24
    # (v1+v5) = 2 first, then 2^24 + 2 is exact.
    assert oracle.block_sums(c)[0] == np.float32(2.0 ** 24 + 2)


# ---- gemv against f64 brute force (kernels/tests.rs:555-576, 616-639) ------------

Q8_SHAPES = [(1, 32), (8, 64), (64, 128), (256, 256), (512, 512), (2048, 2048)]
Q4_SHAPES = [(1, 32), (8, 64), (64, 128), (256, 256), (512, 512), (1024, 2048), (300, 640)]


@pytest.mark.parametrize("dtype,shapes,seed", [(1, Q8_SHAPES, 0xC8E2), (2, Q4_SHAPES, 0x40E5)])
def test_gemv_matches_f64(oracle, dtype, shapes, seed):
    rng = oracle.Rng(seed)
    for rows, cols in shapes:
        w = rng.vec(rows * cols, -1.0, 1.0).reshape(rows, cols)
        if dtype == 1:
            w = oracle.bf16_array_to_f32(np.array([oracle.f32_to_bf16(float(v)) for v in w.ravel()], np.uint16)
                                         ).reshape(rows, cols) if rows * cols <= 4096 else w
        m = oracle.QMatrix.from_f32(dtype, w)
        x = rng.vec(cols, -1.0, 1.0)
        want = m.dequant().astype(np.float64) @ x.astype(np.float64)
        for backend in ("scalar", "avx2"):
            y = oracle.gemv_batch(m, x, backend=backend)
            assert close(y, want, 1e-3).all(), (rows, cols, backend)


def test_weight_products_are_exact(oracle):
    # f32(q) * bf16(scale) is exact for every Q8 quant and Q4 nibble, so
    # dequantizing in f64 and rounding never differs from the f32 product.
    rng = oracle.Rng(7)
    sc = np.array([oracle.f32_to_bf16(float(v)) for v in rng.vec(2000, 1e-6, 10.0)], np.uint16)
    s = oracle.bf16_array_to_f32(sc).astype(np.float64)
    q = np.arange(-127, 128, dtype=np.float64)
    exact = np.outer(s, q)
    assert np.array_equal(exact.astype(np.float32).astype(np.float64), exact)


# ---- invariants (kernels/tests.rs:641-741) ----------------------------------------

def test_gemv_batch_matches_rows(oracle):
    rng = oracle.Rng(0xBA7C)
    for n_batch in (2, 3, 4, 7):
        for rows, cols in [(64, 256), (512, 2048), (68, 96), (6, 64)]:
            w = rng.vec(rows * cols, -1.0, 1.0).reshape(rows, cols)
            xs, ys = cols + 32, rows + 3
            x = rng.vec(n_batch * xs, -1.0, 1.0)
            for dtype in (1, 2):
                m = oracle.QMatrix.from_f32(dtype, w)
                for backend in ("scalar", "avx2"):
                    yb = oracle.gemv_batch(m, x, n_batch, xs, ys, backend=backend)
                    for t in range(n_batch):
                        y1 = oracle.gemv_batch(m, x[t * xs:t * xs + cols], backend=backend)
                        assert np.array_equal(bits(y1), bits(yb[t * ys:t * ys + rows])), (n_batch, rows, cols)


def test_scalar_equals_avx2_bits(oracle):
    if not oracle.avx_available():
        pytest.skip("no AVX2+FMA on this host")
    rng = oracle.Rng(0x5CA1)
    for rows, cols in [(300, 640), (64, 1152), (17, 6912), (5, 96)]:
        w = rng.normals(rows * cols, 0.02).reshape(rows, cols)
        x = rng.normals(3 * cols, 1.0)
        for dtype in (1, 2):
            m = oracle.QMatrix.from_f32(dtype, w)
            for n in (1, 3):
                a = oracle.gemv_batch(m, x, n, cols, rows, backend="scalar")
                b = oracle.gemv_batch(m, x, n, cols, rows, backend="avx2")
                assert np.array_equal(bits(a), bits(b)), (rows, cols, dtype, n)


def test_results_do_not_depend_on_thread_count(oracle):
    rng = oracle.Rng(0x7417)
    rows, cols, n_batch = 1024, 512, 5
    w = rng.vec(rows * cols, -1.0, 1.0).reshape(rows, cols)
    x = rng.vec(n_batch * cols, -1.0, 1.0)
    old = oracle.avx_threads()
    try:
        outs = {}
        for nt in (1, 2, 3, 7, 16):
            oracle.avx_set_threads(nt)
            outs[nt] = [bits(oracle.gemv_batch(oracle.QMatrix.from_f32(d, w), x, n, cols, rows, backend="avx2"))
                        for d in (1, 2) for n in (1, n_batch)]
        for nt in (2, 3, 7, 16):
            for a, b in zip(outs[1], outs[nt]):
                assert np.array_equal(a, b), nt
    finally:
        oracle.avx_set_threads(old)


# ---- model/tests.rs:404-423: a wide Q4 with an exact answer -----------------------

def test_wide_q4_exact(oracle):
    cols, rows = 32 * 1025, 2
    n = cols * rows
    qs = np.full(n // 2, 0x11, np.uint8)
    sc = np.full(n // 32, 0x3F80, np.uint16)
    bi = np.full(n // 32, 0x3F00, np.uint16)
    m = oracle.QMatrix(2, rows, cols, (qs, sc, bi))
    y = oracle.gemv_batch(m, np.ones(cols, np.float32))
    assert np.array_equal(y, np.full(2, 1.5 * cols, np.float32))


# ---- argmax (model/forward.rs:1003-1011) ------------------------------------------

def test_argmax_ties_and_nan(oracle):
    v = np.array([1.0, 3.0, 2.0, 3.0], np.float32)
    assert oracle.argmax(v) == 1
    v = np.array([np.nan, 5.0, 1.0], np.float32)
    assert oracle.argmax(v) == 0
    v = np.array([1.0, np.nan, 5.0, 5.0], np.float32)
    assert oracle.argmax(v) == 2
    v = np.array([-0.0, 0.0], np.float32)
    assert oracle.argmax(v) == 0


# ---- dot_bf16_f32 (scalar.rs:334-347) ----------------------------------------------

def test_dot_bf16_tail_is_unfused(oracle):
    # Known answers (tests/row_kats.py): the 8-lane fused body, hsum8, then
    # the tail s += a*b with the product rounded before the add. A fused
    # tail, the tail folded into the lanes, another hsum8 tree or one chain
    # each give other bits on these inputs, and the oracle gives these.
    for seed, n, want in DOT_KATS:
        a, b = dot_inputs(seed, n)
        bv = [bf16_value(h) for h in a]
        assert f32_bits(dot_bf16_ref(bv, b)) == want
        for name, v in dot_candidates(a, b).items():
            assert f32_bits(v) != want, (n, name)
        got = oracle.dot_bf16_f32(np.array(a, np.uint16), np.array(b, np.float32))
        assert f32_bits(got) == want, (n, hex(f32_bits(got)))
    # And within 1e-5 of the f64 dot on random data.
    rng = oracle.Rng(0xD07)
    for n in (1, 7, 8, 9, 36, 37, 1025):
        a = np.array([oracle.f32_to_bf16(float(v)) for v in rng.vec(n, -1, 1)], np.uint16)
        b = rng.vec(n, -1, 1)
        want = (oracle.bf16_array_to_f32(a).astype(np.float64) * b).sum()
        assert abs(oracle.dot_bf16_f32(a, b) - want) <= 1e-5 * max(1.0, abs(want))


# ---- q8_row / q4_row reduction order (scalar.rs:108-117, 626-742) -------------------

def test_q8_row_known_answers(oracle):
    # 32 fused chains (element e of every block into accumulator e // 8, lane
    # e % 8), blocks in order, add8(add8(a0, a1), add8(a2, a3)), hsum8. The
    # inputs make every other order give other bits; scalar and AVX2
    # restatements, one row and a batch of three (q8_row3) give these.
    for seed, nb, want in Q8_KATS:
        q, s, x, w = q8_inputs(seed, nb)
        assert f32_bits(row_ref(w, x, nb)) == want
        for name, v in row_candidates(w, x, nb).items():
            assert f32_bits(v) != want, (nb, name)
        m = oracle.QMatrix(1, 1, 32 * nb, q8_split(q, s))
        xv = np.array(x, np.float32)
        for backend in ("scalar", "avx2"):
            assert f32_bits(oracle.gemv_batch(m, xv, backend=backend)[0]) == want, backend
            y3 = oracle.gemv_batch(m, np.tile(xv, 3), 3, backend=backend)
            assert all(f32_bits(v) == want for v in y3), backend


def test_q4_row_known_answers(oracle):
    # As q8_row with byte i of a block giving element i (low nibble) and
    # i + 16 (high), plus the bias term dot_bf16_f32(biases, block_sums(x))
    # added once; ggml's interleaved nibbles and each wrong bias-dot form give
    # other bits.
    for seed, nb, want in Q4_KATS:
        qb, s, bi, x = q4_inputs(seed, nb)
        assert f32_bits(q4_ref(qb, s, bi, x, nb)) == want
        for name, v in q4_candidates(qb, s, bi, x, nb).items():
            if name.startswith("bias_") and nb not in Q4_BIAS_DISCRIMINATED:
                continue
            assert f32_bits(v) != want, (nb, name)
        m = oracle.QMatrix(2, 1, 32 * nb, q4_split(qb, s, bi))
        xv = np.array(x, np.float32)
        for backend in ("scalar", "avx2"):
            assert f32_bits(oracle.gemv_batch(m, xv, backend=backend)[0]) == want, backend
            y3 = oracle.gemv_batch(m, np.tile(xv, 3), 3, backend=backend)
            assert all(f32_bits(v) == want for v in y3), backend


def test_block_sums_known_answer(oracle):
    # block_sums' tree on full-mantissa inputs: oracle == exact-rounding restatement.
    g = Lcg(0xB5)
    x = [g.f32_wide(-10, 10) for _ in range(32 * 5)]
    want = [f32_bits(v) for v in block_sums_ref(x)]
    got = oracle.block_sums(np.array(x, np.float32))
    assert [f32_bits(float(v)) for v in got] == want


# ---- int8 path: exact block dots and the exact-sum reference -----------------------

@pytest.mark.parametrize("dtype", [1, 2])
def test_block_dots_brute_force(oracle, dtype):
    rng = oracle.Rng(0x1D07 + dtype)
    rows, cols = 24, 160
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    qx, sx = oracle.quantize_act(rng.normals(cols, 1.0))
    P = oracle.block_dots(m, qx)
    if dtype == 1:
        qw = m.parts[0].astype(np.int64).reshape(rows, cols // 32, 32)
    else:
        blk = m.parts[0].reshape(rows, cols // 32, 16).astype(np.int64)
        qw = np.concatenate([blk & 15, blk >> 4], axis=2)
    want = (qw * qx.astype(np.int64).reshape(1, cols // 32, 32)).sum(2)
    assert np.array_equal(P, want)


@pytest.mark.parametrize("dtype", [1, 2])
def test_i8_exact_sum_within_reference_error(oracle, dtype):
    # The exact-sum value vs the reference kernel fed the dequantized
    # activations: the north-star tolerances, 1e-3 relative L2, 1e-5 abs.
    rng = oracle.Rng(0xE8 + dtype)
    rows, cols = 256, 4096
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    qx, sx = oracle.quantize_act(rng.normals(cols, 1.0))
    exact = oracle.gemv_i8_exact(m, qx, sx)
    ref = oracle.gemv_batch(m, oracle.dequant_act(qx, sx))
    f64 = m.dequant().astype(np.float64) @ oracle.dequant_act(qx, sx).astype(np.float64)
    assert np.abs(exact - f64).max() <= np.spacing(np.abs(f64).astype(np.float32)).max()
    assert np.abs(exact - ref).max() <= 1e-5
    assert np.linalg.norm(exact - ref) <= 1e-3 * np.linalg.norm(ref)


# ---- golden vectors -----------------------------------------------------------------

def _golden_cases():
    path = os.path.join(GOLDEN, "manifest.json")
    if not os.path.exists(path):
        return []
    return json.load(open(path))["cases"]


@pytest.mark.parametrize("case", _golden_cases(), ids=lambda c: c["name"])
def test_oracle_matches_golden(oracle, case):
    from golden_io import load_case
    m, x, y, extra = load_case(oracle, case)
    if case["kind"] == "gemv_f32":
        got = oracle.gemv_batch(m, x, case["n_tok"], case["x_stride"], case["y_stride"])
        assert np.array_equal(bits(got), bits(y))
    elif case["kind"] == "gemv_i8":
        qx, sx = oracle.quantize_act(x)
        assert np.array_equal(qx, extra["qx"]) and np.array_equal(sx, extra["sx"])
        assert np.array_equal(bits(oracle.gemv_i8_exact(m, qx, sx)), bits(y))
        assert np.array_equal(oracle.block_dots(m, qx), extra["P"])


# ---- BF16 weights (kernels/tests.rs:433-498; kernels/mod.rs:337-406) ---------------

BF16_SHAPES = [(1, 8), (7, 5), (16, 1536), (1536, 1536), (2048, 1536), (6144, 1536), (6, 64), (5, 24), (260, 512)]


def bf16s(oracle, rng, n, lo, hi):
    """kernels/tests.rs:47-49: f32_to_bf16 of each uniform draw."""
    return oracle.f32_array_to_bf16(rng.vec(n, lo, hi))


def test_bf16_encoder_matches_scalar(oracle):
    rng = oracle.Rng(0xBF16)
    v = np.concatenate([rng.vec(4096, -1e4, 1e4),
                        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -3.4e38], np.float32),
                        np.array([0x3F808000, 0x3F818000, 0x7F7FFFFF], np.uint32).view(np.float32)])
    want = np.array([oracle.f32_to_bf16(float(x)) for x in v], np.uint16)
    assert np.array_equal(oracle.f32_array_to_bf16(v), want)


def test_bf16_gemv_matches_f64(oracle):
    # kernels/tests.rs:433-459: U(-1,1) BF16 weights and x, f64 reference, 1e-3;
    # the shapes take every path (f64 fallback, 4-row, 1-row with and without
    # cols % 32).
    rng = oracle.Rng(0xB16E)
    for rows, cols in BF16_SHAPES:
        w = bf16s(oracle, rng, rows * cols, -1.0, 1.0)
        x = rng.vec(cols, -1.0, 1.0)
        want = oracle.bf16_array_to_f32(w).astype(np.float64).reshape(rows, cols) @ x.astype(np.float64)
        y = oracle.gemv_bf16(w, x, rows, cols)
        assert close(y, want, 1e-3).all(), (rows, cols)


# One product per step (x = 1, exact BF16 weights), chosen so the candidate
# reduction orders give different f32 sums: the 4-row kernel's hadd tree
# ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)) (scalar.rs:555-571), the 1-row kernel's
# hsum8 ((v0+v4)+(v1+v5))+((v2+v6)+(v3+v7)) (scalar.rs:108-117, 573-591), and
# with 32 columns the 4-row kernel's sequential chains (a_l over elements l,
# 8+l, 16+l, 24+l) against the 1-row kernel's add8 of four accumulators.
TREE8 = [0.00164794921875, -0.15625, -8704.0, -1.1953125, -0.83984375, 0.09375, -0.0015106201171875,
         -0.002838134765625]
TREE8_QUAD, TREE8_HSUM8 = -8706.099609375, -8706.1005859375
TREE32 = [-0.00579833984375, 0.0869140625, -1.9453125, 2.75, -0.00183868408203125, 5824.0, 1.375,
          -0.021240234375, -0.0166015625, 163.0, 1.2265625, 0.06640625, -1.5390625, -0.0225830078125,
          0.00799560546875, 0.14453125, 15744.0, -0.004425048828125, -11.0, 8000.0, -2.234375, -0.3515625,
          14.4375, 0.015869140625, -68.5, 0.00188446044921875, 13.5, -0.0024566650390625, -0.00144195556640625,
          0.0390625, 242.0, 1.953125]
TREE32_QUAD, TREE32_ROW = 29922.95703125, 29922.958984375


def test_bf16_reduction_trees(oracle):
    for vals, quad, row in ((TREE8, TREE8_QUAD, TREE8_HSUM8), (TREE32, TREE32_QUAD, TREE32_ROW)):
        cols = len(vals)
        wrow = oracle.f32_array_to_bf16(np.array(vals, np.float32))
        assert np.array_equal(oracle.bf16_array_to_f32(wrow), np.array(vals, np.float32))  # exact BF16
        x = np.ones(cols, np.float32)
        y4 = oracle.gemv_bf16(np.tile(wrow, 4), x, 4, cols)   # rows % 4 == 0: the 4-row kernel
        y5 = oracle.gemv_bf16(np.tile(wrow, 5), x, 5, cols)   # else the 1-row kernel
        assert quad != row
        assert np.all(y4 == np.float32(quad)), (cols, y4)
        assert np.all(y5 == np.float32(row)), (cols, y5)


def test_bf16_f64_fallback(oracle):
    # cols % 8 != 0 (mod.rs:556-564): f64 products summed in order, one rounding.
    rng = oracle.Rng(0xF64)
    for rows, cols in ((3, 5), (8, 13), (4, 1001)):
        w = bf16s(oracle, rng, rows * cols, -1.0, 1.0)
        x = rng.vec(cols, -1.0, 1.0)
        wf = oracle.bf16_array_to_f32(w).astype(np.float64).reshape(rows, cols)
        want = np.empty(rows, np.float32)
        for r in range(rows):
            s = 0.0
            for k in range(cols):
                s += wf[r, k] * float(x[k])
            want[r] = np.float32(s)
        assert np.array_equal(bits(oracle.gemv_bf16(w, x, rows, cols)), bits(want))


def test_bf16_argmax(oracle):
    # kernels/tests.rs:461-498: against the gemv (first max), a tie to the
    # lower row, and all-NaN gives 0.
    rng = oracle.Rng(0xA12A)
    for rows, cols in [(4, 32), (16, 256), (2048, 256), (256, 1536), (7, 5), (6, 64)]:
        w = bf16s(oracle, rng, rows * cols, -1.0, 1.0)
        x = rng.vec(cols, -1.0, 1.0)
        y = oracle.gemv_bf16(w, x, rows, cols)
        assert oracle.gemv_bf16_argmax(w, x, rows, cols) == oracle.argmax(y), (rows, cols)
    rows, cols = 512, 256
    w = np.zeros(rows * cols, np.uint16)
    for r in (100, 300, 301):
        w[r * cols] = oracle.f32_to_bf16(1.0)
    x = np.zeros(cols, np.float32)
    x[0] = 2.0
    assert oracle.gemv_bf16_argmax(w, x, rows, cols) == 100
    x[0] = np.nan
    assert oracle.gemv_bf16_argmax(w, x, rows, cols) == 0
    # The 4-row kernel's running best starts from -inf with no row (scalar.rs:
    # 612-628): a NaN row 0 is passed over, where the first-max argmax of the
    # materialised logits (rows % 4 != 0) keeps row 0.
    cols = 8
    for rows, want in ((8, 5), (7, 0)):
        w = np.zeros(rows * cols, np.uint16)
        w[0] = 0x7FC0  # NaN weight: row 0 is NaN
        for r in range(1, rows):
            w[r * cols] = oracle.f32_to_bf16(float(r if r != 5 else 50))
        x = np.ones(cols, np.float32)
        assert oracle.gemv_bf16_argmax(w, x, rows, cols) == want, rows
    # -inf is never taken either: all rows -inf gives 0 as well.
    w = np.full(8 * 8, 0, np.uint16)
    w[::8] = 0xFF80  # -inf
    assert oracle.gemv_bf16_argmax(w, np.ones(8, np.float32), 8, 8) == 0


# ---- GGUF block decoding (kernels/quant.rs:97-291; kernels/tests.rs:745-950) -------

def fp32_to_fp16(f):
    """kernels/tests.rs:747-771: binary32 -> binary16, round to nearest even (normals only)."""
    b = int(np.array([f], np.float32).view(np.uint32)[0])
    s, e, m = (b >> 31) & 1, ((b >> 23) & 0xFF) - 127 + 15, b & 0x7FFFFF
    inf = (s << 15) | (0x1F << 10)
    if e >= 31:
        return inf
    if e <= 0:
        return s << 15
    rnd, sticky = (m >> 12) & 1, int(m & 0xFFF != 0)
    mh = (m >> 13) + (rnd & (sticky | ((m >> 13) & 1)))
    if mh & 0x400:
        mh, e = 0, e + 1
        if e >= 31:
            return inf
    return (s << 15) | (e << 10) | (mh & 0x3FF)


def le16(v):
    return [v & 0xFF, (v >> 8) & 0xFF]


def q4k_unit_block(qs):
    b = np.zeros(144, np.uint8)
    b[:2] = le16(fp32_to_fp16(1.0))
    b[4:8] = 1
    b[12:16] = 1
    b[16:] = qs
    return b


def test_dequantize_q8_0_kat(oracle):
    blocks = np.zeros(68, np.uint8)
    blocks[:2] = le16(fp32_to_fp16(0.25))
    blocks[34:36] = le16(fp32_to_fp16(-2.0))
    for k in range(32):
        blocks[2 + k] = np.uint8((k - 16) & 0xFF)
        blocks[36 + k] = np.uint8((127 - 4 * k) & 0xFF)
    ok, out = oracle.dequantize_to_f32(8, blocks, 64)
    assert ok
    for k in range(32):
        assert out[k] == 0.25 * (k - 16.0)
        assert out[32 + k] == -2.0 * (127 - 4 * k)


def test_dequantize_legacy_kat(oracle):
    d, m = 0.5, -1.25
    for ty, has_min, has_high in [(2, False, False), (3, True, False), (6, False, True), (7, True, True)]:
        q = [((j * 11 + 5) % 32) if has_high else ((j * 7 + 3) % 16) for j in range(32)]
        block = le16(fp32_to_fp16(d))
        if has_min:
            block += le16(fp32_to_fp16(m))
        if has_high:
            qh = 0
            for j in range(32):
                qh |= ((q[j] >> 4) & 1) << j
            block += [(qh >> (8 * i)) & 0xFF for i in range(4)]
        block += [(q[j] & 0x0F) | ((q[j + 16] & 0x0F) << 4) for j in range(16)]
        ok, out = oracle.dequantize_to_f32(ty, np.array(block, np.uint8), 32)
        assert ok
        centre = 0 if has_min else 16 if has_high else 8
        want = np.array([np.float32(q[j] - centre) * np.float32(d) + np.float32(m if has_min else 0.0)
                         for j in range(32)], np.float32)
        assert np.array_equal(out, want), ty


def test_dequantize_k_quants_kat(oracle):
    # Q4_K: low nibbles 1, high nibbles 2 -> each 64-run is 32 ones then 32 twos.
    ok, out = oracle.dequantize_to_f32(12, q4k_unit_block(np.full(128, 0x21, np.uint8)), 256)
    assert ok and all((run[:32] == 1).all() and (run[32:] == 2).all() for run in out.reshape(4, 64))
    # Q5_K: the same with qh all 0 / all 1.
    b = np.zeros(176, np.uint8)
    b[:2] = le16(fp32_to_fp16(1.0))
    b[4:8] = 1
    b[12:16] = 1
    b[48:] = 0x21
    for qh, lo, hi in [(0x00, 1.0, 2.0), (0xFF, 17.0, 18.0)]:
        b[16:48] = qh
        ok, out = oracle.dequantize_to_f32(13, b, 256)
        assert ok and all((run[:32] == lo).all() and (run[32:] == hi).all() for run in out.reshape(4, 64))
    # Subnormal fp16 super-scale (kernels/tests.rs:889-900): d = 2^-24.
    b = np.zeros(144, np.uint8)
    b[:2] = le16(1)
    b[4] = 1
    b[16:] = 0x11
    ok, out = oracle.dequantize_to_f32(12, b, 256)
    assert ok and out[0] == np.float32(2.0 ** -24)
    # Q6_K: d = 1, scales 1, ql = 0x10, qh = 0 -> -32 and -31.
    b = np.zeros(210, np.uint8)
    b[:128] = 0x10
    b[192:208] = 1
    b[208:] = le16(fp32_to_fp16(1.0))
    ok, out = oracle.dequantize_to_f32(14, b, 256)
    assert ok and all((h[:64] == -32).all() and (h[64:] == -31).all() for h in out.reshape(2, 128))


def test_dequantize_k_quant_bit_positions(oracle):
    # Where each high bit and each packed 6-bit scale / min lands (ggml's
    # layout as quant.rs:197-291 reads it), one bit or one field at a time.
    base = np.zeros(176, np.uint8)
    base[:2] = le16(fp32_to_fp16(1.0))
    base[4:8] = 1
    base[12:16] = 1
    for run in range(4):
        for half in range(2):
            for l in (0, 13, 31):
                b = base.copy()
                b[16 + l] = 1 << (2 * run + half)  # qh bit 2j (low nibbles) / 2j+1 (high) of byte l
                ok, out = oracle.dequantize_to_f32(13, b, 256)
                want = np.zeros(256, np.float32)
                want[64 * run + 32 * half + l] = 16.0
                assert ok and np.array_equal(out, want), (run, half, l)
    # Q4_K scales: sub-block j < 4 scale = byte 4+j & 63, min = byte 8+j & 63;
    # j >= 4 scale = (byte 12+j-4 & 15) | (byte 4+j-4 >> 6) << 4, min = (byte
    # 12+j-4 >> 4) | (byte 8+j-4 >> 6) << 4.
    b = np.zeros(144, np.uint8)
    b[:2] = le16(fp32_to_fp16(1.0))
    b[2:4] = le16(fp32_to_fp16(1.0))
    b[4:16] = [0x41, 0x82, 0xC3, 0x04, 0x45, 0x86, 0xC7, 0x08, 0x9A, 0xBC, 0xDE, 0xF1]
    b[16:] = 0x11  # q = 1 everywhere
    ok, out = oracle.dequantize_to_f32(12, b, 256)
    sc = b[4:16].astype(int)
    for j in range(8):
        if j < 4:
            d, m = sc[j] & 63, sc[j + 4] & 63
        else:
            d, m = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4), (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4)
        seg = out[32 * j:32 * (j + 1)]
        assert ok and (seg == np.float32(d) - np.float32(m)).all(), j
    # Q6_K: bit pairs of qh and the int8 scale per 16 values.
    for h in range(2):
        for l in (0, 17, 31):
            for pair in range(4):
                b = np.zeros(210, np.uint8)
                b[192:208] = [(i + 1) & 0xFF for i in range(16)]
                b[192 + 8 * h + 3] = 0xFE  # a negative scale (-2)
                b[208:] = le16(fp32_to_fp16(1.0))
                b[:128] = 0x00
                b[128 + 32 * h + l] = 1 << (2 * pair)  # value 16 in the 2 high bits of output pair
                ok, out = oracle.dequantize_to_f32(14, b, 256)
                is_ = l // 16 + 2 * pair
                s = np.float32(np.int8(b[192 + 8 * h + is_]))
                e = 128 * h + 32 * pair + l
                assert ok and out[e] == np.float32(1.0) * s * np.float32(16 - 32), (h, l, pair)


def test_dequantize_float_types_and_rejects(oracle):
    vals = np.array([1.5, -2.25, 0.0, 3e-3, -7.0], np.float32)
    ok, out = oracle.dequantize_to_f32(0, vals.view(np.uint8), 5)
    assert ok and np.array_equal(out, vals)
    f16 = np.array([fp32_to_fp16(float(v)) for v in vals], np.uint16)
    ok, out = oracle.dequantize_to_f32(1, f16.view(np.uint8), 5)
    assert ok and (np.abs(out - vals) <= np.abs(vals) * 1e-3).all()
    assert np.array_equal(out, f16.view(np.float16).astype(np.float32))  # IEEE half, exactly
    bf = oracle.f32_array_to_bf16(vals)
    ok, out = oracle.dequantize_to_f32(30, bf.view(np.uint8), 5)
    assert ok and np.array_equal(out, oracle.bf16_array_to_f32(bf))
    # Every half bit pattern, subnormals, infinities and NaN payloads included.
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ok, out = oracle.dequantize_to_f32(1, allh.view(np.uint8), 65536)
    want = allh.view(np.float16).astype(np.float32)
    fin = ~np.isnan(want)
    assert ok and np.array_equal(out[fin].view(np.uint32), want[fin].view(np.uint32))
    nan_bits = out[~fin].view(np.uint32)
    hb = allh[~fin].astype(np.uint32)
    assert np.array_equal(nan_bits, ((hb & 0x8000) << 16) | 0x7F800000 | ((hb & 0x3FF) << 13))
    # Unknown types, partial blocks and short input leave dst untouched.
    for ty, nbytes, n in [(9, 64, 32), (10, 128, 32), (8, 33, 32), (8, 68, 33)]:
        ok, out = oracle.dequantize_to_f32(ty, np.zeros(nbytes, np.uint8), n)
        assert not ok and (out == 9.0).all()
