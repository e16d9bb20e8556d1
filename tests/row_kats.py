"""Known answers for nncpu's row kernels that tell the reduction orders apart
(test data and its generator; used by test_oracle.py on the CPU and by
test_gemv_gpu.py on the device).

Each case is one weight row and one x, generated from a seed by ``Lcg`` (no
library RNG): full-mantissa x over a wide exponent range, so that every
candidate order a restatement might take (unfused FMAs, blocks in reverse,
another add8 pairing, another hsum8 tree, 8 chains instead of 32, one
chain, the exact sum rounded once; for Q4 also ggml's interleaved nibbles and
each wrong form of the bias dot) gives an f32 result different from nncpu's
order. The expected bits were derived with ``f32_exact`` (exact rational
arithmetic rounded per operation as crates/nncpu/src/kernels/scalar.rs
:108-117, :334-359, :626-742 specify), and the seeds were searched so that
every candidate differs; the tests re-derive both facts.
"""
from __future__ import annotations

import numpy as np

from f32_exact import (Lcg, add32, bf16_value, block_sums_ref, dot_bf16_candidates, dot_bf16_ref, row_candidates,
                       row_ref)

# (seed, blocks per row, expected f32 bits of the row's output)
Q8_KATS = [(46, 3, 0x4AA65699), (5, 67, 0xCAE91E78)]
# Q4: the 11-block case tells every candidate apart, the bias-dot forms
# included; the 67-block case (a row long enough for the streamed long-row
# kernels) every candidate but the bias-dot forms, which the 11-block case
# and DOT_KATS pin.
Q4_KATS = [(372, 11, 0x461B5250), (14, 67, 0xC9D74A74)]
Q4_BIAS_DISCRIMINATED = {11}
# dot_bf16_f32 alone: (seed, length, expected bits); 11 = one 8-lane body
# and a 3-value tail, 36 = four bodies and a tail of 4.
DOT_KATS = [(29, 11, 0x3F15102A), (30, 36, 0xC206A5D4)]


def q8_inputs(seed: int, nb: int):
    """(quants int8[32 nb], BF16 scale bits[nb], x f32[32 nb], exact products q*s)."""
    g = Lcg(seed)
    q = [int(g.u32() % 255) - 127 for _ in range(32 * nb)]
    s = [g.bf16_wide(-8, 4, positive=True) for _ in range(nb)]
    x = [g.f32_wide(-10, 10) for _ in range(32 * nb)]
    w = [float(q[i]) * bf16_value(s[i // 32]) for i in range(32 * nb)]
    return q, s, x, w


def q4_inputs(seed: int, nb: int):
    """(quant bytes[16 nb], BF16 scale bits[nb], BF16 bias bits[nb], x f32[32 nb])."""
    g = Lcg(seed)
    qb = [int(g.u32() & 0xFF) for _ in range(16 * nb)]
    s = [g.bf16_wide(-8, 4, positive=True) for _ in range(nb)]
    bi = [g.bf16_wide(-8, 4) for _ in range(nb)]
    x = [g.f32_wide(-10, 10) for _ in range(32 * nb)]
    return qb, s, bi, x


def q4_products(qb, s, nb, interleaved=False):
    """The exact products nibble * scale in element order: byte i of a block
    holds element i (low nibble) and i + 16 (high) (runtime.rs:58-62);
    ``interleaved`` is ggml's order (elements 2i, 2i + 1), a wrong candidate."""
    w = []
    for b in range(nb):
        sc = bf16_value(s[b])
        blk = qb[16 * b:16 * b + 16]
        if interleaved:
            el = [v for i in range(16) for v in (blk[i] & 15, blk[i] >> 4)]
        else:
            el = [blk[i] & 15 for i in range(16)] + [blk[i] >> 4 for i in range(16)]
        w += [float(e) * sc for e in el]
    return w


def q4_ref(qb, s, bi, x, nb):
    """q4_row plus dot_bf16_f32(biases, block_sums(x)), one f32 add (scalar.rs:706-742)."""
    y = row_ref(q4_products(qb, s, nb), x, nb)
    return add32(y, dot_bf16_ref([bf16_value(h) for h in bi], block_sums_ref(x)))


def q4_candidates(qb, s, bi, x, nb):
    w = q4_products(qb, s, nb)
    xs = block_sums_ref(x)
    bv = [bf16_value(h) for h in bi]
    bias = dot_bf16_ref(bv, xs)
    out = {k: add32(v, bias) for k, v in row_candidates(w, x, nb).items()}
    out["nibbles_interleaved"] = add32(row_ref(q4_products(qb, s, nb, interleaved=True), x, nb), bias)
    y = row_ref(w, x, nb)
    for k, v in dot_bf16_candidates(bv, xs).items():
        out["bias_" + k] = add32(y, v)
    return out


def dot_inputs(seed: int, n: int):
    g = Lcg(seed)
    a = [g.bf16_wide(-6, 6) for _ in range(n)]
    b = [g.f32_wide(-6, 6) for _ in range(n)]
    return a, b


def q8_split(q, s):
    """One row in the Q8_0 split layout parts (runtime.rs:136-147)."""
    return np.array(q, np.int8), np.array(s, np.uint16)


def q4_split(qb, s, bi):
    return np.array(qb, np.uint8), np.array(s, np.uint16), np.array(bi, np.uint16)


def dot_candidates(a, b):
    return dot_bf16_candidates([bf16_value(h) for h in a], b)
