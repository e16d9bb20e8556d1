"""Exact IEEE f32 arithmetic in Python (test helper), for deriving known
answers of nncpu's row kernels independently of the C oracle.

Every operation is computed exactly on Fractions and rounded once to the
nearest f32, ties to even (normal range only: the known-answer inputs stay
far from the subnormal and overflow ranges, which ``round32`` asserts).
``fma32`` is the fused multiply-add (one rounding), ``mul32``/``add32`` the
unfused steps. On top of these, the reduction orders of
crates/nncpu/src/kernels/scalar.rs (``hsum8`` :108-117, ``dot_bf16_f32``
:334-347, ``block_sums`` :355-359, ``q8_row`` / ``q4_row`` :626-674) and
plausible wrong alternatives to each, so a test can show that its inputs
tell them apart.
"""
from __future__ import annotations

import struct
from fractions import Fraction


def f32_bits(v: float) -> int:
    return struct.unpack("<I", struct.pack("<f", v))[0]


def from_bits(u: int) -> float:
    return struct.unpack("<f", struct.pack("<I", u & 0xFFFFFFFF))[0]


def bf16_value(h: int) -> float:
    """BF16 bits -> value (exact: the top half of an f32)."""
    return from_bits(h << 16)


def round32(v: Fraction) -> float:
    """The f32 nearest v, ties to even (normal range)."""
    if v == 0:
        return 0.0
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    # Normalise so 2^23 <= a / 2^(e-23) < 2^24.
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    assert -126 <= e <= 127, "outside the normal f32 range"
    q = a / Fraction(2) ** (e - 23)
    m = q.numerator // q.denominator
    r = q - m
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and m % 2 == 1):
        m += 1
    out = Fraction(m) * Fraction(2) ** (e - 23)
    f = float(out)  # exact: m has at most 24 bits
    assert f32_bits(f) is not None
    return sign * f


def F(v: float) -> Fraction:
    return Fraction(v)


def add32(a: float, b: float) -> float:
    return round32(F(a) + F(b))


def mul32(a: float, b: float) -> float:
    return round32(F(a) * F(b))


def fma32(a: float, b: float, c: float) -> float:
    return round32(F(a) * F(b) + F(c))


# ---- reduction trees ---------------------------------------------------------------

def hsum8(v):
    """scalar.rs:115-117: ((v0+v4)+(v1+v5))+((v2+v6)+(v3+v7))."""
    return add32(add32(add32(v[0], v[4]), add32(v[1], v[5])), add32(add32(v[2], v[6]), add32(v[3], v[7])))


def hsum8_pairwise(v):
    """A plausible wrong tree: ((v0+v1)+(v2+v3))+((v4+v5)+(v6+v7))."""
    return add32(add32(add32(v[0], v[1]), add32(v[2], v[3])), add32(add32(v[4], v[5]), add32(v[6], v[7])))


def hsum8_seq(v):
    s = v[0]
    for t in v[1:]:
        s = add32(s, t)
    return s


# ---- q8_row / q4_row: 32 chains over the blocks, then add8 and hsum8 ----------------

def row_chains(w, x, nb, fused=True, reverse=False, n_chains=32):
    """Chain c accumulates element c of every block (c = 8k + l: accumulator
    a_k, lane l), block 0 first; `w` holds the exact products q*s."""
    acc = [0.0] * n_chains
    order = range(nb - 1, -1, -1) if reverse else range(nb)
    for b in order:
        for e in range(32):
            c = e % n_chains
            wv, xv = w[32 * b + e], x[32 * b + e]
            acc[c] = fma32(wv, xv, acc[c]) if fused else add32(mul32(wv, xv), acc[c])
    return acc


def combine_ref(a):
    """add8(add8(a0, a1), add8(a2, a3)) then hsum8 (scalar.rs:648,673)."""
    v = [add32(add32(a[l], a[8 + l]), add32(a[16 + l], a[24 + l])) for l in range(8)]
    return hsum8(v)


def combine_seq(a):
    v = [add32(add32(add32(a[l], a[8 + l]), a[16 + l]), a[24 + l]) for l in range(8)]
    return hsum8(v)


def combine_cross(a):
    v = [add32(add32(a[l], a[16 + l]), add32(a[8 + l], a[24 + l])) for l in range(8)]
    return hsum8(v)


def combine_pairwise_hsum(a):
    v = [add32(add32(a[l], a[8 + l]), add32(a[16 + l], a[24 + l])) for l in range(8)]
    return hsum8_pairwise(v)


def row_ref(w, x, nb):
    return combine_ref(row_chains(w, x, nb))


def row_candidates(w, x, nb):
    """Wrong orders a restatement might take, by name."""
    out = {
        "unfused": combine_ref(row_chains(w, x, nb, fused=False)),
        "reversed_blocks": combine_ref(row_chains(w, x, nb, reverse=True)),
        "add8_sequential": combine_seq(row_chains(w, x, nb)),
        "add8_cross_pairs": combine_cross(row_chains(w, x, nb)),
        "hsum8_pairwise": combine_pairwise_hsum(row_chains(w, x, nb)),
        "eight_chains": hsum8(row_chains(w, x, nb, n_chains=8)),
    }
    s = 0.0
    for i in range(32 * nb):
        s = fma32(w[i], x[i], s)
    out["one_chain"] = s
    out["exact_rounded_once"] = round32(sum(F(w[i]) * F(x[i]) for i in range(32 * nb)))
    return out


# ---- dot_bf16_f32 (the Q4 bias term) and block_sums --------------------------------

def dot_bf16_ref(a, b):
    """scalar.rs:334-347: 8 lanes fused over the body, hsum8, then an
    unfused tail s += a*b."""
    n = len(a)
    body = n & ~7
    acc = [0.0] * 8
    for j in range(0, body, 8):
        for l in range(8):
            acc[l] = fma32(a[j + l], b[j + l], acc[l])
    s = hsum8(acc)
    for i in range(body, n):
        s = add32(s, mul32(a[i], b[i]))
    return s


def dot_bf16_candidates(a, b):
    n = len(a)
    body = n & ~7
    acc = [0.0] * 8
    for j in range(0, body, 8):
        for l in range(8):
            acc[l] = fma32(a[j + l], b[j + l], acc[l])
    out = {}
    s = hsum8(acc)
    for i in range(body, n):
        s = fma32(a[i], b[i], s)
    out["fused_tail"] = s
    t = list(acc)
    for i in range(body, n):  # the tail folded into the lanes before hsum8
        t[i - body] = fma32(a[i], b[i], t[i - body])
    out["tail_in_lanes"] = hsum8(t)
    s = hsum8_pairwise(acc)
    for i in range(body, n):
        s = add32(s, mul32(a[i], b[i]))
    out["hsum8_pairwise"] = s
    s = 0.0
    for i in range(n):
        s = fma32(a[i], b[i], s)
    out["one_chain"] = s
    return out


def block_sums_ref(x):
    """scalar.rs:355-359: hsum8 over l of ((c[l]+c[8+l])+c[16+l])+c[24+l]."""
    out = []
    for b in range(len(x) // 32):
        c = x[32 * b:32 * b + 32]
        out.append(hsum8([add32(add32(add32(c[l], c[8 + l]), c[16 + l]), c[24 + l]) for l in range(8)]))
    return out


# ---- deterministic inputs (no library RNG) ------------------------------------------

class Lcg:
    """64-bit LCG (Knuth's MMIX constants), top bits out: inputs that any
    Python reproduces."""

    def __init__(self, seed: int):
        self.s = seed & (2**64 - 1)

    def u32(self) -> int:
        self.s = (self.s * 6364136223846793005 + 1442695040888963407) & (2**64 - 1)
        return self.s >> 32

    def f32_wide(self, lo_exp: int, hi_exp: int) -> float:
        """A full-mantissa f32 with a random sign and exponent in [lo_exp, hi_exp]."""
        e = lo_exp + self.u32() % (hi_exp - lo_exp + 1)
        m = (1 << 23) | (self.u32() & ((1 << 23) - 1))
        v = float(Fraction(m) * Fraction(2) ** (e - 23))
        return -v if self.u32() & 1 else v

    def bf16_wide(self, lo_exp: int, hi_exp: int, positive: bool = False) -> int:
        e = lo_exp + self.u32() % (hi_exp - lo_exp + 1)
        h = ((e + 127) << 7) | (self.u32() & 0x7F)
        if not positive and self.u32() & 1:
            h |= 0x8000
        return h
