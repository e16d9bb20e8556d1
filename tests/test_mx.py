"""Pins of the oracle's MX int8 restatement (no GPU): the power-of-two block
exponent against a direct search, the quantizer against known answers and
its closed-form properties, the BF16 limb split, and the batched exact GEMM
against the independent C restatement (or_gemv_i8_exact). The MX path has no
counterpart in nncpu (which never quantizes activations), so these checks,
not the reference, fix its arithmetic.
"""
import numpy as np
import pytest

U32 = 2.0 ** -24


def f32(bits_):
    return np.array([bits_], np.uint32).view(np.float32)[0]


def search_exponent(amax):
    """The least E in [-126, 127] with 127 * 2^E >= amax, by trying each E
    (exact in f64: amax is an f32, 127 * 2^E has 7 significant bits)."""
    for e in range(-126, 128):
        if 127.0 * 2.0 ** e >= float(amax):
            return e
    return 127


def test_mx_exponent_matches_search(oracle):
    vals = [0.0, f32(1), f32(0x007FFFFF), f32(0x00800000), 1e-30, 1.0, 127.0, 127.5, 128.0, 254.0, 254.0001,
            f32(0x7F7FFFFF), 3e38]
    for e in range(-126, 128):
        for mant in (0x000000, 0x000001, 0x7E0000, 0x7E0001, 0x7FFFFF, 0x400000):
            vals.append(f32(((e + 127) << 23) | mant))
    rng = np.random.default_rng(5)
    vals += list(np.abs(rng.standard_normal(2000).astype(np.float32)) * np.float32(10.0) ** rng.integers(-30, 30, 2000))
    a = np.array(vals, np.float32)
    got = oracle.mx_exponent(a)
    want = np.array([search_exponent(v) for v in a])
    assert np.array_equal(got, want)


def test_mx_quantizer_known_answers(oracle):
    # amax 127: scale 1, integers kept; halves round to even.
    x = np.zeros(32, np.float32)
    x[0], x[1], x[2], x[3], x[4] = 127.0, -3.0, 2.5, 3.5, -0.5
    q, s = oracle.quantize_act_mx(x)
    assert s[0] == 0x3F80  # 1.0
    assert list(q[:5]) == [127, -3, 2, 4, 0]
    # amax 1: 2^-6 (127/64 >= 1 > 127/128), q = rint(64 x).
    x = np.zeros(32, np.float32)
    x[0], x[1] = 1.0, -0.25
    q, s = oracle.quantize_act_mx(x)
    assert oracle.bf16_to_f32(int(s[0])) == 2.0 ** -6 and q[0] == 64 and q[1] == -16
    # Mantissa boundary: 1.984375 = 127 * 2^-6 keeps 2^-6 (q = 127); one ulp more needs 2^-5.
    x[0] = f32(0x3FFE0000)
    q, s = oracle.quantize_act_mx(x)
    assert oracle.bf16_to_f32(int(s[0])) == 2.0 ** -6 and q[0] == 127
    x[0] = f32(0x3FFE0001)
    q, s = oracle.quantize_act_mx(x)
    assert oracle.bf16_to_f32(int(s[0])) == 2.0 ** -5 and q[0] == 64
    # Zero block: scale 0, q 0. NaN: skipped for the scale, q 0.
    q, s = oracle.quantize_act_mx(np.zeros(32, np.float32))
    assert s[0] == 0 and not q.any()
    x = np.full(32, 0.5, np.float32)
    x[7] = np.nan
    q, s = oracle.quantize_act_mx(x)
    assert oracle.bf16_to_f32(int(s[0])) == 2.0 ** -7 and q[7] == 0 and q[0] == 64


def test_mx_quantizer_properties(oracle):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(32 * 4000) * 10.0 ** rng.integers(-20, 20, 32 * 4000 // 32).repeat(32)).astype(np.float32)
    q, s = oracle.quantize_act_mx(x)
    sf = oracle.bf16_array_to_f32(s).astype(np.float64)
    xb = x.astype(np.float64).reshape(-1, 32)
    qb = q.astype(np.float64).reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    # the scale is a power of two, the least with 127 s >= amax
    m, _ = np.frexp(sf)
    assert np.all(m == 0.5)
    assert np.all(127 * sf >= amax) and np.all(127 * sf / 2 < amax)
    # q is x / s rounded to nearest: within half a step, |q| <= 127, and the
    # largest |q| of a block is at least 64 (nothing wasted on the scale)
    assert np.all(np.abs(xb - qb * sf[:, None]) <= sf[:, None] / 2)
    assert np.abs(qb).max() <= 127 and np.all(np.abs(qb).max(axis=1) >= 64)
    # q 2^E is a BF16 value (what the GEMM's MFMA operand holds)
    v = (qb * sf[:, None]).astype(np.float32)
    assert np.all((v.view(np.uint32) & 0xFFFF) == 0)


def test_mx_limbs_exact(oracle):
    rng = np.random.default_rng(3)
    qsum = rng.integers(-4064, 4065, 5000)
    e = rng.integers(-126, 100, 5000)
    X = np.ldexp(qsum.astype(np.float64), e).astype(np.float32)
    hi, lo = oracle.mx_limbs(X)
    h = oracle.bf16_array_to_f32(hi).astype(np.float64)
    lw = oracle.bf16_array_to_f32(lo).astype(np.float64)
    assert np.array_equal(h + lw, X.astype(np.float64))


@pytest.mark.parametrize("dtype", [1, 2])
@pytest.mark.parametrize("mx", [False, True])
def test_gemm_exact_matches_c_restatement(oracle, dtype, mx):
    rows, cols, n_tok = 37, 288, 5
    rng = oracle.Rng(0x9E11 + dtype + 2 * mx)
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    x = rng.normals(n_tok * cols, 1.0)
    quant = oracle.quantize_act_mx if mx else oracle.quantize_act
    qs, ss = zip(*[quant(x[t * cols:(t + 1) * cols]) for t in range(n_tok)])
    y, mag = oracle.gemm_exact(m, np.concatenate(qs), np.concatenate(ss), n_tok)
    for t in range(n_tok):
        c = oracle.gemv_i8_exact(m, qs[t], ss[t])
        assert np.all(np.abs(y[t].astype(np.float32) - c) <= np.spacing(np.abs(c))), t
    assert np.all(mag >= np.abs(y))


def test_gemm_bound_catches_planted_mistakes(oracle):
    # The GPU test's bound (64 u sum|terms| + 1 ulp for Q4) must reject the
    # plausible slips: a dropped bias term, one block's scale off by one BF16
    # step, a block dot taken against the neighbouring block's quants.
    rows, cols, n_tok = 64, 1152, 4
    rng = oracle.Rng(0x9E12)
    m = oracle.QMatrix.from_f32(2, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    x = rng.normals(n_tok * cols, 1.0)
    qs, ss = zip(*[oracle.quantize_act_mx(x[t * cols:(t + 1) * cols]) for t in range(n_tok)])
    q, s = np.concatenate(qs), np.concatenate(ss)
    y, mag = oracle.gemm_exact(m, q, s, n_tok)
    bound = 64 * U32 * mag + np.spacing(np.abs(y).astype(np.float32))

    def caught(y2):
        return np.any(np.abs(y2 - y) > bound)

    nb = cols // 32
    no_bias = oracle.QMatrix(2, rows, cols, (m.parts[0], m.parts[1], np.zeros_like(m.parts[2])))
    assert caught(oracle.gemm_exact(no_bias, q, s, n_tok)[0])
    sc = m.parts[1].copy()
    sc[5] += 1
    assert caught(oracle.gemm_exact(oracle.QMatrix(2, rows, cols, (m.parts[0], sc, m.parts[2])), q, s, n_tok)[0])
    qsh = q.reshape(n_tok, nb, 32).copy()
    qsh[:, 3] = qsh[:, 4]
    assert caught(oracle.gemm_exact(m, qsh.reshape(-1), s, n_tok)[0])
