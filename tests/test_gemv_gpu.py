"""Parity of the HIP path with the oracle, through the C-ABI (needs an MI355X).

f32 path: bit-exact against the oracle (nncpu's kernels restated) on the
golden vectors, the reference's own test shapes and the BASELINE shapes.
int8 path: the device quantizer bit-exact against nncpu's Q8_0 encoder, the
int32 block dots bit-exact, and the outputs within the north-star tolerance
(1e-3 relative L2, 1e-5 absolute) of the reference kernel fed the
dequantized activations; also within one f32 ulp of the exact sum (up to 16
vectors) or within the f32 rounding bound of the MFMA GEMM's epilogue.
"""
import os
import sys

import numpy as np
import pytest

from conftest import bits, close
from golden_io import cases, load_case

pytestmark = pytest.mark.gpu

N = pytest.importorskip("nncpu_amd")


@pytest.fixture(scope="module", autouse=True)
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    N.init(0)


def upload(m):
    if m.dtype == 1:
        return N.Weight.q8_0(m.parts[0], m.parts[1], m.rows, m.cols)
    return N.Weight.q4(m.parts[0], m.parts[1], m.parts[2], m.rows, m.cols)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


# ---- f32 path: bit-exact ----------------------------------------------------------

def kat_weight(dtype, seed, nb, rows):
    """A matrix of `rows` copies of a known-answer row (tests/row_kats.py) and its x."""
    from row_kats import q4_inputs, q4_split, q8_inputs, q8_split
    if dtype == 1:
        q, s, x, _ = q8_inputs(seed, nb)
        qs, sc = q8_split(q, s)
        w = N.Weight.q8_0(np.tile(qs, rows), np.tile(sc, rows), rows, 32 * nb)
    else:
        qb, s, bi, x = q4_inputs(seed, nb)
        qs, sc, b = q4_split(qb, s, bi)
        w = N.Weight.q4(np.tile(qs, rows), np.tile(sc, rows), np.tile(b, rows), rows, 32 * nb)
    return w, np.array(x, np.float32)


def kat_cases():
    from row_kats import Q4_KATS, Q8_KATS
    return [(1,) + k for k in Q8_KATS] + [(2,) + k for k in Q4_KATS]


@pytest.mark.parametrize("rows", [4, 2048, 16384, 32768])
@pytest.mark.parametrize("kat", kat_cases(), ids=lambda k: f"{'Q8' if k[0] == 1 else 'Q4'}_nb{k[2]}")
def test_f32_known_answers(kat, rows):
    # The hand-derived known answers whose inputs tell nncpu's reduction
    # order from every plausible other one: every kernel of the bit-exact
    # path (few rows, the streamed long-row kernels from 64 blocks, the
    # 8-lane tall kernel from 12288 rows with one or four rows per lane
    # group, 2-4 vectors) gives those bits.
    dtype, seed, nb, want = kat
    say("kat", dtype, seed, nb, rows)
    w, x = kat_weight(dtype, seed, nb, rows)
    y = N.model_gemv(w, x)
    assert np.all(bits(y) == want), (hex(int(bits(y)[0])), hex(want))
    y3 = np.zeros(3 * rows, np.float32)
    N.gemv_batch(w, np.tile(x, 3), 32 * nb, y3, rows, 3, N.ACT_F32)
    assert np.all(bits(y3) == want)
    w.free()


@pytest.mark.parametrize("case", [c for c in cases() if c["kind"] == "gemv_f32"], ids=lambda c: c["name"])
def test_f32_golden_bit_exact(oracle, case):
    say("case", case["name"])
    m, x, y, _ = load_case(oracle, case)
    w = upload(m)
    n, xs, ys = case["n_tok"], case["x_stride"], case["y_stride"]
    got = np.full_like(y, 7.0)  # stride gaps must stay untouched
    N.gemv_batch(w, x, xs, got, ys, n, N.ACT_F32)
    for t in range(n):
        assert np.array_equal(bits(got[t * ys:t * ys + m.rows]), bits(y[t * ys:t * ys + m.rows])), t
        gap = got[t * ys + m.rows:(t + 1) * ys] if t + 1 < n else []
        assert np.all(np.asarray(gap) == 7.0)


@pytest.mark.parametrize("dtype", [1, 2])
def test_f32_reference_shapes(oracle, dtype):
    # kernels/tests.rs:555-576 and 616-639: U(-1,1) weights and x, against f64
    # brute force at 1e-3, and bit-exact against the oracle.
    rng = oracle.Rng(0xC8E2 if dtype == 1 else 0x40E5)
    shapes = [(1, 32), (8, 64), (64, 128), (256, 256), (512, 512), (2048, 2048)] if dtype == 1 else \
        [(1, 32), (8, 64), (64, 128), (256, 256), (512, 512), (1024, 2048), (300, 640)]
    for rows, cols in shapes:
        say("shape", dtype, rows, cols)
        m = oracle.QMatrix.from_f32(dtype, rng.vec(rows * cols, -1.0, 1.0).reshape(rows, cols))
        x = rng.vec(cols, -1.0, 1.0)
        w = upload(m)
        y = N.model_gemv(w, x)
        want = m.dequant().astype(np.float64) @ x.astype(np.float64)
        assert close(y, want, 1e-3).all()
        assert np.array_equal(bits(y), bits(oracle.gemv_batch(m, x)))


BASELINE_SHAPES = [
    # Gemma-3-1B decode (config 1): q, k/v, o, gate/up, down.
    (1024, 1152), (256, 1152), (1152, 1024), (6912, 1152), (1152, 6912),
    # Llama-3-8B projections (config 2).
    (4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336),
    # Gemma-4-E2B-like verify shapes (config 4).
    (6144, 1536), (1536, 6144),
]


@pytest.mark.parametrize("dtype", [1, 2])
@pytest.mark.parametrize("rows,cols", BASELINE_SHAPES)
def test_f32_baseline_shapes_bit_exact(oracle, dtype, rows, cols):
    say("baseline", dtype, rows, cols)
    rng = oracle.Rng(0x5EED00 + rows + cols + dtype)
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    x = rng.normals(cols, 1.0)
    assert np.array_equal(bits(N.model_gemv(w, x)), bits(oracle.gemv_batch(m, x)))


@pytest.mark.parametrize("dtype", [1, 2])
@pytest.mark.parametrize("rows,cols", [(5, 224), (3, 480), (33, 4512), (17, 8192), (17, 8224), (40, 2080),
                                       (300, 2048), (2100, 4096), (4100, 8192), (2050, 4128), (4099, 2080),
                                       (2048, 16384), (2049, 8224), (2048, 18944), (2049, 36864), (2051, 2400),
                                       (2048, 37888)])
def test_f32_one_vector_ring_shapes(oracle, dtype, rows, cols):
    # One vector takes the one-vector kernels up to 8192 columns: rows without
    # a whole group (224 / 480 columns), every tail length class, the
    # 8192-column limit and the first width past it; from 2048 columns the
    # staged kernel with 1 to 8 rows per workgroup (ragged: 300 rows) and 1 to
    # 4 weight copies per wave; from 2048 rows the streamed kernel with 8 or
    # 16 rows per workgroup (ragged: 2049 / 2050 / 2051 / 2100 / 4099 / 4100
    # rows), a partial last group (4128 / 2080 columns; 2400: Q4's bias dot
    # then has body blocks past the whole groups and a 3-block unfused tail),
    # rows past 8192 columns (8224), x of 64 KB (16384), past it (18944:
    # Qwen's down projection) and up to the staging limit of 150 KB (36864:
    # x and Q4's block sums 148.5 KB; 37888: x alone 148 KB, so Q8 streams
    # and Q4 takes the general kernel).
    say("ring", dtype, rows, cols)
    rng = oracle.Rng(0x0E1 + rows + cols + dtype)
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    x = rng.normals(cols, 1.0)
    assert np.array_equal(bits(N.model_gemv(w, x)), bits(oracle.gemv_batch(m, x)))


@pytest.mark.parametrize("dtype", [1, 2])
@pytest.mark.parametrize("rows,cols", [(700, 6912), (2048, 4128), (2048, 8224)])
def test_f32_one_vector_unaligned_x(oracle, dtype, rows, cols):
    # x one float past a 16-byte boundary: the staged and streamed kernels
    # copy x by 16-byte pieces and hand such an x to the register-loading
    # kernel (up to 8192 columns) or the general one (past it).
    import torch
    say("unaligned", dtype, rows, cols)
    rng = oracle.Rng(0xA11 + dtype)
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    x = rng.normals(cols, 1.0)
    want = bits(oracle.gemv_batch(m, x))
    for off in (0, 1):
        xd = torch.zeros(cols + 4, dtype=torch.float32, device="cuda")
        xd[off:off + cols] = torch.from_numpy(x)
        yd = torch.zeros(rows, dtype=torch.float32, device="cuda")
        N.gemv_batch_dev(w, xd.data_ptr() + 4 * off, cols, yd.data_ptr(), rows, 1)
        torch.cuda.synchronize()
        assert np.array_equal(bits(yd.cpu().numpy()), want), off


def rmsnorm_ref(x, r, gamma, eps):
    """nncpu's residual add and RMSNorm restated independently (exact-rounding
    arithmetic of f32_exact.py): v = x + r; sum_sq (scalar.rs:232-250) with
    eight FMA lanes over the whole 8-chunks, hsum8, the tail in f64; the scale
    (float)(1 / sqrt(ss * (1 / dim) + eps)) in f64; (v * scale) * gamma."""
    import math

    from f32_exact import fma32, hsum8
    v = x if r is None else (x + r).astype(np.float32)
    dim = v.size
    body = dim & ~7
    acc = [0.0] * 8
    for i in range(body):
        acc[i % 8] = fma32(float(v[i]), float(v[i]), acc[i % 8])
    ss = float(hsum8(acc)) if dim >= 8 else 0.0
    for i in range(body, dim):
        ss = ss + float(v[i]) * float(v[i])
    inv_dim = float(np.float32(1.0) / np.float32(dim))
    scale = np.float32(1.0 / math.sqrt(ss * inv_dim + float(np.float32(eps))))
    return v, ((v * scale).astype(np.float32) * gamma).astype(np.float32)


@pytest.mark.parametrize("dtype,rows,cols", [(1, 4608, 3584), (2, 4608, 3584), (1, 2048, 3584), (2, 2050, 4128),
                                             (1, 16384, 3584), (2, 16384, 3584), (2, 12300, 1024), (1, 256, 1152),
                                             (2, 3000, 1056), (3, 512, 1024)])
def test_gemv_rmsnorm_dev(oracle, dtype, rows, cols):
    # The fused residual add and RMSNorm in front of the bit-exact gemv
    # (nnh_gemv_rmsnorm_dev): the streamed kernel's prologue (2048+ rows of
    # 64+ blocks; 4608 rows: 16 per workgroup), the tall kernel's (12288+
    # rows), and the norm kernel before the plain gemv otherwise (few rows,
    # short rows, BF16). y, x_out and rec bit-equal an independent
    # restatement of the norm followed by the oracle's gemv; with and without r.
    import torch
    say("rmsnorm gemv", dtype, rows, cols)
    rng = oracle.Rng(0x4E0 + rows + cols + dtype)
    wf = rng.normals(rows * cols, 0.02).reshape(rows, cols)
    if dtype == 3:
        wb = oracle.f32_array_to_bf16(wf.ravel())
        w = N.Weight.bf16(wb, rows, cols)
        wdq = oracle.bf16_array_to_f32(wb).reshape(rows, cols).astype(np.float64)
    else:
        m = oracle.QMatrix.from_f32(dtype, wf)
        w = upload(m)
    x = rng.normals(cols, 1.0)
    rr = rng.normals(cols, 0.5)
    gamma = (1.0 + 0.1 * rng.normals(cols, 1.0)).astype(np.float32)
    eps = 1e-6
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()  # noqa: E731
    xd, rd, gd = dev(x), dev(rr), dev(gamma)
    for use_r in (True, False):
        v, normed = rmsnorm_ref(x, rr if use_r else None, gamma, eps)
        if dtype == 3:
            want = N.model_gemv(w, normed)  # the BF16 path on the normed input (its own parity is tested apart)
        else:
            want = oracle.gemv_batch(m, normed)
        xo = torch.full((cols,), 7.0, device="cuda")
        rec = torch.full((cols,), 7.0, device="cuda")
        scratch = torch.zeros(cols, device="cuda")
        y = torch.zeros(rows, device="cuda")
        N.gemv_rmsnorm_dev(w, xd.data_ptr(), rd.data_ptr() if use_r else 0, gd.data_ptr(), eps, xo.data_ptr(),
                           rec.data_ptr(), scratch.data_ptr(), y.data_ptr())
        torch.cuda.synchronize()
        assert np.array_equal(bits(y.cpu().numpy()), bits(want)), use_r
        assert np.array_equal(bits(xo.cpu().numpy()), bits(v)) and np.array_equal(bits(rec.cpu().numpy()), bits(v))
        assert np.array_equal(bits(xd.cpu().numpy()), bits(x))  # x itself untouched
    with pytest.raises(N.InvalidArgument):
        N.gemv_rmsnorm_dev(w, xd.data_ptr(), rd.data_ptr(), gd.data_ptr(), eps, xd.data_ptr(), 0,
                           scratch.data_ptr(), y.data_ptr())
    w.free()


@pytest.mark.parametrize("dtype,rows,cols", [(1, 4608, 3584), (2, 4608, 3584), (1, 4100, 4096), (2, 20000, 3584),
                                             (2, 2050, 8192), (1, 1000, 6144), (1, 300, 3200), (2, 37, 4128),
                                             (1, 512, 1024), (2, 96, 2048)])
def test_gemv_rmsnorm_i8_dev(oracle, dtype, rows, cols):
    # The int8 mode of the fused norm (nnh_gemv_rmsnorm_act_dev, NNH_ACT_I8):
    # rows of 97..256 blocks run the norm and nncpu's Q8_0 quantizer in the
    # int8 GEMV's prologue (112, 128, 192 and 256 blocks; row groups past
    # four per CU and ragged last groups), other
    # rows the norm kernel before the plain path (1024 and 2048 columns).
    # y bit-equals the independent norm restatement followed by the plain
    # int8 GEMV (nnh_gemv_batch_dev, NNH_ACT_I8) on the same device weight,
    # whose own parity the int8 tests pin; x_out and rec bit-equal v.
    import torch
    say("rmsnorm gemv i8", dtype, rows, cols)
    rng = oracle.Rng(0x18E0 + rows + cols + dtype)
    dw = torch.from_numpy(rng.normals(rows * cols, 0.02)).cuda()
    w = N.Weight.encode_dev(dtype, dw.data_ptr(), rows, cols)
    del dw
    x = rng.normals(cols, 1.0)
    rr = rng.normals(cols, 0.5)
    gamma = (1.0 + 0.1 * rng.normals(cols, 1.0)).astype(np.float32)
    eps = 1e-6
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()  # noqa: E731
    xd, rd, gd = dev(x), dev(rr), dev(gamma)
    for use_r in (True, False):
        v, normed = rmsnorm_ref(x, rr if use_r else None, gamma, eps)
        want = torch.zeros(rows, device="cuda")
        nd = dev(normed)
        N.gemv_batch_dev(w, nd.data_ptr(), cols, want.data_ptr(), rows, 1, N.ACT_I8)
        xo = torch.full((cols,), 7.0, device="cuda")
        rec = torch.full((cols,), 7.0, device="cuda")
        scratch = torch.zeros(cols, device="cuda")
        y = torch.zeros(rows, device="cuda")
        N.gemv_rmsnorm_dev(w, xd.data_ptr(), rd.data_ptr() if use_r else 0, gd.data_ptr(), eps, xo.data_ptr(),
                           rec.data_ptr(), scratch.data_ptr(), y.data_ptr(), act=N.ACT_I8)
        torch.cuda.synchronize()
        got, exp = y.cpu().numpy(), want.cpu().numpy()
        assert np.array_equal(bits(got), bits(exp)), (use_r, int(np.sum(bits(got) != bits(exp))))
        assert np.array_equal(bits(xo.cpu().numpy()), bits(v)) and np.array_equal(bits(rec.cpu().numpy()), bits(v))
        assert np.array_equal(bits(xd.cpu().numpy()), bits(x))
    with pytest.raises(N.InvalidArgument):
        N.gemv_rmsnorm_dev(w, xd.data_ptr(), rd.data_ptr(), gd.data_ptr(), eps, xd.data_ptr(), 0,
                           scratch.data_ptr(), y.data_ptr(), act=N.ACT_I8)
    w.free()


@pytest.mark.parametrize("dtype", [1, 2])
def test_f32_batch_equals_single(oracle, dtype):
    # kernels/tests.rs:641-691: every vector of a batch gets the single-vector bits.
    rng = oracle.Rng(0xBA7C + dtype)
    for n_batch in (2, 3, 4, 7, 16):
        for rows, cols in [(64, 256), (512, 2048), (68, 96), (6, 64)]:
            m = oracle.QMatrix.from_f32(dtype, rng.vec(rows * cols, -1.0, 1.0).reshape(rows, cols))
            w = upload(m)
            xs, ys = cols + 32, rows + 3
            x = rng.vec(n_batch * xs, -1.0, 1.0)
            yb = np.zeros(n_batch * ys, np.float32)
            N.gemv_batch(w, x, xs, yb, ys, n_batch)
            for t in range(n_batch):
                y1 = N.model_gemv(w, x[t * xs:t * xs + cols])
                assert np.array_equal(bits(y1), bits(yb[t * ys:t * ys + rows])), (n_batch, rows, cols, t)
                assert np.array_equal(bits(y1), bits(oracle.gemv_batch(m, x[t * xs:t * xs + cols])))


@pytest.mark.parametrize("dtype", [1, 2])
@pytest.mark.parametrize("rows,cols", [(16400, 96), (16390, 1056), (16384, 32), (16384, 544), (16384, 8192),
                                       (12288, 544), (32800, 1056), (131100, 96)])
def test_f32_tall_layout_bit_exact(oracle, dtype, rows, cols):
    # Matrices of 12288 rows or more take the 8-lane layout; these shapes give
    # it partial groups (nb = 3, 33, 1, 17), a ragged last workgroup, strided
    # batches, the Q4 bias tail, (K = 8192) x too big for four tokens in LDS
    # at once (two per launch), and both lane-group forms of several vectors:
    # one row per lane group, and four (three or more vectors from 32768
    # rows, two from 131072).
    say("tall", dtype, rows, cols)
    rng = oracle.Rng(0x7A11 + rows + cols + dtype)
    m = oracle.QMatrix.from_f32(dtype, rng.vec(rows * cols, -1.0, 1.0).reshape(rows, cols))
    w = upload(m)
    for n_tok in ((1, 3) if cols > 4096 else (1, 3, 4, 6)):
        xs, ys = cols + 32, rows + 3
        x = rng.vec(n_tok * xs, -1.0, 1.0)
        y = np.full(n_tok * ys, 5.0, np.float32)
        N.gemv_batch(w, x, xs, y, ys, n_tok)
        ref = oracle.gemv_batch(m, x, n_tok, xs, ys)
        for t in range(n_tok):
            assert np.array_equal(bits(y[t * ys:t * ys + rows]), bits(ref[t * ys:t * ys + rows])), (n_tok, t)
            assert np.all(y[t * ys + rows:(t + 1) * ys] == 5.0) or t == n_tok - 1


def test_f32_lm_head_gemma_vocab(oracle):
    # The largest decode gemv: the tied Gemma-3 lm_head, 262144 x 1152, Q8_0.
    rows, cols = 262144, 1152
    rng = oracle.Rng(0x5EED03)
    m = oracle.QMatrix.from_f32(1, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    x = rng.normals(cols, 1.0)
    y = N.model_gemv(w, x)
    ref = oracle.gemv_batch(m, x)
    assert np.array_equal(bits(y), bits(ref))
    assert N.model_argmax(w, x) == oracle.argmax(ref)


def test_wide_q4_exact():
    # model/tests.rs:404-423: every weight 1.5, x = 1 -> y = 1.5 * cols exactly.
    cols, rows = 32 * 1025, 2
    n = cols * rows
    w = N.Weight.q4(np.full(n // 2, 0x11, np.uint8), np.full(n // 32, 0x3F80, np.uint16),
                    np.full(n // 32, 0x3F00, np.uint16), rows, cols)
    y = N.model_gemv(w, np.ones(cols, np.float32), act=N.ACT_F32)
    assert np.array_equal(y, np.full(2, 1.5 * cols, np.float32))
    # int8 activations: x = 1 quantizes to q = 127 at scale bf16(1/127), so
    # x' = 127 * 0x3C01 (0.00787353515625) and y = 1.5 * cols * x' exactly.
    xq = 127 * np.float64(np.array([0x3C010000], np.uint32).view(np.float32)[0])
    y = N.model_gemv(w, np.ones(cols, np.float32), act=N.ACT_I8)
    assert np.array_equal(y, np.full(2, np.float32(1.5 * cols * xq)))


def test_argmax_ties_and_nan(oracle):
    rows, cols = 4096, 64
    rng = oracle.Rng(0xA4)
    m = oracle.QMatrix.from_f32(1, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    qs, sc = m.parts[0].copy(), m.parts[1].copy()
    x = rng.normals(cols, 1.0)
    # Rows 3000 and 1000 identical and dominant: the lower row wins.
    qs.reshape(rows, cols)[1000] = 127 * np.sign(x).astype(np.int8)
    qs.reshape(rows, cols)[3000] = qs.reshape(rows, cols)[1000]
    sc.reshape(rows, 2)[[1000, 3000]] = 0x3F80
    w = N.Weight.q8_0(qs, sc, rows, cols)
    assert N.model_argmax(w, x) == 1000
    # A NaN in row 0 keeps row 0 (every `v > NaN` is false).
    sc.reshape(rows, 2)[0] = 0x7FC0
    w = N.Weight.q8_0(qs, sc, rows, cols)
    assert N.model_argmax(w, x) == 0
    # A NaN elsewhere never wins.
    sc.reshape(rows, 2)[0] = 0x3F80
    sc.reshape(rows, 2)[2000] = 0x7FC0
    w = N.Weight.q8_0(qs, sc, rows, cols)
    assert np.isnan(N.model_gemv(w, x)[2000])
    assert N.model_argmax(w, x) == 1000


def test_preconditions():
    w = N.Weight.q8_0(np.zeros(64, np.int8), np.zeros(2, np.uint16), 2, 32)
    with pytest.raises(N.InvalidArgument):
        N.gemv_batch(w, np.zeros(64, np.float32), 32, np.zeros(64, np.float32), 1, 2)
    with pytest.raises(N.InvalidArgument):
        N.Weight.q8_0(np.zeros(40, np.int8), np.zeros(2, np.uint16), 1, 40)
    y = np.full(2, 3.0, np.float32)
    N.gemv_batch(w, np.zeros(32, np.float32), 32, y, 2, 0)  # empty batch: a no-op
    assert np.all(y == 3.0)


def gen_weight(dtype, rows, cols, seed):
    """A device weight of 0.02 N(0, 1) values (torch's generator on the
    GPU), re-encoded by the library's device encoder."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    dw = torch.randn(rows * cols, generator=g, device="cuda", dtype=torch.float32).mul_(0.02)
    w = N.Weight.encode_dev(dtype, dw.data_ptr(), rows, cols)
    del dw
    return w



@pytest.mark.parametrize("dtype", [1, 2])
def test_i8_quantizing_prologue_bit_identity(oracle, dtype):
    # One f32 vector through nnh_gemv_batch_dev(..., NNH_ACT_I8): rows of
    # 97..384 blocks quantize x in the int8 GEMV's own prologue (each
    # pieces-per-thread bound, 128 and 256 blocks, and one past it; the
    # xor and DPP lane trees; ragged grids), except tall Q8 matrices of rows
    # that are not whole 64-block groups; other rows run the quantizer
    # kernel first (96, 385 and 592 blocks). y bit-equals the library
    # quantizer followed by the int8 GEMV on the pre-quantized buffer
    # (nnh_gemv_act_dev), whose parity the int8 tests above pin against the
    # oracle.
    import torch
    for i, (rows, nb) in enumerate([(3584, 97), (1000, 128), (3584, 129), (300, 256), (4100, 257), (3584, 288),
                                    (2000, 384), (777, 385), (3584, 592), (500, 96), (16384, 112), (16400, 128)]):
        cols = nb * 32
        say("i8 quantizing prologue", dtype, rows, cols)
        w = gen_weight(dtype, rows, cols, 0x9A0 + i + dtype)
        x = torch.from_numpy(oracle.Rng(0x9A1 + i).normals(cols, 1.0)).cuda()
        y = torch.zeros(rows, device="cuda")
        N.gemv_batch_dev(w, x.data_ptr(), cols, y.data_ptr(), rows, 1, N.ACT_I8)
        _, _, nbytes = N.act_layout(cols, 1)
        act = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
        N.quantize_act_dev(x.data_ptr(), cols, cols, 1, act.data_ptr())
        want = torch.zeros(rows, device="cuda")
        N.gemv_act_dev(w, N.ACT_I8, act.data_ptr(), 1, want.data_ptr(), rows)
        torch.cuda.synchronize()
        got, exp = y.cpu().numpy(), want.cpu().numpy()
        assert np.array_equal(bits(got), bits(exp)), (rows, nb, int(np.sum(bits(got) != bits(exp))))
        w.free()


# ---- int8 path ---------------------------------------------------------------------

def torch_dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def quantize_on_device(x, cols, n_tok, x_stride=None):
    import torch
    xs = cols if x_stride is None else x_stride
    dx = torch_dev(x)
    off_s, off_sx, nbytes = N.act_layout(cols, n_tok)
    act = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    N.quantize_act_dev(dx.data_ptr(), xs, cols, n_tok, act.data_ptr())
    N.sync()
    a = act.cpu().numpy()
    nb = cols // 32
    q = a[:n_tok * cols].view(np.int8).reshape(n_tok, cols)
    s = a[off_s:off_s + n_tok * nb * 2].view(np.uint16).reshape(n_tok, nb)
    return act, q, s


@pytest.mark.parametrize("cols", [32, 1152, 4096, 18944])
def test_act_quantizer_matches_nncpu_encoder(oracle, cols):
    rng = oracle.Rng(0xAC7 + cols)
    n_tok = 3
    x = rng.normals(n_tok * cols, 1.0)
    x[5] = 0.0
    if cols >= 96:
        x[64:96] = 0.0  # an all-zero block
    _, q, s = quantize_on_device(x, cols, n_tok)
    for t in range(n_tok):
        qo, so = oracle.quantize_act(x[t * cols:(t + 1) * cols])
        assert np.array_equal(q[t], qo) and np.array_equal(s[t], so), t


def test_act_quantizer_reciprocal_tie():
    # An input where amax*(1/127) and amax/127 round to different BF16 scales.
    from oracle import oracle as O
    x = np.zeros(64, np.float32)
    x[3] = np.array([0x3FFEFE01], np.uint32).view(np.float32)[0]
    x[40] = -1.25
    _, q, s = quantize_on_device(x, 64, 1)
    qo, so = O.quantize_act(x)
    assert np.array_equal(s[0], so) and np.array_equal(q[0], qo)


@pytest.mark.parametrize("dtype", [1, 2])
@pytest.mark.parametrize("rows,cols", [(32, 256), (16, 1152), (300, 640), (1024, 4096)])
def test_block_dots_bit_exact(oracle, dtype, rows, cols):
    import torch
    rng = oracle.Rng(0xB0 + rows + dtype)
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    n_tok = 2
    x = rng.normals(n_tok * cols, 1.0)
    act, q, _ = quantize_on_device(x, cols, n_tok)
    P = torch.zeros(n_tok * rows * (cols // 32), dtype=torch.int32, device="cuda")
    N.block_dots_dev(w, act.data_ptr(), n_tok, P.data_ptr())
    N.sync()
    P = P.cpu().numpy().reshape(n_tok, rows, cols // 32)
    for t in range(n_tok):
        assert np.array_equal(P[t], oracle.block_dots(m, q[t]))


@pytest.mark.parametrize("case", [c for c in cases() if c["kind"] == "gemv_i8"], ids=lambda c: c["name"])
def test_i8_golden(oracle, case):
    m, x, y, extra = load_case(oracle, case)
    w = upload(m)
    got = N.model_gemv(w, x, act=N.ACT_I8)
    ulp = np.spacing(np.abs(y))
    assert np.all(np.abs(got - y) <= ulp)


@pytest.mark.parametrize("dtype", [1, 2])
@pytest.mark.parametrize("rows,cols,n_tok", [
    (4096, 4096, 1), (1024, 4096, 1), (14336, 4096, 1), (4096, 14336, 1),
    (6144, 1536, 2), (1536, 6144, 4), (6144, 1536, 8), (1536, 6144, 16),
    (512, 3584, 3), (3584, 18944, 1),
    (3584, 3584, 1), (4100, 3584, 1), (300, 8224, 1),  # one vector: 112 blocks, ragged rows; 257 blocks
])
def test_i8_within_tolerance_of_reference(oracle, dtype, rows, cols, n_tok):
    say("i8", dtype, rows, cols, n_tok)
    rng = oracle.Rng(0x5EED00 + 7 * rows + cols + dtype)
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    x = rng.normals(n_tok * cols, 1.0)
    y = np.zeros(n_tok * rows, np.float32)
    N.gemv_batch(w, x, cols, y, rows, n_tok, N.ACT_I8)
    for t in range(n_tok):
        qx, sx = oracle.quantize_act(x[t * cols:(t + 1) * cols])
        ref = oracle.gemv_batch(m, oracle.dequant_act(qx, sx))
        got = y[t * rows:(t + 1) * rows]
        # north-star tolerances against nncpu's kernel on the same (dequantized) inputs
        assert np.abs(got - ref).max() <= 1e-5
        assert np.linalg.norm(got - ref) <= 1e-3 * np.linalg.norm(ref)
        if rows * cols <= 4096 * 4096:
            exact = oracle.gemv_i8_exact(m, qx, sx)
            assert np.all(np.abs(got - exact) <= np.spacing(np.abs(exact)))


@pytest.mark.parametrize("dtype,rows,cols", [
    (1, 8200, 4096), (1, 8192, 6144), (1, 3600, 8192), (1, 4096, 14336), (1, 9000, 4096), (1, 3584, 10240),
    (2, 3584, 9216), (2, 3584, 18944), (2, 5000, 8224),
])
def test_i8_staged_kernel_shapes(oracle, dtype, rows, cols):
    # One vector at the shapes of the int8 kernel with the activations staged
    # in LDS and rows taken grid-stride (Q8 rows of whole 64-block groups at
    # 8192+ rows or of 256+ blocks; Q4 rows of 257+ blocks that are not whole
    # groups; both lane trees, ragged grids and chunks): within
    # one ulp of the oracle's exact sum of the exact block terms; against
    # nncpu's kernel fed x', within 1e-5 except where nncpu's own f32 chains
    # are farther from the exact sum than this kernel (as the config-5 test
    # counts them: at K = 18944 nncpu is up to ~1.6e-5 from exact).
    say("i8 staged", dtype, rows, cols)
    rng = oracle.Rng(0x57A6 + rows + cols + dtype)
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    x = rng.normals(cols, 1.0)
    got = N.model_gemv(w, x, act=N.ACT_I8)
    qx, sx = oracle.quantize_act(x)
    exact = oracle.gemv_i8_exact(m, qx, sx)
    assert np.all(np.abs(got - exact) <= np.spacing(np.abs(exact)))
    ref = oracle.gemv_batch(m, oracle.dequant_act(qx, sx))
    over = np.abs(got - ref) > 1e-5
    print(f"above 1e-5 against nncpu: {int(over.sum())} of {rows}, max {np.abs(got - ref).max():.3g}")
    assert np.all(np.abs(got - exact)[over] < np.abs(ref - exact)[over].astype(np.float64))
    assert np.linalg.norm(got - ref) <= 1e-3 * np.linalg.norm(ref)
    w.free()


def i8_abs_terms(oracle, m, qx, sx):
    """sum_b |s_w s_x P_b| (+ |bias s_x sum q_x| for Q4) per row, in f64."""
    nb = m.cols // 32
    P = oracle.block_dots(m, qx).astype(np.float64)
    sw = oracle.bf16_array_to_f32(m.parts[1]).astype(np.float64).reshape(m.rows, nb)
    sxf = oracle.bf16_array_to_f32(np.ascontiguousarray(sx)).astype(np.float64)
    t = np.abs(sw * sxf[None, :] * P).sum(axis=1)
    if m.dtype == 2:
        bi = oracle.bf16_array_to_f32(m.parts[2]).astype(np.float64).reshape(m.rows, nb)
        qsum = np.asarray(qx, np.int64).reshape(nb, 32).sum(axis=1).astype(np.float64)
        t += np.abs(bi * (sxf * qsum)[None, :]).sum(axis=1)
    return t


@pytest.mark.parametrize("dtype", [1, 2])
@pytest.mark.parametrize("rows,cols,n_tok", [
    (512, 3584, 512),   # Qwen2.5-7B k/v projection, a full 512-token prefill (config 5)
    (300, 640, 100),    # ragged rows and tokens
    (1536, 1536, 16),   # Gemma-4-E2B-like verify, M = 16 (config 4)
    (200, 96, 37),      # nb = 3
    (129, 6144, 5),     # the smallest GEMM batch, K = 6144
    (1536, 64, 2048),   # 192 tiles: the unsplit path, nb = 2 (one partial chunk)
    (4100, 1536, 12),   # few-token kernel: ragged row group, K split over 2 workgroups
    (200, 96, 9),       # few-token kernel: nb = 3, a lone block in the last pair
    (1536, 6144, 5),    # few-token kernel at its lower bound, K split over 5 workgroups
    (96, 4128, 11),     # few-token kernel: nb = 129, a partial last stage, 3 row groups
    (6144, 1536, 8),    # few-token kernel, unsplit, tokens in registers 0-3 only
    (333, 1536, 4),     # few-token kernel at its lower bound (4 tokens), ragged rows
    (1536, 6144, 16),   # few-token kernel, 16 tokens staged, K split
])
def test_i8_gemm_bit_exact_sums(oracle, dtype, rows, cols, n_tok):
    # The MFMA GEMM (17 vectors or more) forms every block dot exactly and
    # sums the block terms in f32 over chunks of 8 blocks, the chunks in
    # f64: each output must be within 16 f32 roundings of its absolute block
    # terms (8 FMAs per chunk, the Q4 bias products and their sums) plus one
    # ulp of the oracle's exact sum (any wrong P_b would be far off); the
    # few-token kernels keep one ulp. And within the north-star tolerance of
    # nncpu's kernel fed x'.
    say("gemm", dtype, rows, cols, n_tok)
    rng = oracle.Rng(0x6E33 + rows + cols + n_tok + dtype)
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    xs, ys = cols + 32, rows + 7
    x = rng.normals(n_tok * xs, 1.0)
    y = np.full(n_tok * ys, 7.0, np.float32)
    N.gemv_batch(w, x, xs, y, ys, n_tok, N.ACT_I8)
    deq = []
    for t in range(n_tok):
        qx, sx = oracle.quantize_act(x[t * xs:t * xs + cols])
        exact = oracle.gemv_i8_exact(m, qx, sx)
        got = y[t * ys:t * ys + rows]
        bound = np.spacing(np.abs(exact))
        if n_tok > 16:
            bound = bound + 16 * 2.0 ** -24 * i8_abs_terms(oracle, m, qx, sx)
        assert np.all(np.abs(got - exact) <= bound), t
        assert np.all(y[t * ys + rows:(t + 1) * ys] == 7.0) or t == n_tok - 1
        deq.append(oracle.dequant_act(qx, sx))
    sample = list(range(0, n_tok, max(1, n_tok // 8)))
    xd = np.concatenate([deq[t] for t in sample])
    ref = oracle.gemv_batch(m, xd, len(sample), cols, rows)
    for i, t in enumerate(sample):
        got = y[t * ys:t * ys + rows]
        r = ref[i * rows:(i + 1) * rows]
        assert np.abs(got - r).max() <= 1e-5
        assert np.linalg.norm(got - r) <= 1e-3 * np.linalg.norm(r)


@pytest.mark.parametrize("dtype", [1, 2])
def test_i8_few_token_split_repeated_and_graph(oracle, dtype):
    # With K split, the few-token kernel's partials meet in the workspace and
    # a second kernel adds them: calls in a row on one weight (different token
    # counts) and replays of a captured graph, with eager work between them,
    # each keep one ulp of the exact sum, and the replays the eager bits.
    import torch
    rows, cols = 1536, 6144
    say("split repeat", dtype, rows, cols)
    rng = oracle.Rng(0x5C17 + dtype)
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)

    def check(x, n_tok, y):
        for t in range(n_tok):
            qx, sx = oracle.quantize_act(x[t * cols:(t + 1) * cols])
            exact = oracle.gemv_i8_exact(m, qx, sx)
            assert np.all(np.abs(y[t * rows:(t + 1) * rows] - exact) <= np.spacing(np.abs(exact))), (n_tok, t)

    for n_tok in (8, 4, 16, 5, 8):
        x = rng.normals(n_tok * cols, 1.0)
        y = np.zeros(n_tok * rows, np.float32)
        N.gemv_batch(w, x, cols, y, rows, n_tok, N.ACT_I8)
        check(x, n_tok, y)
    n_tok = 8
    x = rng.normals(n_tok * cols, 1.0)
    dx = torch_dev(x)
    dy = torch.zeros(n_tok * rows, device="cuda")
    st = torch.cuda.Stream()
    N.gemv_batch_dev(w, dx.data_ptr(), cols, dy.data_ptr(), rows, n_tok, N.ACT_I8, st.cuda_stream)
    torch.cuda.synchronize()
    ref = dy.cpu().numpy().copy()
    check(x, n_tok, ref)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        N.gemv_batch_dev(w, dx.data_ptr(), cols, dy.data_ptr(), rows, n_tok, N.ACT_I8, st.cuda_stream)
    for _ in range(3):
        dy.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(dy.cpu().numpy(), ref)
        y2 = np.zeros(4 * rows, np.float32)  # eager work between replays
        N.gemv_batch(w, x[:4 * cols], cols, y2, rows, 4, N.ACT_I8)
        assert np.array_equal(y2, ref[:4 * rows])


# ---- device re-encoder (kernels/quant.rs:31-95 on the GPU) ----------------------------

def encode_on_device(dtype, w, rows, cols):
    import torch
    dw = torch_dev(np.ascontiguousarray(w, np.float32).ravel())
    return N.Weight.encode_dev(dtype, dw.data_ptr(), rows, cols)


@pytest.mark.parametrize("dtype", [1, 2])
def test_device_encoder_bit_exact(oracle, dtype):
    rng = oracle.Rng(0xE7C0 + dtype)
    rows, cols = 333, 1152
    w = rng.normals(rows * cols, 0.02).reshape(rows, cols)
    # Edge blocks: signed zeros (first occurrence wins for Q4 lo/hi), flat,
    # all zero, NaN in b[0] and elsewhere, large values, reciprocal ties.
    w[0, :32] = 0.0
    w[0, 5] = -0.0
    w[1, :32] = np.where(np.arange(32) % 2 == 0, -0.0, 0.0)
    w[2, :32] = 3.5
    w[3, 0] = np.nan
    w[4, 7] = np.nan
    w[5, :32] = rng.vec(32, -3e4, 3e4)
    w[6, :32] = 0.0
    w[6, 3] = np.array([0x3FFEFE01], np.uint32).view(np.float32)[0]
    w[7, :32] = 0.0
    w[7, 9] = np.array([0x3F895800], np.uint32).view(np.float32)[0]
    w[8, 32:64] = -1.0
    w[8, 40] = 2.0
    dev = encode_on_device(dtype, w, rows, cols)
    got = dev.download()
    want = oracle.QMatrix.from_f32(dtype, w).buf
    assert got.size == want.size
    assert np.array_equal(got, want), np.nonzero(got != want)[0][:10]


@pytest.mark.parametrize("dtype", [1, 2, 3])
def test_encode_is_complete_when_it_returns(oracle, dtype):
    # nnh_encode_dev (and the uploads) return only once the weight is written:
    # the f32 source freed and its memory overwritten straight after the call
    # must not reach the encoded weight. Then the split layout is read through
    # the int8 GEMV of one vector (no derived layout for Q8_0) on torch's
    # stream, with no other ordering.
    import torch
    rng = oracle.Rng(0xE7D0 + dtype)
    rows, cols = 4096, 4096
    w = rng.normals(rows * cols, 0.02).reshape(rows, cols)
    dw = torch_dev(np.ascontiguousarray(w, np.float32).ravel())
    dev = N.Weight.encode_dev(dtype, dw.data_ptr(), rows, cols)
    dw.fill_(1e6)
    del dw
    junk = torch.full((rows * cols,), -7.0, device="cuda")
    torch.cuda.synchronize()
    del junk
    got = dev.download()
    if dtype == 3:
        want = oracle.f32_array_to_bf16(w.ravel()).view(np.uint8)
    else:
        want = oracle.QMatrix.from_f32(dtype, w).buf
    assert np.array_equal(got, want), np.nonzero(got != want)[0][:10]
    if dtype != 3:
        x = rng.normals(cols, 1.0)
        assert np.abs(N.model_gemv(dev, x, act=N.ACT_I8) - oracle.gemv_batch(
            oracle.QMatrix.from_f32(dtype, w), oracle.dequant_act(*oracle.quantize_act(x)))).max() <= 1e-5
    dev.free()


@pytest.mark.parametrize("dtype", [1, 2])
def test_device_encoded_weight_matmul(oracle, dtype):
    # The encoded weight is a complete weight: its f32 matmul matches the
    # oracle bit for bit.
    rng = oracle.Rng(0xE7C5 + dtype)
    rows, cols = 1024, 4096
    w = rng.normals(rows * cols, 0.02).reshape(rows, cols)
    dev = encode_on_device(dtype, w, rows, cols)
    m = oracle.QMatrix.from_f32(dtype, w)
    x = rng.normals(cols, 1.0)
    assert np.array_equal(bits(N.model_gemv(dev, x)), bits(oracle.gemv_batch(m, x)))


@pytest.mark.parametrize("dtype", [1, 2])
@pytest.mark.parametrize("rows,cols", [(16384, 1152), (20000, 64), (3000, 1152)])
def test_model_argmax_dev(oracle, dtype, rows, cols):
    # model_argmax (forward.rs:989-1011) on device buffers: tall matrices take
    # the gemv with the argmax's first stage fused in, the rest the two-kernel
    # argmax; both the first largest logit (ties to the lower row, a NaN in
    # row 0 keeps row 0). The logits are written either way.
    import torch
    say("argmax_dev", dtype, rows, cols)
    rng = oracle.Rng(0xA5 + rows + dtype)
    w = rng.normals(rows * cols, 0.02).reshape(rows, cols)
    m = oracle.QMatrix.from_f32(dtype, w)
    wt = upload(m)
    work = torch.zeros(N.model_argmax_work_bytes(wt), dtype=torch.uint8, device="cuda")
    logits = torch.zeros(rows, dtype=torch.float32, device="cuda")
    out = torch.zeros(1, dtype=torch.int64, device="cuda")
    for case in ("plain", "nan0"):
        x = rng.normals(cols, 1.0)
        if case == "nan0":
            x[0] = np.nan  # every logit NaN: row 0
        want_y = oracle.gemv_batch(m, x)
        xd = torch.from_numpy(x).cuda()
        N.model_argmax_dev(wt, xd.data_ptr(), logits.data_ptr(), work.data_ptr(), out.data_ptr())
        torch.cuda.synchronize()
        assert np.array_equal(bits(logits.cpu().numpy()), bits(want_y)), case
        assert int(out.item()) == oracle.argmax(want_y), case
        assert N.model_argmax(wt, x) == oracle.argmax(want_y), case


def test_model_argmax_dev_ties(oracle):
    # Equal maxima in several rows of a tall Q8 matrix: the lowest row.
    import torch
    rows, cols = 16384, 64
    w = np.zeros((rows, cols), np.float32)
    for r in (7000, 300, 16000):
        w[r, 0] = 1.0
    m = oracle.QMatrix.from_f32(1, w)
    wt = upload(m)
    x = np.zeros(cols, np.float32)
    x[0] = 2.0
    work = torch.zeros(N.model_argmax_work_bytes(wt), dtype=torch.uint8, device="cuda")
    logits = torch.zeros(rows, dtype=torch.float32, device="cuda")
    out = torch.zeros(1, dtype=torch.int64, device="cuda")
    N.model_argmax_dev(wt, torch.from_numpy(x).cuda().data_ptr(), logits.data_ptr(), work.data_ptr(), out.data_ptr())
    torch.cuda.synchronize()
    assert int(out.item()) == 300 == oracle.argmax(oracle.gemv_batch(m, x))
