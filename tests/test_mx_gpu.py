"""The MX int8 path (NNH_ACT_MXI8) through the C-ABI (needs an MI355X).

Activations are quantized to int8 blocks of 32 with a power-of-two scale;
from 17 vectors the matmul runs on the BF16 matrix unit with exact block
dots. Checks: the quantizer's whole buffer bit for bit against the oracle
restatement (oracle.quantize_act_mx, pinned in test_mx.py); the int32 block
dots bit for bit; every GEMM output within its f32-chunk rounding bound of
the exact sum of the block terms (a wrong block dot, scale or bias term is
far outside it); and the north-star tolerance (1e-5 absolute, 1e-3 relative
L2) against nncpu's own kernel (the oracle's restatement) fed the dequantized
activations.
"""
import sys

import numpy as np
import pytest

from conftest import bits

pytestmark = pytest.mark.gpu

N = pytest.importorskip("nncpu_amd")

U32 = 2.0 ** -24


@pytest.fixture(scope="module", autouse=True)
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    N.init(0)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def upload(m):
    if m.dtype == 1:
        return N.Weight.q8_0(m.parts[0], m.parts[1], m.rows, m.cols)
    return N.Weight.q4(m.parts[0], m.parts[1], m.parts[2], m.rows, m.cols)


def torch_dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def align(v):
    return (v + 255) // 256 * 256


def mx_buffer(x, cols, n_tok, xs):
    """Quantize on the device; return the buffer and its fields (the layout
    include/nncpu_hip.h documents: the NNH_ACT_I8 layout, then xb, then xl)."""
    import torch
    off_s, off_sx, nbytes = N.act_layout_ex(N.ACT_MXI8, cols, n_tok)
    _, _, i8_bytes = N.act_layout_ex(N.ACT_I8, cols, n_tok)
    dx = torch_dev(x)
    buf = torch.full((nbytes,), 0xA5, dtype=torch.uint8, device="cuda")  # stale bytes must not leak through
    N.quantize_act_ex_dev(N.ACT_MXI8, dx.data_ptr(), xs, cols, n_tok, buf.data_ptr())
    N.sync()
    a = buf.cpu().numpy()
    nb = cols // 32
    nbp8 = (nb + 7) // 8 * 8
    tok_pad = (n_tok + 127) // 128 * 128
    off_xb = i8_bytes
    off_xl = off_xb + align((n_tok + 255) // 256 * 256 * cols * 2)
    tiles = (n_tok + 255) // 256
    # xb: [tile][block][256 tokens][32], chunk c of a row at c ^ ((row >> 2) & 3)
    xt = a[off_xb:off_xb + tiles * 256 * cols * 2].view(np.uint16).reshape(tiles, nb, 256, 4, 8)
    rows = np.arange(256)
    unswz = np.stack([xt[:, :, rows, c ^ ((rows >> 2) & 3), :] for c in range(4)], axis=3)  # [tile][b][row][c][8]
    xb_all = unswz.transpose(0, 2, 1, 3, 4).reshape(tiles * 256, cols)
    f = dict(
        q=a[:n_tok * cols].view(np.int8).reshape(n_tok, cols),
        s=a[off_s:off_s + n_tok * nb * 2].view(np.uint16).reshape(n_tok, nb),
        sx=a[off_sx:off_sx + n_tok * nb * 16].view(np.float64).reshape(n_tok, nb, 2),
        xb=xb_all[:n_tok],
        xb_pad=xb_all[n_tok:],
        xl=a[off_xl:off_xl + tok_pad * nbp8 * 4].view(np.uint16).reshape(tok_pad, nbp8, 2),
    )
    return buf, f


def special_x(rng, n_tok, xs, cols):
    """N(0,1) activations with edge blocks: all zero, a NaN, subnormal-only,
    a mantissa-boundary maximum, huge values."""
    x = rng.normals(n_tok * xs, 1.0)
    row = x[:cols]
    if cols >= 6 * 32:
        row[0:32] = 0.0
        row[37] = np.nan
        row[64:96] = np.float32(1e-40) * np.arange(1, 33, dtype=np.float32)
        row[96:128] *= 0.1
        row[100] = np.uint32(0x3FFE0000).view(np.float32)  # 1.984375: 127 * 2^-6 exactly
        row[128:160] *= np.float32(3e30)
        row[160:192] *= 0.1
        row[175] = -np.uint32(0x3FFE0001).view(np.float32)  # just above: needs 2^-5
        row[170] = np.float32(-1e-30)
    return x


@pytest.mark.parametrize("cols,n_tok", [(32, 3), (1152, 3), (4096, 2), (18944, 1), (256, 130)])
def test_mx_quantizer_buffer_bit_exact(oracle, cols, n_tok):
    say("mx quantizer", cols, n_tok)
    rng = oracle.Rng(0x3A11 + cols + n_tok)
    xs = cols + 32 if n_tok > 1 else cols
    x = special_x(rng, n_tok, xs, cols)
    _, f = mx_buffer(x, cols, n_tok, xs)
    nb = cols // 32
    nbp8 = (nb + 7) // 8 * 8
    for t in range(n_tok):
        q, s = oracle.quantize_act_mx(x[t * xs:t * xs + cols])
        assert np.array_equal(f["q"][t], q), t
        assert np.array_equal(f["s"][t], s), t
        sf = oracle.bf16_array_to_f32(s).astype(np.float64)
        X = sf * q.reshape(nb, 32).astype(np.int64).sum(axis=1)
        assert np.array_equal(f["sx"][t][:, 0], sf)
        assert np.array_equal(f["sx"][t][:, 1], X)
        xb = (oracle.bf16_array_to_f32(s).repeat(32) * q.astype(np.float32)).astype(np.float32)
        assert np.array_equal(f["xb"][t], (xb.view(np.uint32) >> 16).astype(np.uint16))
        hi, lo = oracle.mx_limbs(X.astype(np.float32))
        assert np.array_equal(f["xl"][t][:nb, 0], hi) and np.array_equal(f["xl"][t][:nb, 1], lo)
        assert np.all(f["xl"][t][nb:] == 0)
    assert np.all(f["xl"][n_tok:] == 0)  # pad tokens
    assert np.all(f["xb_pad"] == 0)
    assert nbp8 % 8 == 0


@pytest.mark.parametrize("dtype", [1, 2])
def test_mx_block_dots_bit_exact(oracle, dtype):
    import torch
    rows, cols, n_tok = 77, 1152, 3
    rng = oracle.Rng(0xB10C + dtype)
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    x = rng.normals(n_tok * cols, 1.0)
    buf, f = mx_buffer(x, cols, n_tok, cols)
    P = torch.zeros(n_tok * rows * (cols // 32), dtype=torch.int32, device="cuda")
    N.block_dots_dev(w, buf.data_ptr(), n_tok, P.data_ptr())
    N.sync()
    got = P.cpu().numpy().reshape(n_tok, rows, cols // 32)
    for t in range(n_tok):
        assert np.array_equal(got[t], oracle.block_dots(m, f["q"][t])), t


def check_gemm(oracle, m, y, ys, x, xs, n_tok, sample_ref=True):
    """y (host, n_tok rows ys apart) against the exact sum and nncpu's kernel."""
    rows, cols = m.rows, m.cols
    qs, ss = [], []
    for t in range(n_tok):
        q, s = oracle.quantize_act_mx(x[t * xs:t * xs + cols])
        qs.append(q)
        ss.append(s)
    exact, mag = oracle.gemm_exact(m, np.concatenate(qs), np.concatenate(ss), n_tok)
    got = np.stack([y[t * ys:t * ys + rows] for t in range(n_tok)]).astype(np.float64)
    # f32 chunks of 16 blocks: 16 FMAs each (Q4: plus two bias MFMAs of up to
    # 17 roundings), each chunk added into an f32 total (at most one rounding
    # per 8-block group, the split tiles' partials summed in f64): within
    # (K + groups) u sum|terms| + one ulp of the result.
    groups = (cols // 32 + 7) // 8
    k = (16 if m.dtype == 1 else 64) + groups
    bound = k * U32 * mag + np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    bad = np.abs(got - exact) > bound
    assert not bad.any(), (np.argwhere(bad)[:5], (got - exact)[bad][:5], bound[bad][:5])
    if not sample_ref:
        return
    sample = sorted(set([0, n_tok - 1] + list(range(0, n_tok, max(1, n_tok // 6)))))
    xd = np.concatenate([oracle.dequant_act(qs[t], ss[t]) for t in sample])
    ref = oracle.gemv_batch(m, xd, len(sample), cols, rows)
    for i, t in enumerate(sample):
        r = ref[i * rows:(i + 1) * rows]
        assert np.abs(got[t] - r).max() <= 1e-5, t
        assert np.linalg.norm(got[t] - r) <= 1e-3 * np.linalg.norm(r), t


@pytest.mark.parametrize("dtype", [1, 2])
@pytest.mark.parametrize("rows,cols,n_tok", [
    (512, 3584, 512),    # Qwen2.5-7B k/v projection, a full 512-token prefill (config 5)
    (3584, 3584, 512),   # Qwen2.5-7B q/o projection, M = 512 (config 5)
    (300, 640, 100),     # ragged rows and tokens
    (200, 96, 37),       # nb = 3: one partial group
    (1000, 1152, 129),   # nb = 36 (4.5 groups), two token tiles, the second with one token
    (128, 18944, 17),    # one row tile over many teams: the fixup adds dozens of partial tiles
    (1536, 64, 2048),    # nb = 2, sixteen token tiles
    (4100, 1536, 300),   # ragged row tile, three token tiles
    (1536, 1536, 17),    # the smallest GEMM batch at a Gemma-4-E2B-like shape (config 4)
    (18944, 3584, 512),  # Qwen2.5-7B gate/up, M = 512: a data-parallel round, then a stream-K tail
    (18944, 512, 300),   # a tail of fewer units than teams: empty tail shares, tiles split in two
])
def test_mx_gemm_exact_bound_and_tolerance(oracle, dtype, rows, cols, n_tok):
    say("mx gemm", dtype, rows, cols, n_tok)
    rng = oracle.Rng(0x4D58 + rows + cols + n_tok + dtype)
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    xs, ys = cols + 32, rows + 7
    x = rng.normals(n_tok * xs, 1.0)
    y = np.full(n_tok * ys, 7.0, np.float32)
    N.gemv_batch(w, x, xs, y, ys, n_tok, N.ACT_MXI8)
    for t in range(n_tok - 1):
        assert np.all(y[t * ys + rows:(t + 1) * ys] == 7.0), t  # stride gaps untouched
    check_gemm(oracle, m, y, ys, x, xs, n_tok, sample_ref=rows * cols <= 4096 * 4096)


@pytest.mark.parametrize("dtype", [1, 2])
@pytest.mark.parametrize("n_tok", [1, 3, 4, 16])
def test_mx_few_vectors_one_ulp(oracle, dtype, n_tok):
    # Below 17 vectors the MX buffer goes through the GEMV / few-token
    # kernels, which keep one ulp of the exact sum.
    rows, cols = 1536, 1536
    rng = oracle.Rng(0x4D59 + n_tok + dtype)
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    x = rng.normals(n_tok * cols, 1.0)
    y = np.zeros(n_tok * rows, np.float32)
    N.gemv_batch(w, x, cols, y, rows, n_tok, N.ACT_MXI8)
    for t in range(n_tok):
        q, s = oracle.quantize_act_mx(x[t * cols:(t + 1) * cols])
        exact = oracle.gemv_i8_exact(m, q, s)
        got = y[t * rows:(t + 1) * rows]
        assert np.all(np.abs(got - exact) <= np.spacing(np.abs(exact))), t


@pytest.mark.parametrize("dtype", [1, 2])
def test_mx_gemm_deterministic_and_graph_replay(oracle, dtype):
    # Repeated calls give the same bits (split tiles are added in a fixed
    # order), and so do replays of a captured call with eager work between.
    import torch
    rows, cols, n_tok = 1000, 3584, 200
    rng = oracle.Rng(0x4D5A + dtype)
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    x = rng.normals(n_tok * cols, 1.0)
    dx = torch_dev(x)
    dy = torch.zeros(n_tok * rows, device="cuda")
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        N.gemv_batch_dev(w, dx.data_ptr(), cols, dy.data_ptr(), rows, n_tok, N.ACT_MXI8, st.cuda_stream)
    torch.cuda.synchronize()
    eager = dy.cpu().numpy().copy()
    check_gemm(oracle, m, eager, rows, x, cols, n_tok, sample_ref=False)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        N.gemv_batch_dev(w, dx.data_ptr(), cols, dy.data_ptr(), rows, n_tok, N.ACT_MXI8, st.cuda_stream)
    for rep in range(3):
        dy.fill_(-1.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(dy.cpu().numpy()), bits(eager)), rep
        junk = torch.randn(1 << 20, device="cuda").sum()  # eager work between replays
        torch.cuda.synchronize()
        del junk


def test_mx_argmax_and_model_gemv(oracle):
    rows, cols = 5000, 1152
    rng = oracle.Rng(0x4D5B)
    m = oracle.QMatrix.from_f32(1, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    x = rng.normals(cols, 1.0)
    y = N.model_gemv(w, x, act=N.ACT_MXI8)
    q, s = oracle.quantize_act_mx(x)
    exact = oracle.gemv_i8_exact(m, q, s)
    assert np.all(np.abs(y - exact) <= np.spacing(np.abs(exact)))
    assert N.model_argmax(w, x, act=N.ACT_MXI8) == oracle.argmax(y)


@pytest.mark.parametrize("dtype", [1, 2])
def test_mx_gemm_edge_blocks(oracle, dtype):
    # Activations with zero, NaN, subnormal, mantissa-boundary and ~1e30
    # blocks (scales from 2^-126 to about 2^96, X limbs at both ends) through the
    # BF16 GEMM: within the exact-sum bound like any other input.
    rows, cols, n_tok = 200, 1152, 20
    rng = oracle.Rng(0x4D5C + dtype)
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    x = special_x(rng, n_tok, cols, cols)
    for t in range(1, n_tok, 3):  # the edge blocks in other tokens too, shifted
        x[t * cols:(t + 1) * cols] = np.roll(x[:cols], 32 * t)
    y = np.zeros(n_tok * rows, np.float32)
    N.gemv_batch(w, x, cols, y, rows, n_tok, N.ACT_MXI8)
    assert np.all(np.isfinite(y))
    check_gemm(oracle, m, y, rows, x, cols, n_tok, sample_ref=False)
