"""Device memory of the library (needs an MI355X): derived weight layouts
built on first use, one scratch buffer per calling stream, and captured
calls that stay valid after the scratch grows."""
import sys

import numpy as np
import pytest

from conftest import bits

pytestmark = pytest.mark.gpu

N = pytest.importorskip("nncpu_amd")


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


def align(v):
    return (v + 255) // 256 * 256


@pytest.mark.parametrize("dtype", [1, 2])
def test_layouts_are_built_on_first_use(oracle, dtype):
    # An upload holds nncpu's split layout only; each mode adds its own
    # layouts once, and results do not depend on when they were built.
    rows, cols = 1000, 1152
    say("lazy layouts", dtype)
    rng = oracle.Rng(0x1A2 + dtype)
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    n = rows * cols
    raw = n + n // 16 if dtype == 1 else n // 2 + n // 8
    assert w.device_bytes() == align(raw)
    x = rng.normals(20 * cols, 1.0)
    y = N.model_gemv(w, x[:cols])
    assert np.array_equal(bits(y), bits(oracle.gemv_batch(m, x[:cols])))
    after_f32 = w.device_bytes()
    assert after_f32 > align(raw)
    N.model_gemv(w, x[:cols])
    assert w.device_bytes() == after_f32  # built once
    y1 = N.model_gemv(w, x[:cols], act=N.ACT_I8)
    after_gemv = w.device_bytes()
    assert (after_gemv > after_f32) == (dtype == 2)  # Q4: the packed scale | bias words
    y20 = np.zeros(20 * rows, np.float32)
    N.gemv_batch(w, x, cols, y20, rows, 20, N.ACT_MXI8)
    after_mx = w.device_bytes()
    # The MX GEMM reads the quants in place: it adds the block-major f32
    # scales (Q8 one spare block row; Q4 the biases too) and Q4's BF16 bias
    # table, rows padded to whole 128-row tiles, and no copy of the quants.
    rows_pad, nb = (rows + 127) // 128 * 128, cols // 32
    swt = rows_pad * 4 * (nb + 1 if dtype == 1 else 2 * nb)
    wbi = rows_pad * ((nb + 7) // 8 * 8) * 4 if dtype == 2 else 0
    assert after_mx - after_gemv == align(swt) + (align(wbi) if wbi else 0)
    qx, sx = oracle.quantize_act(x[:cols])
    exact = oracle.gemv_i8_exact(m, qx, sx)
    assert np.all(np.abs(y1 - exact) <= np.spacing(np.abs(exact)))
    # Prepared ahead on a fresh upload: same bytes as lazily, same results.
    w2 = upload(m).prepare(N.ACT_F32).prepare(N.ACT_I8, 1).prepare(N.ACT_MXI8, 20)
    assert w2.device_bytes() == after_mx
    y20b = np.zeros(20 * rows, np.float32)
    N.gemv_batch(w2, x, cols, y20b, rows, 20, N.ACT_MXI8)
    assert np.array_equal(bits(y20), bits(y20b))


@pytest.mark.parametrize("act", [0, 1, 2])
def test_captured_call_survives_scratch_growth(oracle, act):
    # A call captured in a HIP graph keeps its scratch: after a larger call
    # on the same stream grows that stream's scratch, replays still give the
    # eager bits (the old buffer is kept, not freed).
    import torch
    rows, cols, n_small = 512, 3584, 20
    say("capture then grow", act)
    rng = oracle.Rng(0xC4 + act)
    dtype = 2  # Q4: the f32 path uses the scratch for its block sums too
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    st = torch.cuda.Stream()
    x = torch.from_numpy(rng.normals(600 * cols, 1.0)).cuda()
    y = torch.zeros(n_small * rows, device="cuda")
    yl = torch.zeros(600 * rows, device="cuda")
    N.gemv_batch_dev(w, x.data_ptr(), cols, y.data_ptr(), rows, n_small, act, st.cuda_stream)
    torch.cuda.synchronize()
    eager = y.cpu().numpy().copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        N.gemv_batch_dev(w, x.data_ptr(), cols, y.data_ptr(), rows, n_small, act, st.cuda_stream)
    for big in (200, 600):
        N.gemv_batch_dev(w, x.data_ptr(), cols, yl.data_ptr(), rows, big, act, st.cuda_stream)
        torch.cuda.synchronize()
        y.fill_(-1.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(y.cpu().numpy()), bits(eager)), big
    if act == 0:  # f32 path: every vector keeps its single-call bits in any batch
        assert np.array_equal(bits(yl[:n_small * rows].cpu().numpy()), bits(eager))


def test_streams_have_their_own_scratch(oracle):
    # Calls queued on two streams at once (int8 path: quantized activations
    # and split-K partials in scratch) do not disturb each other.
    import torch
    rows, cols = 1536, 6144
    say("two streams")
    rng = oracle.Rng(0x257)
    m = oracle.QMatrix.from_f32(1, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    xa = torch.from_numpy(rng.normals(8 * cols, 1.0)).cuda()
    xb = torch.from_numpy(rng.normals(8 * cols, 1.0)).cuda()
    ya = torch.zeros(8 * rows, device="cuda")
    yb = torch.zeros(8 * rows, device="cuda")
    torch.cuda.synchronize()
    for _ in range(20):
        N.gemv_batch_dev(w, xa.data_ptr(), cols, ya.data_ptr(), rows, 8, N.ACT_I8, sa.cuda_stream)
        N.gemv_batch_dev(w, xb.data_ptr(), cols, yb.data_ptr(), rows, 8, N.ACT_I8, sb.cuda_stream)
    torch.cuda.synchronize()
    for x, y in ((xa, ya), (xb, yb)):
        xh = x.cpu().numpy()
        yh = y.cpu().numpy()
        for t in range(8):
            qx, sx = oracle.quantize_act(xh[t * cols:(t + 1) * cols])
            exact = oracle.gemv_i8_exact(m, qx, sx)
            assert np.all(np.abs(yh[t * rows:(t + 1) * rows] - exact) <= np.spacing(np.abs(exact))), t


@pytest.mark.parametrize("act", [0, 1, 2])
def test_reserved_stream_captures_without_allocating(oracle, act):
    # nnh_stream_reserve sizes a fresh stream's scratch ahead of time: the
    # first call on that stream may then be captured (no allocation inside the
    # capture), and replays give the eager bits. nnh_stream_release frees the
    # stream's scratch; the next call on it allocates afresh, same bits.
    import torch
    rows, cols, n_tok = 640, 2048, 24
    say("reserve then capture", act)
    rng = oracle.Rng(0x5E5 + act)
    m = oracle.QMatrix.from_f32(2, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    st = torch.cuda.Stream()
    x = torch.from_numpy(rng.normals(n_tok * cols, 1.0)).cuda()
    y = torch.zeros(n_tok * rows, device="cuda")
    N.stream_reserve(w, act, n_tok, st.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        N.gemv_batch_dev(w, x.data_ptr(), cols, y.data_ptr(), rows, n_tok, act, st.cuda_stream)
    outs = []
    for _ in range(3):
        y.fill_(-1.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy().copy())
    del g
    y.fill_(-1.0)
    N.gemv_batch_dev(w, x.data_ptr(), cols, y.data_ptr(), rows, n_tok, act, st.cuda_stream)
    torch.cuda.synchronize()
    eager = y.cpu().numpy().copy()
    for o in outs:
        assert np.array_equal(bits(o), bits(eager))
    N.stream_release(st.cuda_stream)
    y.fill_(-1.0)
    N.gemv_batch_dev(w, x.data_ptr(), cols, y.data_ptr(), rows, n_tok, act, st.cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(bits(y.cpu().numpy()), bits(eager))
    N.stream_release(st.cuda_stream)
