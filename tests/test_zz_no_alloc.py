"""nnh_gemv_batch_dev_noalloc (needs an MI355X): the allocation-free variant
of nnh_gemv_batch_dev, whose scratch is a fixed device array of the library.
Through the C-ABI it must give nnh_gemv_batch_dev's bits, on two calls in a
row with the second smaller, in every activation mode; refuse a weight whose
layouts are not built and a call beyond its scratch maximum."""
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


@pytest.mark.parametrize("dtype,act,rows,cols,n_big,n_small", [
    (2, 0, 1000, 1152, 3, 1),      # f32 path, Q4: block sums in the scratch
    (1, 1, 1536, 6144, 8, 5),      # few-token int8 kernel with K split: partials in the scratch
    (2, 1, 3584, 3584, 40, 17),    # int8 MFMA GEMM, split K
    (2, 2, 512, 3584, 64, 20),     # MX GEMM with its partial tiles
    (1, 2, 18944, 1152, 4, 2),     # MX buffer through the few-token / GEMV kernels
])
def test_noalloc_matches_gemv_batch_dev(oracle, dtype, act, rows, cols, n_big, n_small):
    import torch
    say("noalloc", dtype, act, rows, cols, n_big, n_small)
    rng = oracle.Rng(0x40A1 + rows + act + dtype)
    m = oracle.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    w.prepare(act, n_big).prepare(act, n_small)
    xs, ys = cols + 32, rows + 5
    x = torch.from_numpy(rng.normals(n_big * xs, 1.0)).cuda()
    st = torch.cuda.Stream()
    for n in (n_big, n_small):  # two calls in a row, the second smaller
        want = torch.full((n * ys,), 3.0, device="cuda")
        got = torch.full((n * ys,), 3.0, device="cuda")
        torch.cuda.synchronize()
        N.gemv_batch_dev(w, x.data_ptr(), xs, want.data_ptr(), ys, n, act, st.cuda_stream)
        N.gemv_batch_dev_noalloc(w, x.data_ptr(), xs, got.data_ptr(), ys, n, act, st.cuda_stream)
        torch.cuda.synchronize()
        assert np.array_equal(bits(got.cpu().numpy()), bits(want.cpu().numpy())), n
    # and the first call's result is right, not only equal (f32 path: the oracle's bits)
    if act == 0:
        y = torch.zeros(n_small * ys, device="cuda")
        N.gemv_batch_dev_noalloc(w, x.data_ptr(), xs, y.data_ptr(), ys, n_small, act, st.cuda_stream)
        torch.cuda.synchronize()
        ref = oracle.gemv_batch(m, x.cpu().numpy(), n_small, xs, ys)
        got = y.cpu().numpy()
        for t in range(n_small):
            assert np.array_equal(bits(got[t * ys:t * ys + rows]), bits(ref[t * ys:t * ys + rows]))


def test_noalloc_refusals(oracle):
    import torch
    rng = oracle.Rng(0x40A2)
    rows, cols = 128, 32768
    m = oracle.QMatrix.from_f32(1, rng.normals(rows * cols, 0.02).reshape(rows, cols))
    w = upload(m)
    n = 1024
    x = torch.zeros(n * cols, device="cuda")
    y = torch.full((n * rows,), 5.0, device="cuda")
    torch.cuda.synchronize()
    # Layouts not built for this mode and batch: refused, nothing written.
    with pytest.raises(N.NnhError) as e:
        N.gemv_batch_dev_noalloc(w, x.data_ptr(), cols, y.data_ptr(), rows, 20, N.ACT_MXI8)
    assert "nnh_weight_prepare" in str(e.value)
    w.prepare(N.ACT_MXI8, n)
    # 1024 vectors of 32768 columns: the MX buffer alone exceeds the maximum.
    with pytest.raises(N.InvalidArgument) as e:
        N.gemv_batch_dev_noalloc(w, x.data_ptr(), cols, y.data_ptr(), rows, n, N.ACT_MXI8)
    assert "no-alloc maximum" in str(e.value)
    torch.cuda.synchronize()
    assert torch.all(y == 5.0)
