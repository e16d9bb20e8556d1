"""BF16 weights on the GPU against the oracle's restatement of nncpu's BF16
kernels (kernels/mod.rs:337-406, 454-485; scalar.rs:555-628), bit for bit,
through the C-ABI (needs an MI355X)."""
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


def bf16s(oracle, rng, n, lo, hi):
    return oracle.f32_array_to_bf16(rng.vec(n, lo, hi))


# kernels/tests.rs:433-447 shapes (every path: f64 fallback, 4-row, 1-row with
# and without cols % 32), a ragged last workgroup on each chain path, a
# partial last block of 8 steps (cols / C % 8 != 0), wide rows whose x does not
# fit the LDS staging (x read from global memory), and tall matrices.
SHAPES = [(1, 8), (7, 5), (16, 1536), (1536, 1536), (2048, 1536), (6144, 1536), (6, 64), (5, 24), (260, 512),
          (33, 96), (37, 1056), (41, 72), (12, 200), (4100, 2048), (64, 24576), (13, 24576), (20, 24584),
          (16384, 1152)]


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_bf16_gemv_bit_exact(oracle, rows, cols):
    say("bf16", rows, cols)
    rng = oracle.Rng(0xB16E + rows + cols)
    w = bf16s(oracle, rng, rows * cols, -1.0, 1.0)
    x = rng.vec(cols, -1.0, 1.0)
    wt = N.Weight.bf16(w, rows, cols)
    got = N.model_gemv(wt, x)
    assert np.array_equal(bits(got), bits(oracle.gemv_bf16(w, x, rows, cols)))


def test_bf16_batch_equals_single(oracle):
    # kernels/tests.rs:641-691: strided batches, each vector the single-vector bits.
    rng = oracle.Rng(0xBA7C)
    for n_batch in (2, 3, 4, 5, 7, 16):
        for rows, cols in [(64, 256), (512, 2048), (68, 96), (6, 64), (7, 13), (9, 4096)]:
            w = oracle.f32_array_to_bf16(rng.vec(rows * cols, -1.0, 1.0))
            wt = N.Weight.bf16(w, rows, cols)
            xs, ys = cols + 32, rows + 3
            x = rng.vec(n_batch * xs, -1.0, 1.0)
            yb = np.full(n_batch * ys, 7.0, np.float32)
            N.gemv_batch(wt, x, xs, yb, ys, n_batch)
            want = oracle.gemv_bf16(w, x, rows, cols, n_batch, xs, ys)
            for t in range(n_batch):
                assert np.array_equal(bits(yb[t * ys:t * ys + rows]), bits(want[t * ys:t * ys + rows])), \
                    (n_batch, rows, cols, t)
                if t + 1 < n_batch:
                    assert np.all(yb[t * ys + rows:(t + 1) * ys] == 7.0)


def test_bf16_argmax(oracle):
    # kernels/tests.rs:461-498, and the running best's NaN / -inf rules.
    rng = oracle.Rng(0xA12A)
    for rows, cols in [(4, 32), (16, 256), (2048, 256), (256, 1536), (7, 5), (6, 64), (262144, 64)]:
        w = bf16s(oracle, rng, rows * cols, -1.0, 1.0)
        x = rng.vec(cols, -1.0, 1.0)
        wt = N.Weight.bf16(w, rows, cols)
        assert N.model_argmax(wt, x) == oracle.gemv_bf16_argmax(w, x, rows, cols), (rows, cols)
    rows, cols = 512, 256
    w = np.zeros(rows * cols, np.uint16)
    for r in (100, 300, 301):
        w[r * cols] = oracle.f32_to_bf16(1.0)
    wt = N.Weight.bf16(w, rows, cols)
    x = np.zeros(cols, np.float32)
    x[0] = 2.0
    assert N.model_argmax(wt, x) == 100
    x[0] = np.nan
    assert N.model_argmax(wt, x) == 0
    cols = 8
    for rows in (8, 7):
        w = np.zeros(rows * cols, np.uint16)
        w[0] = 0x7FC0
        for r in range(1, rows):
            w[r * cols] = oracle.f32_to_bf16(float(r if r != 5 else 50))
        x = np.ones(cols, np.float32)
        wt = N.Weight.bf16(w, rows, cols)
        assert N.model_argmax(wt, x) == oracle.gemv_bf16_argmax(w, x, rows, cols), rows
    w = np.zeros(64, np.uint16)
    w[::8] = 0xFF80
    wt = N.Weight.bf16(w, 8, 8)
    assert N.model_argmax(wt, np.ones(8, np.float32)) == 0


def test_bf16_device_encoder_and_download(oracle):
    import torch
    rng = oracle.Rng(0xE1F)
    rows, cols = 300, 1000
    v = rng.normals(rows * cols, 0.02)
    v[:5] = [0.0, -0.0, np.inf, -np.inf, np.nan]
    wt = N.Weight.encode_dev(N.BF16, torch.from_numpy(v).cuda().data_ptr(), rows, cols)
    got = wt.download().view(np.uint16)
    assert np.array_equal(got, oracle.f32_array_to_bf16(v))
    x = rng.vec(cols, -1.0, 1.0)
    assert np.array_equal(bits(N.model_gemv(wt, x)), bits(oracle.gemv_bf16(got, x, rows, cols)))


def test_bf16_rejects_int8_activations(oracle):
    wt = N.Weight.bf16(np.zeros(64, np.uint16), 4, 16)
    with pytest.raises(N.InvalidArgument):
        N.model_gemv(wt, np.zeros(16, np.float32), act=N.ACT_I8)
