"""Load-time GGUF decoding on the GPU (kernels/quant.rs:97-291) against the
oracle's restatement, and the decode -> re-encode upload (model/load.rs:182-206)
against the oracle's decoder and encoders (needs an MI355X)."""
import sys

import numpy as np
import pytest

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


TYPES = [0, 1, 30, 2, 3, 6, 7, 8, 12, 13, 14]


def random_blocks(oracle, ggml_type, n, seed, finite=True):
    """n values of random blocks; with `finite`, every fp16 / f32 field holds
    a finite value (random bytes elsewhere)."""
    bytes_, per = oracle.GGML_BLOCKS[ggml_type]
    nb = n // per
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=nb * bytes_, dtype=np.uint8).reshape(nb, bytes_)
    if not finite:
        return b.ravel()
    h = lambda v: np.asarray(v, np.float16).view(np.uint16)
    if ggml_type == 0:
        return rng.normal(0, 1, n).astype(np.float32).view(np.uint8)
    if ggml_type == 1:
        return h(rng.normal(0, 1, n)).view(np.uint8)
    if ggml_type == 30:
        return oracle.f32_array_to_bf16(rng.normal(0, 1, n).astype(np.float32)).view(np.uint8)
    fields = {2: [0], 3: [0, 2], 6: [0], 7: [0, 2], 8: [0], 12: [0, 2], 13: [0, 2], 14: [208]}[ggml_type]
    for off in fields:
        v = h(rng.uniform(-0.05, 0.05, nb)).view(np.uint8).reshape(nb, 2)
        b[:, off:off + 2] = v
    return b.ravel()


def same(a, b):
    """Bit-equal, NaN where NaN (payloads of NaNs made by arithmetic may differ by hardware)."""
    na, nb_ = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb_) and np.array_equal(a[~na].view(np.uint32), b[~nb_].view(np.uint32))


@pytest.mark.parametrize("ggml_type", TYPES)
def test_dequantize_dev_bit_exact(oracle, ggml_type):
    import torch
    for finite in (True, False):
        n = 256 * 333
        blk = random_blocks(oracle, ggml_type, n, 0x6617 + ggml_type, finite)
        say("dequant", ggml_type, finite)
        ok, want = oracle.dequantize_to_f32(ggml_type, blk, n)
        assert ok
        db = torch.from_numpy(blk.copy()).cuda()
        out = torch.full((n,), 9.0, dtype=torch.float32, device="cuda")
        N.dequantize_dev(ggml_type, db.data_ptr(), blk.size, out.data_ptr(), n)
        N.sync()
        got = out.cpu().numpy()
        if finite or ggml_type in (0, 1, 30, 8):
            # every NaN here comes from the input bits: the payload is the reference's too
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)) or same(got, want)
        assert same(got, want)


def test_dequantize_dev_rejects(oracle):
    import torch
    d = torch.zeros(512, dtype=torch.uint8, device="cuda")
    out = torch.full((64,), 9.0, dtype=torch.float32, device="cuda")
    for ty, nbytes, n in [(9, 64, 32), (10, 128, 32), (8, 33, 32), (8, 68, 33), (12, 143, 256)]:
        with pytest.raises(N.InvalidArgument):
            N.dequantize_dev(ty, d.data_ptr(), nbytes, out.data_ptr(), n)
    N.sync()
    assert (out.cpu().numpy() == 9.0).all()


@pytest.mark.parametrize("ggml_type", [1, 2, 7, 8, 12, 13, 14, 30])
@pytest.mark.parametrize("dtype", [1, 2, 3])
def test_upload_gguf_reencodes_like_the_loader(oracle, ggml_type, dtype):
    rows, cols = 96, 1024
    n = rows * cols
    blk = random_blocks(oracle, ggml_type, n, 0x10AD + ggml_type)
    say("gguf", ggml_type, "->", dtype)
    ok, f = oracle.dequantize_to_f32(ggml_type, blk, n)
    assert ok
    w = N.Weight.from_gguf(ggml_type, blk, rows, cols, dtype)
    got = w.download()
    if dtype == 3:
        want = oracle.f32_array_to_bf16(f).view(np.uint8)
    else:
        want = oracle.QMatrix.from_f32(dtype, f.reshape(rows, cols)).buf
    assert np.array_equal(got, want)
    x = np.random.default_rng(3).normal(0, 1, cols).astype(np.float32)
    y = N.model_gemv(w, x)
    assert np.isfinite(y).all()
