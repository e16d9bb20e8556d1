"""The C-ABI library, without a GPU: it loads, exports exactly what
include/nncpu_hip.h declares, and its host-side checks work."""
import ctypes as C
import subprocess

import pytest

import nncpu_amd as N
from nncpu_amd import _lib


def test_library_loads_and_exports_every_declared_symbol():
    names = N.declared_functions()
    assert len(names) >= 15
    L = N.lib()
    for name in names:
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True)
    exported = {line.split()[-1] for line in out.stdout.splitlines() if " T nnh_" in line}
    assert exported == set(names)


def test_library_targets_gfx950_only():
    # The offload bundle names its targets in the clear: gfx950 and nothing else.
    import re
    data = open(_lib.LIB_PATH, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-z]+)", data))
    assert targets == {b"gfx950"}


def test_null_arguments_are_rejected_without_a_device():
    L = N.lib()
    assert L.nnh_weight_info(None, None, None, None) == _lib.NNH_E_INVALID
    assert b"null" in L.nnh_last_error()
    h = C.c_void_p()
    assert L.nnh_upload(7, None, 1, 32, C.byref(h)) == _lib.NNH_E_INVALID
    L.nnh_free(None)


def test_act_layout_is_aligned():
    off_s, off_sx, total = N.act_layout(4096, 3)
    assert off_s >= 3 * 4096 and off_s % 256 == 0
    assert off_sx >= off_s + 3 * 128 * 2 and off_sx % 256 == 0
    assert total >= off_sx + 3 * 128 * 16
    with pytest.raises(N.InvalidArgument):
        N.act_layout(100, 1)


def test_init_without_gpu_fails_cleanly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    rc = N.lib().nnh_init(0)
    assert rc in (_lib.NNH_E_DEVICE, _lib.NNH_E_STATE)
    assert N.lib().nnh_last_error()


def test_mx_act_layout_extends_the_int8_layout():
    # The MX buffer is the NNH_ACT_I8 layout followed by xb (BF16, tokens in
    # tiles of 256) and xl[n_tok rounded up to 256][cols/32 rounded up to 8][2] BF16
    # (include/nncpu_hip.h); the int8 kernels read its prefix unchanged.
    for cols, n_tok in [(32, 1), (1152, 3), (4096, 17), (18944, 512), (96, 300)]:
        s8, sx8, b8 = N.act_layout_ex(N.ACT_I8, cols, n_tok)
        assert (s8, sx8, b8) == N.act_layout(cols, n_tok)
        s, sx, b = N.act_layout_ex(N.ACT_MXI8, cols, n_tok)
        assert (s, sx) == (s8, sx8)
        xb = ((n_tok + 255) // 256 * 256) * cols * 2
        nbp8 = (cols // 32 + 7) // 8 * 8
        xl = (((n_tok + 255) // 256 * 256) * nbp8 * 4 + 255) // 256 * 256
        assert b == b8 + xb + xl


def test_act_modes_are_checked_without_a_device():
    L = N.lib()
    sz = C.c_size_t()
    assert L.nnh_act_layout_ex(N.ACT_F32, 64, 1, None, None, C.byref(sz)) == _lib.NNH_E_INVALID
    assert L.nnh_act_layout_ex(7, 64, 1, None, None, C.byref(sz)) == _lib.NNH_E_INVALID
    assert L.nnh_act_layout_ex(N.ACT_MXI8, 100, 1, None, None, C.byref(sz)) == _lib.NNH_E_INVALID
    assert b"multiple of 32" in L.nnh_last_error()


def test_calibration_library_exports_its_header():
    # libnncpu_calib.so (the benchmark's peak calibration) exports exactly
    # what include/nncpu_calib.h declares, for gfx950 only.
    import os
    import re
    root = os.path.dirname(_lib.HEADER)
    text = re.sub(r"/\*.*?\*/", "", open(os.path.join(root, "nncpu_calib.h")).read(), flags=re.S)
    names = set(re.findall(r"^\s*(?:long long|int)\s+(nnc_\w+)\s*\(", text, flags=re.M))
    assert names == {"nnc_read_stream", "nnc_mfma_loop", "nnc_mfma_ops", "nnc_clock_probe"}
    path = os.path.join(os.path.dirname(_lib.LIB_PATH), "libnncpu_calib.so")
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True)
    assert {line.split()[-1] for line in out.stdout.splitlines() if " T nnc_" in line} == names
    L = C.CDLL(path)
    L.nnc_mfma_ops.restype = C.c_longlong
    assert L.nnc_mfma_ops(1, 10, 3) == 2 * 32 * 32 * 32 * 4 * 10 * 3 * 4
    assert L.nnc_read_stream(None, 16, 4, None, None) == 1
    assert set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-z]+)", open(path, "rb").read())) == {b"gfx950"}
