"""Writes the golden vectors in tests/golden/ from seeded inputs.

Inputs: W = 0.02*N(0,1) or U(-1,1), x = N(0,1), from the reference's
xorshift64* test generator (crates/nncpu/src/kernels/tests.rs:9-50, restated
in oracle/oracle.cpp), re-encoded with the restated nncpu encoder
(kernels/quant.rs:31-95). Expected outputs come from the oracle, which
tests/test_oracle.py pins against the reference's known answers first.
Shapes follow SURVEY's fixture list: the reference's test shapes, strided
batches (x_stride = K+32, y_stride = N+3), K = 1152 for the Q4 bias tail.

    python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle as O  # noqa: E402


def save(name, key, arr, tag, arrays):
    fname = f"{name}.{key}.bin"
    arr = np.ascontiguousarray(arr)
    arr.astype(arr.dtype.newbyteorder("<")).tofile(os.path.join(HERE, fname))
    arrays[key] = {"file": fname, "dtype": tag, "n": int(arr.size)}


def weight_arrays(name, m, arrays):
    if m.dtype == 1:
        save(name, "qs", m.parts[0], "i8", arrays)
        save(name, "scales", m.parts[1], "u16", arrays)
    else:
        save(name, "qs", m.parts[0], "u8", arrays)
        save(name, "scales", m.parts[1], "u16", arrays)
        save(name, "biases", m.parts[2], "u16", arrays)


def main():
    for f in os.listdir(HERE):
        if f.endswith(".bin"):
            os.remove(os.path.join(HERE, f))
    cases = []
    seed = 0x60D0
    f32_shapes = [(8, 64, 1), (64, 128, 1), (300, 640, 1), (68, 96, 3), (6, 64, 7), (16, 1152, 1),
                  (16, 1152, 4), (8, 6912, 2), (33, 288, 5)]
    for dtype in (1, 2):
        for rows, cols, n_tok in f32_shapes:
            seed += 1
            rng = O.Rng(seed)
            w = rng.normals(rows * cols, 0.02).reshape(rows, cols)
            m = O.QMatrix.from_f32(dtype, w)
            xs, ys = (cols + 32, rows + 3) if n_tok > 1 else (cols, rows)
            x = rng.normals((n_tok - 1) * xs + cols, 1.0)
            y = O.gemv_batch(m, x, n_tok, xs, ys)
            name = f"f32_{'q8' if dtype == 1 else 'q4'}_{rows}x{cols}_m{n_tok}"
            arrays = {}
            weight_arrays(name, m, arrays)
            save(name, "x", x, "f32", arrays)
            save(name, "y", y, "f32", arrays)
            cases.append(dict(name=name, kind="gemv_f32", dtype=dtype, rows=rows, cols=cols, n_tok=n_tok,
                              x_stride=xs, y_stride=ys, seed=seed, arrays=arrays))
    for dtype in (1, 2):
        for rows, cols in [(32, 256), (16, 1152), (12, 4096)]:
            seed += 1
            rng = O.Rng(seed)
            m = O.QMatrix.from_f32(dtype, rng.normals(rows * cols, 0.02).reshape(rows, cols))
            x = rng.normals(cols, 1.0)
            qx, sx = O.quantize_act(x)
            P = O.block_dots(m, qx)
            y = O.gemv_i8_exact(m, qx, sx)
            name = f"i8_{'q8' if dtype == 1 else 'q4'}_{rows}x{cols}"
            arrays = {}
            weight_arrays(name, m, arrays)
            save(name, "x", x, "f32", arrays)
            save(name, "qx", qx, "i8", arrays)
            save(name, "sx", sx, "u16", arrays)
            save(name, "P", P, "i32", arrays)
            save(name, "y", y, "f32", arrays)
            cases.append(dict(name=name, kind="gemv_i8", dtype=dtype, rows=rows, cols=cols, n_tok=1, seed=seed,
                              arrays=arrays))
    json.dump({"generator": "tests/golden/make_golden.py", "cases": cases},
              open(os.path.join(HERE, "manifest.json"), "w"), indent=1)
    total = sum(os.path.getsize(os.path.join(HERE, f)) for f in os.listdir(HERE))
    print(f"{len(cases)} cases, {total} bytes")


if __name__ == "__main__":
    main()
