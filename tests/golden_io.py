"""Reading the golden vectors under tests/golden/ (raw little-endian .bin + manifest.json)."""
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DTYPES = {"f32": np.float32, "i8": np.int8, "u8": np.uint8, "u16": np.uint16, "i32": np.int32}


def cases():
    path = os.path.join(GOLDEN, "manifest.json")
    return json.load(open(path))["cases"] if os.path.exists(path) else []


def array(case, key):
    spec = case["arrays"][key]
    a = np.fromfile(os.path.join(GOLDEN, spec["file"]), dtype=np.dtype(DTYPES[spec["dtype"]]).newbyteorder("<"))
    return a.astype(DTYPES[spec["dtype"]])


def load_case(oracle, case):
    """(QMatrix, x, y, extra) for a manifest entry."""
    rows, cols, dtype = case["rows"], case["cols"], case["dtype"]
    if dtype == 1:
        parts = (array(case, "qs").view(np.int8), array(case, "scales"))
    else:
        parts = (array(case, "qs"), array(case, "scales"), array(case, "biases"))
    m = oracle.QMatrix(dtype, rows, cols, parts)
    extra = {k: array(case, k) for k in case["arrays"] if k not in ("qs", "scales", "biases", "x", "y")}
    if "P" in extra:
        extra["P"] = extra["P"].reshape(rows, cols // 32)
    return m, array(case, "x"), array(case, "y"), extra
