"""CPU check of the transcribed transfer fixture (tests/golden/
transfer_contract.json from tests/fixtures/transfer_contract.php): every
dtype holds eight complete elements, and the float patterns decode to the
special values the contract exercises (signed zeros, infinities, a NaN with
a payload, the smallest subnormal, one and the largest finite value), so a
mistyped byte fails here before any GPU run."""
import json
import math
import os

import numpy as np

FIX = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "transfer_contract.json")))
NP = {"float16": np.float16, "float32": np.float32, "float64": np.float64, "int8": np.int8,
      "int16": np.int16, "int32": np.int32, "int64": np.int64, "uint8": np.uint8, "uint16": np.uint16,
      "uint32": np.uint32, "uint64": np.uint64, "bool": np.uint8, "bfloat16": np.uint16}


def test_thirteen_dtypes_of_eight_elements():
    assert len(FIX["patterns"]) == 13
    for dt, hx in FIX["patterns"].items():
        raw = bytes.fromhex(hx)
        assert len(raw) == 8 * np.dtype(NP[dt]).itemsize, dt


def test_float_patterns_are_the_special_values():
    for dt in ("float16", "float32", "float64"):
        v = np.frombuffer(bytes.fromhex(FIX["patterns"][dt]), NP[dt]).astype(np.float64)
        fi = np.finfo(NP[dt])
        assert v[0] == 0 and not math.copysign(1, v[0]) < 0, dt
        assert v[1] == 0 and math.copysign(1, v[1]) < 0, dt
        assert v[2] == math.inf and v[3] == -math.inf, dt
        assert math.isnan(v[4]), dt
        assert v[5] == float(fi.smallest_subnormal), dt
        assert v[6] == 1.0 and v[7] == float(fi.max), dt
    bf = np.frombuffer(bytes.fromhex(FIX["patterns"]["bfloat16"]), np.uint16).astype(np.uint32) << 16
    v = bf.view(np.float32).astype(np.float64)
    assert v[0] == 0 and v[2] == math.inf and v[3] == -math.inf and math.isnan(v[4])
    assert v[6] == 1.0 and v[7] == float(np.float32(3.3895314e38))


def test_integer_patterns_cover_extremes():
    for dt in ("int8", "int16", "int32", "int64"):
        v = np.frombuffer(bytes.fromhex(FIX["patterns"][dt]), NP[dt])
        info = np.iinfo(NP[dt])
        assert v[0] == 0 and v[1] == info.min and v[2] == info.max and v[3] == -1, dt
    assert list(np.frombuffer(bytes.fromhex(FIX["patterns"]["bool"]), np.uint8)) == [0, 1, 0, 1, 1, 0, 1, 0]


def test_layout_indices_match_shapes():
    for name, spec in FIX["layouts"].items():
        n = int(np.prod(spec["shape"])) if spec["shape"] else 1
        assert len(spec["indices"]) == n, name
        assert all(0 <= i < 8 for i in spec["indices"]), name
