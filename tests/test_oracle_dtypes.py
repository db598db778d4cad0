"""Pins the oracle's fp16/bf16 converters (data_types.c:46-131).

Checks: the reference's own conversion vectors (matmul_low_precision.phpt:
28-46) and bulk agreement with independent RNE implementations (numpy's
float16 cast, torch's bfloat16 cast), which a wrong rounding rule, a wrong
rebias or a lost subnormal path would fail.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle_lib as O

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_expectations.json")))


def _value(v):
    return float(v) if not isinstance(v, str) else float(v)


@pytest.mark.parametrize("case", GOLDEN["conversions"], ids=lambda c: c["id"])
def test_reference_conversion_vectors(case):
    x = np.array([case["input"]], np.float32)
    if case["dtype"] == "bfloat16":
        got = float(O.bf16_to_f32(O.f32_to_bf16(x))[0])
    else:
        got = float(O.f16_to_f32(O.f32_to_f16(x))[0])
    if case.get("expected_positive"):
        assert got > 0.0
        return
    exp = _value(case["expected"])
    if math.isinf(exp):
        assert math.isinf(got) and got > 0
    else:
        assert got == exp


def _random_float_bits(n, seed):
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)
    return bits.view(np.float32)


def test_f16_matches_numpy_rne_bulk():
    x = _random_float_bits(2_000_000, 1)
    # also concentrate around the fp16 range, subnormals and ties
    y = (np.random.default_rng(2).standard_normal(1_000_000) *
         np.exp2(np.random.default_rng(3).integers(-26, 17, 1_000_000))).astype(np.float32)
    ties = (np.arange(1, 200_000, dtype=np.float32) * np.float32(2.0 ** -11) +
            np.float32(2.0 ** -12)).astype(np.float32)
    for arr in (x, y, ties):
        ours = O.f32_to_f16(arr)
        ref = arr.astype(np.float16).view(np.uint16)
        finite = ~np.isnan(arr)
        assert np.array_equal(ours[finite], ref[finite])
        # NaN stays NaN (payload kept non-zero)
        nan_bits = ours[~finite]
        assert np.all((nan_bits & 0x7c00) == 0x7c00) and np.all((nan_bits & 0x3ff) != 0)


def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = O.f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    same = (ours.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(ours) & np.isnan(ref))
    assert same.all()


def test_bf16_matches_torch_rne_bulk():
    torch = pytest.importorskip("torch")
    x = _random_float_bits(2_000_000, 4)
    ours = O.f32_to_bf16(x)
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    finite = ~np.isnan(x)
    assert np.array_equal(ours[finite], ref[finite])
    assert np.all(np.isnan(O.bf16_to_f32(ours[~finite])))


def test_bf16_round_trip_exact_for_representable():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = O.bf16_to_f32(bits)
    back = O.f32_to_bf16(vals)
    ok = ~np.isnan(vals)
    assert np.array_equal(back[ok], bits[ok])
