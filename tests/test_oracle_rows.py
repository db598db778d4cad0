"""Pins the oracle's softmax (cuda_array_ce.c:1942-2001) and layerNorm
(cuda_array_ce.c:2215-2339) restatements.

Checks: the reference's printed vectors, a float64 numpy evaluation within
a few float32 ulps, rows summing to one, and mean-0 / variance-1 outputs.
A missing max shift overflows on the 1000-logit vector; eps outside the
sqrt or a biased/unbiased mix-up moves the -0.99998 vector.
"""
import json
import os

import numpy as np
import pytest

import oracle_lib as O

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_expectations.json")))


def _rows_softmax(x, axis):
    x = np.moveaxis(x, axis, -1)
    out = O.softmax_lastaxis(np.ascontiguousarray(x))
    return np.moveaxis(out, -1, axis)


@pytest.mark.parametrize("case", GOLDEN["softmax"], ids=lambda c: c["id"])
def test_softmax_reference_vectors(case):
    src = np.array(case["data"], np.float64).reshape(case["shape"])
    x = src.astype(np.float64 if case["dtype"] != "float32" else np.float32)
    out = _rows_softmax(x, case["axis"])
    d = case["decimals"]
    if "expected_index" in case:
        assert out.dtype == np.float64
        assert round(float(out.ravel()[case["expected_index"]]), d) == case["expected_value"]
    else:
        assert [round(float(v), d) for v in out.ravel()] == case["expected"]


def test_softmax_matches_float64_and_sums_to_one():
    # float32 rounding of x - max is amplified by exp (relative error ~
    # |x - max| * 2^-24) and the sequential sum adds ~sqrt(n) ulps.
    rng = np.random.default_rng(21)
    for scale, rtol in ((1.0, 1e-5), (4.0, 3e-5)):
        x = (rng.standard_normal((32, 4096)) * scale).astype(np.float32)
        out = O.softmax_lastaxis(x)
        xd = x.astype(np.float64)
        e = np.exp(xd - xd.max(axis=1, keepdims=True))
        ref = e / e.sum(axis=1, keepdims=True)
        assert np.allclose(out, ref, rtol=rtol, atol=1e-12)
        assert np.allclose(out.astype(np.float64).sum(axis=1), 1.0, atol=1e-5)


@pytest.mark.parametrize("case", GOLDEN["layernorm"], ids=lambda c: c["id"])
def test_layernorm_reference_vectors(case):
    if "data" in case:
        x = np.array(case["data"], np.float32).reshape(case["shape"])
    else:
        x = np.full(case["shape"], case["fill"], np.float32)
    axis = case["axes"][0]
    xt = np.ascontiguousarray(np.moveaxis(x, axis, -1))
    g = np.array(case["scale"], np.float32) if "scale" in case else None
    b = np.array(case["bias"], np.float32) if "bias" in case else None
    out = np.moveaxis(O.layernorm_lastaxis(xt, case["eps"], g, b), -1, axis)
    if "expected_first_row" in case:
        assert [round(float(v), case["decimals"]) for v in out[0]] == case["expected_first_row"]
    elif "expected_at" in case:
        idx, val = case["expected_at"]
        assert round(float(out[tuple(idx)]), case["decimals"]) == val
    else:
        assert out.ravel().tolist() == case["expected"]


def test_layernorm_matches_float64():
    rng = np.random.default_rng(22)
    x = (rng.standard_normal((16, 4096)) * 2 + 0.5).astype(np.float32)
    g = rng.standard_normal(4096).astype(np.float32)
    b = rng.standard_normal(4096).astype(np.float32)
    out = O.layernorm_lastaxis(x, 1e-5, g, b)
    xd = x.astype(np.float64)
    mu = xd.mean(axis=1, keepdims=True)
    var = ((xd - mu) ** 2).mean(axis=1, keepdims=True)
    ref = (xd - mu) / np.sqrt(var + 1e-5) * g + b
    assert np.allclose(out, ref, rtol=1e-4, atol=1e-5)
    plain = O.layernorm_lastaxis(x, 1e-5).astype(np.float64)
    assert np.allclose(plain.mean(axis=1), 0.0, atol=1e-5)
    assert np.allclose(plain.var(axis=1), 1.0, atol=1e-3)
