"""CPU: pin the oracle's tanh GELU (the fused GELU producer's input transform).

The transform has no reference counterpart: it is the FLUX MLP activation
nn.GELU(approximate="tanh") as a fixed float32 sequence (convrot_oracle.c), so that the HIP
producer can be bit-exact against it.  These tests pin that sequence to the mathematics --
the float64 value of 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) -- and to torch's own
GELU, on every finite bf16 input and on a million float32 samples.  A wrong constant, sign
or branch (e.g. 1 - q for 1 + tanh on the negative side) moves thousands of the exhaustive
bf16 outputs and fails the first test.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc


def _exact(x64: np.ndarray) -> np.ndarray:
    """float64 tanh GELU, 1 + tanh(u) as 2 / (1 + exp(-2u)) (no cancellation)."""
    u = math.sqrt(2.0 / math.pi) * (x64 + 0.044715 * x64 ** 3)
    with np.errstate(over="ignore", invalid="ignore"):
        return 0.5 * x64 * (2.0 / (1.0 + np.exp(-2.0 * u)))


def _bf16_bits(v64: np.ndarray) -> np.ndarray:
    """float64 -> bf16 bit patterns, one round to nearest even (torch's double -> bf16)."""
    return torch.from_numpy(v64).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _all_bf16():
    b = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    return b[np.isfinite(orc.to_f32(b, "bfloat16"))]


def test_every_bf16_input_against_float64():
    """All 65280 finite bf16 inputs: the oracle's bf16 output is the correctly rounded bf16 of
    the float64 GELU everywhere except the far negative tail, where the exact value is below
    2^-124 in magnitude and the producer's exp cutoff (2|u| > 88) returns -0 (5 inputs,
    x in [-10.31, -10.06])."""
    x = _all_bf16()
    got = orc.gelu_tanh(x, "bfloat16")
    ex = _exact(orc.to_f32(x, "bfloat16").astype(np.float64))
    want = _bf16_bits(ex)
    bad = np.nonzero(got != want)[0]
    assert len(bad) <= 8, f"{len(bad)} bf16 outputs differ from the correctly rounded GELU"
    assert (np.abs(ex[bad]) < 2.0 ** -124).all()
    assert (got[bad] == 0x8000).all()  # -0


def test_float32_error_bounds():
    """A million float32 samples ~ N(0, 4^2): within 4 ulps for x >= 0 and 32 ulps on
    [-3, 0); below -3 (where the tail's relative error follows the float32 rounding of the
    tanh argument) within 2e-5 relative while |gelu| >= 1e-30."""
    rng = np.random.default_rng(20260823)
    x = (rng.standard_normal(1_000_000) * 4.0).astype(np.float32)
    got = orc.gelu_tanh(x, "float32").astype(np.float64)
    ex = _exact(x.astype(np.float64))
    keep = np.abs(ex) >= 1e-30
    x, got, ex = x[keep], got[keep], ex[keep]
    ulp = np.abs(np.spacing(ex.astype(np.float32))).astype(np.float64)
    err = np.abs(got - ex) / ulp
    assert err[x >= 0].max() <= 4
    assert err[(x >= -3) & (x < 0)].max() <= 32
    assert (np.abs(got - ex)[x < -3] <= 2e-5 * np.abs(ex[x < -3])).all()


def test_agrees_with_torch_gelu_within_one_ulp():
    """torch.nn.functional.gelu(approximate="tanh") on every finite bf16 input >= -3: the
    bf16 outputs agree on >= 99.9 % of them and never differ by more than one bf16 ulp.
    (Below -3 torch forms 1 + tanh(u) in float32, which cancels: it returns -0 where the
    exact GELU is a small negative number; the float64 test above covers that range.)"""
    x = _all_bf16()
    xf = orc.to_f32(x, "bfloat16")
    x = x[xf >= -3.0]
    got = orc.gelu_tanh(x, "bfloat16")
    t = torch.nn.functional.gelu(torch.from_numpy(orc.to_f32(x, "bfloat16")), approximate="tanh")
    tb = t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    diff = got != tb
    assert diff.mean() <= 1e-3
    g = got[diff].astype(np.int32)
    w = tb[diff].astype(np.int32)
    assert ((g & 0x8000) == (w & 0x8000)).all() and (np.abs(g - w) <= 1).all()


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_closed_forms(dtype):
    """gelu(+-0) keeps the sign of zero; gelu(x) = x once tanh has saturated (x >= 10); the
    negative tail underflows to -0; +inf -> +inf; -inf and NaN -> NaN."""
    vals = np.array([0.0, -0.0, 10.0, 12.5, 100.0, -30.0, -1000.0, np.inf, -np.inf, np.nan], np.float32)
    x = orc.from_f32(vals, dtype)
    y = orc.to_f32(orc.gelu_tanh(x, dtype), dtype)
    xr = orc.to_f32(x, dtype)
    assert y[0] == 0.0 and not np.signbit(y[0])
    assert y[1] == 0.0 and np.signbit(y[1])
    assert np.array_equal(y[2:5], xr[2:5])
    assert (y[5:7] == 0.0).all() and np.signbit(y[5:7]).all()
    assert y[7] == np.inf
    assert np.isnan(y[8]) and np.isnan(y[9])


def test_producer_rows_concatenate_head_and_gelu():
    """gelu_producer_rows = [head | gelu(x)] along features, head untouched."""
    rng = np.random.default_rng(3)
    head = orc.from_f32(rng.normal(size=(3, 32)).astype(np.float32), "bfloat16")
    x = orc.from_f32(rng.normal(size=(3, 48)).astype(np.float32), "bfloat16")
    rows = orc.gelu_producer_rows(head, x, "bfloat16")
    assert rows.shape == (3, 80)
    assert np.array_equal(rows[:, :32], head)
    assert np.array_equal(rows[:, 32:], orc.gelu_tanh(x, "bfloat16"))
    assert np.array_equal(orc.gelu_producer_rows(None, x, "bfloat16"), orc.gelu_tanh(x, "bfloat16"))
