"""CPU: pin the oracle's gated residual (the consumer of the gated-residual GEMM epilogue).

The operation has no reference counterpart: it is a DiT block's `x + gate * linear(...)`
as torch evaluates it eagerly, two elementwise ops that each round to the array dtype.
These tests pin oracle.gated_residual to torch's own CPU evaluation of that expression,
bit for bit, over every output dtype and the gate shapes a DiT uses ([B, 1, N] per image,
one [N] vector, a full [B, L, N] gate), and show that the comparison detects a missing
intermediate rounding (the plausible fused-multiply-add shortcut).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc

DT = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _bits(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.float32:
        return t.numpy().copy()
    return t.view(torch.int16).numpy().view(np.uint16).copy()


def _tensor(bits: np.ndarray, dtype: str) -> torch.Tensor:
    if dtype == "float32":
        return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.float32))
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(DT[dtype])


def _operands(seed, B, L, N, dtype, gate_shape):
    rng = np.random.default_rng(seed)
    lin = orc.from_f32((rng.normal(size=(B * L, N)) * 3.0).astype(np.float32), dtype)
    res = orc.from_f32((rng.normal(size=(B * L, N)) * 10.0).astype(np.float32), dtype)
    gate = orc.from_f32(rng.normal(size=gate_shape).astype(np.float32), dtype) if gate_shape else None
    return lin, res, gate


def _same(a, b):
    if a.dtype == np.float32:
        return np.array_equal(a.view(np.uint32), b.view(np.uint32))
    return np.array_equal(a, b)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("gate_form", ["per_image", "vector", "full", "none"])
def test_matches_torch_eager(dtype, gate_form):
    B, L, N = 3, 40, 96
    gate_shape = {"per_image": (B, 1, N), "vector": (N,), "full": (B, L, N), "none": None}[gate_form]
    lin, res, gate = _operands(7, B, L, N, dtype, gate_shape)
    tl = _tensor(lin, dtype).reshape(B, L, N)
    tr = _tensor(res, dtype).reshape(B, L, N)
    if gate is None:
        want = _bits((tr + tl).reshape(B * L, N))
        got = orc.gated_residual(lin, res, None, 1, dtype)
    else:
        tg = _tensor(gate, dtype)
        want = _bits((tr + tg * tl).reshape(B * L, N))
        rpg = {"per_image": L, "vector": B * L, "full": 1}[gate_form]
        rows = gate.reshape(-1, N)
        got = orc.gated_residual(lin, res, rows, rpg, dtype)
    assert _same(got, want)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_single_rounding_shortcut_is_detected(dtype):
    """Rounding only once, dt(res + g * lin) in float32, differs from torch's two-step
    evaluation on a measurable share of outputs: the eager comparison above would catch an
    oracle (or kernel) that dropped the intermediate rounding."""
    B, L, N = 2, 64, 128
    lin, res, gate = _operands(11, B, L, N, dtype, (B, 1, N))
    l32, r32 = orc.to_f32(lin, dtype), orc.to_f32(res, dtype)
    g32 = orc.to_f32(gate.reshape(B, N), dtype)[np.arange(B * L) // L]
    shortcut = orc.from_f32(r32 + g32 * l32, dtype)
    exact = orc.gated_residual(lin, res, gate.reshape(B, N), L, dtype)
    assert (shortcut != exact).mean() > 1e-3


def test_closed_forms():
    """Gate of ones equals the plain residual add; a zero residual leaves dt(gate * lin);
    a zero gate returns the (non-zero) residual unchanged."""
    dtype, M, N = "bfloat16", 16, 32
    lin, res, _ = _operands(3, 1, M, N, dtype, None)
    ones = orc.from_f32(np.ones((1, N), np.float32), dtype)
    zeros = orc.from_f32(np.zeros((1, N), np.float32), dtype)
    assert np.array_equal(orc.gated_residual(lin, res, ones, M, dtype), orc.gated_residual(lin, res, None, 1, dtype))
    g = orc.from_f32(np.full((1, N), 0.37, np.float32), dtype)
    zres = orc.from_f32(np.zeros((M, N), np.float32), dtype)
    prod = orc.from_f32(orc.to_f32(g, dtype)[0] * orc.to_f32(lin, dtype), dtype)
    got = orc.gated_residual(lin, zres, g, M, dtype)
    assert np.array_equal(orc.to_f32(got, dtype), orc.to_f32(prod, dtype))  # +0 + (-0) -> +0 aside
    nz = res.copy()
    nz[orc.to_f32(nz, dtype) == 0] = orc.from_f32(np.ones(1, np.float32), dtype)[0]
    assert np.array_equal(orc.gated_residual(lin, nz, zeros, M, dtype), nz)
