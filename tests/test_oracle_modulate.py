"""Pinning the oracle's modulated-producer transform (`oracle.modulate`) on the CPU.

The transform has no reference counterpart: it is the adaLN pattern
`(1 + scale) * layer_norm(x) + shift` of a diffusion transformer, evaluated as
an eager bf16/f16 graph.  It is pinned against torch's own CPU operators (an
independent implementation of LayerNorm and of per-op rounded bf16/f16
arithmetic) and against closed forms.  Its LayerNorm moments come from float64
sums, torch's from a float32 Welford pass, so a normalized value may land one
unit in the last place apart when it sits next to a rounding boundary; every
such difference must be exactly that, and rare.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as orc

TDT = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _t(a: np.ndarray, dtype: str) -> torch.Tensor:
    if dtype == "float32":
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(TDT[dtype])


def _np(t: torch.Tensor, dtype: str) -> np.ndarray:
    return t.numpy() if dtype == "float32" else t.view(torch.int16).numpy().view(np.uint16)


def _inputs(seed, rows, K, vectors, dtype, loc=0.0, std=1.0):
    rng = np.random.default_rng(seed)
    x = orc.from_f32((rng.normal(loc, std, size=(rows, K))).astype(np.float32), dtype)
    sh = orc.from_f32(rng.normal(size=(vectors, K)).astype(np.float32), dtype)
    sc = orc.from_f32((0.3 * rng.normal(size=(vectors, K))).astype(np.float32), dtype)
    return x, sh, sc


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("seed,rows,K,vectors,loc,std", [(1, 48, 3072, 3, 0.0, 1.0), (2, 20, 256, 20, 0.5, 3.0),
                                                          (3, 9, 12288, 1, -2.0, 0.1)])
def test_modulate_matches_torch(dtype, seed, rows, K, vectors, loc, std):
    x, sh, sc = _inputs(seed, rows, K, vectors, dtype, loc, std)
    per = rows // vectors
    ln = orc.modulate(x, dtype, np.zeros_like(sh), np.zeros_like(sc), per)  # shift 0, scale 0: rb(rb(1*ln)+0) = ln
    a = orc.to_f32(ln, dtype)
    # torch's LayerNorm in float64, rounded once to the dtype: the oracle's float32 evaluation
    # of (x - mean) * rstd may sit one unit in the last place away only next to a rounding
    # boundary.  torch's own dtype LayerNorm (float32 Welford moments) is less accurate and
    # is held to the same one-unit bound.  (The fraction that differs depends on how the
    # bf16 inputs cluster: rows of mean -2, std 0.1 put 0.5 % of values on one boundary.)
    exact = F.layer_norm(_t(x, dtype).double(), (K,), eps=1e-6).to(TDT[dtype]).float().numpy()
    native = F.layer_norm(_t(x, dtype), (K,), eps=1e-6).float().numpy()
    # (float32 rows round twice, (x - mean) then * rstd, so they get a few units instead.)
    mant = {"bfloat16": 8, "float16": 11, "float32": 24}[dtype]
    units = 4.0 if dtype == "float32" else 1.0
    for b, max_frac in ((exact, 2e-2), (native, 5e-2)):
        diff = np.abs(a - b)
        if dtype != "float32":
            assert (diff > 0).mean() < max_frac, f"{int((diff > 0).sum())} of {diff.size} normalized values differ"
        # (float32: plus an absolute term of the size of the mean's own float32 rounding,
        # carried through rstd, which dominates where x - mean cancels)
        if dtype == "float32":
            xf = orc.to_f32(x, dtype).astype(np.float64)
            c = (np.abs(xf.mean(axis=1)) / xf.std(axis=1) + 1.0)[:, None]
            tol = units * (np.abs(b) + c) * 2.0 ** (1 - mant)
        else:
            tol = units * np.maximum(np.abs(b), 2.0**-14) * 2.0 ** (1 - mant)
        assert (diff <= tol).all(), "a normalized value differs by more than the allowed units in the last place"
    # the modulation arithmetic itself, on the oracle's normalized rows, is exact against torch
    y = orc.modulate(x, dtype, sh, sc, per)
    ln_tt = _t(ln, dtype)
    sh_t = _t(sh, dtype).repeat_interleave(per, 0)
    sc_t = _t(sc, dtype).repeat_interleave(per, 0)
    want = (1 + sc_t) * ln_tt + sh_t
    if dtype == "float32":
        assert np.array_equal(y.view(np.uint32), want.numpy().view(np.uint32))
    else:
        assert np.array_equal(y, _np(want, dtype))


def test_modulate_closed_forms():
    """Constant rows normalize to 0, so y = rb(rb(rb(1+scale)*0) + shift) = shift; rows of +-a
    (a^2 >> eps) normalize to +-1 exactly in bf16, so y = rb(rb(1+scale)*(+-1) + shift)."""
    K, dtype = 1024, "bfloat16"
    rng = np.random.default_rng(7)
    sh = orc.from_f32(rng.normal(size=(2, K)).astype(np.float32), dtype)
    sc = orc.from_f32(rng.normal(size=(2, K)).astype(np.float32), dtype)
    const = orc.from_f32(np.full((2, K), 3.25, np.float32), dtype)
    assert np.array_equal(orc.modulate(const, dtype, sh, sc, 1), sh)
    sign = np.where(np.arange(K) % 2 == 0, 1.0, -1.0).astype(np.float32)
    alt = orc.from_f32(np.stack([2.0 * sign, 0.75 * sign]), dtype)
    y = orc.to_f32(orc.modulate(alt, dtype, sh, sc, 1), dtype)
    one_plus = orc.to_f32(orc.from_f32(1.0 + orc.to_f32(sc, dtype), dtype), dtype)
    want = orc.to_f32(orc.from_f32(orc.to_f32(orc.from_f32(one_plus * sign, dtype), dtype)
                                   + orc.to_f32(sh, dtype), dtype), dtype)
    assert np.array_equal(y, want)


def test_modulate_vector_rows():
    """Row r uses vector r // rows_per_vector: permuting the vectors permutes the row blocks."""
    dtype = "bfloat16"
    x, sh, sc = _inputs(11, 12, 256, 4, dtype)
    y = orc.modulate(x, dtype, sh, sc, 3)
    perm = [2, 0, 3, 1]
    xp = np.concatenate([x[3 * p: 3 * p + 3] for p in perm])
    yp = orc.modulate(xp, dtype, sh[perm].copy(), sc[perm].copy(), 3)
    assert np.array_equal(yp, np.concatenate([y[3 * p: 3 * p + 3] for p in perm]))
