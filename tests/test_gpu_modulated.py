"""GPU parity of the fused modulated producer (LayerNorm + adaLN modulation + ConvRot
preparation in one kernel) against the oracle, bit for bit: codes, scales and rotated
values, every mode and dtype, one to many modulation vectors, single- and multi-wave rows,
ragged 1024-feature blocks; and ConvRotLinear.forward_modulated against the oracle linear."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import from_dev, to_dev

pytestmark = pytest.mark.gpu


def _api():
    import convrot_mlx_amd as api

    return api


def _inputs(orc, seed, rows, K, vectors, dtype, loc=0.0, std=1.0):
    rng = np.random.default_rng(seed)
    x = rng.normal(loc, std, size=(rows, K)).astype(np.float32)
    x[:, rng.choice(K, size=max(1, K // 200), replace=False)] *= 20.0  # outlier channels
    sh = rng.normal(size=(vectors, K)).astype(np.float32)
    sc = (0.3 * rng.normal(size=(vectors, K))).astype(np.float32)
    return orc.from_f32(x, dtype), orc.from_f32(sh, dtype), orc.from_f32(sc, dtype)


CASES = [  # seed, rows, K, G, vectors
    (1, 7, 64, 64, 7),
    (2, 33, 2688, 64, 11),     # ragged last 1024-feature block
    (3, 64, 3072, 64, 1),
    (4, 6, 12288, 256, 2),     # 12 waves per row
    (5, 130, 256, 4, 65),
    (6, 3, 65536, 1024, 3),    # the largest row
]


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("seed,rows,K,G,vectors", CASES)
def test_modulated_prepare(orc, dev, dtype, seed, rows, K, G, vectors):
    api = _api()
    x, sh, sc = _inputs(orc, seed, rows, K, vectors, dtype)
    y = orc.modulate(x, dtype, sh, sc, rows // vectors)
    codes, scales = orc.prepare_codes(y, dtype, G)
    xd, shd, scd = to_dev(x, dtype, dev), to_dev(sh, dtype, dev), to_dev(sc, dtype, dev)
    q8, s8 = api.hip_fused_modulated_prepare(xd, shd, scd, G, output="int8")
    qp, sp = api.hip_fused_modulated_prepare(xd, shd, scd, G, output="packed")
    rot = api.hip_fused_modulated_prepare(xd, shd, scd, G, output="rotate")
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(s8), scales), f"{int((from_dev(s8) != scales).sum())} row scales differ"
    assert np.array_equal(from_dev(sp), scales)
    bad = int((from_dev(q8) != codes).sum())
    assert bad == 0, f"{bad} of {codes.size} int8 codes differ"
    assert np.array_equal(from_dev(qp), orc.pack_signed_int4(codes))
    want = orc.regular_hadamard(y, dtype, G)
    got = from_dev(rot)
    if dtype == "float32":
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    else:
        assert int((got != want).sum()) == 0


def test_modulated_shifted_rows(orc, dev):
    """Rows far from zero mean (x - mean cancels) and a constant row (variance 0)."""
    api = _api()
    dtype, K, G = "bfloat16", 3072, 64
    x, sh, sc = _inputs(orc, 9, 4, K, 1, dtype, loc=-2.0, std=0.1)
    x[3] = orc.from_f32(np.full(K, 1.5, np.float32), dtype)
    y = orc.modulate(x, dtype, sh, sc, 4)
    codes, scales = orc.prepare_codes(y, dtype, G)
    q, s = api.hip_fused_modulated_prepare(to_dev(x, dtype, dev), to_dev(sh, dtype, dev), to_dev(sc, dtype, dev), G)
    assert np.array_equal(from_dev(s), scales)
    assert np.array_equal(from_dev(q), codes)


@pytest.mark.parametrize("backend", ["hip-w4a4", "mpp-w4a4", "hip-w4a16"])
def test_forward_modulated(orc, dev, backend):
    """layer.forward_modulated(x, shift, scale) on x [B, L, K] with shift/scale [B, 1, K]."""
    api = _api()
    dtype, B, L, K, N, G = "bfloat16", 3, 20, 2688, 70, 64
    rng = np.random.default_rng(21)
    x, sh, sc = _inputs(orc, 22, B * L, K, B, dtype)
    dense_w = orc.from_f32(rng.normal(0, 0.02, size=(N, K)).astype(np.float32), dtype)
    dense_b = rng.normal(size=(N,)).astype(np.float32)
    qw, ws = api.quantize_convrot_weight(to_dev(dense_w, dtype, dev), G)
    layer = api.ConvRotLinear(K, N, group_size=G, backend=backend, device=dev).load_nk_weight(
        qw, ws, torch.from_numpy(dense_b).to(dev))
    xd = to_dev(x, dtype, dev).reshape(B, L, K)
    out = layer.forward_modulated(xd, to_dev(sh, dtype, dev).reshape(B, 1, K), to_dev(sc, dtype, dev).reshape(B, 1, K))
    assert tuple(out.shape) == (B, L, N) and out.dtype == torch.bfloat16
    y = orc.modulate(x, dtype, sh, sc, L)
    if backend.endswith("w4a4"):
        w_codes, wsc = orc.prepare_codes(dense_w, dtype, G)
        a_codes, xs = orc.prepare_codes(y, dtype, G)
        want = orc.w4a4_matmul_codes(a_codes, w_codes, xs, wsc, dense_b, dtype)
        assert np.array_equal(from_dev(out).reshape(-1, N), want)
    else:
        # same kernels as forward() on the explicitly modulated input
        ref = layer(to_dev(y, dtype, dev).reshape(B, L, K))
        assert torch.equal(out, ref)


def test_modulated_argument_errors(dev):
    api = _api()
    x = torch.zeros((6, 256), dtype=torch.bfloat16, device=dev)
    v = torch.zeros((4, 256), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="split evenly"):
        api.hip_fused_modulated_prepare(x, v, v, 64)
    with pytest.raises(ValueError, match="features"):
        api.hip_fused_modulated_prepare(x, v[:, :128], v[:, :128], 64)
    with pytest.raises(ValueError, match="output"):
        api.hip_fused_modulated_prepare(x, v[:2], v[:2], 64, output="fp8")
