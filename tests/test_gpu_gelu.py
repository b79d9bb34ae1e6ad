"""GPU parity of the fused GELU producer ([head | gelu_tanh(x)] + ConvRot preparation in one
kernel) against the oracle, bit for bit: codes, scales and rotated values, every mode and
dtype, with and without a head segment, single- and multi-wave rows, ragged 1024-feature
blocks, row-strided views read in place; and ConvRotLinear.forward_gelu against the oracle
linear."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import from_dev, to_dev

pytestmark = pytest.mark.gpu


def _api():
    import convrot_mlx_amd as api

    return api


def _inputs(orc, seed, rows, Kh, Kx, dtype):
    rng = np.random.default_rng(seed)
    head = rng.normal(size=(rows, Kh)).astype(np.float32)
    x = (rng.normal(size=(rows, Kx)) * 2.0).astype(np.float32)  # pre-activation, both tails of GELU
    x[:, rng.choice(Kx, size=max(1, Kx // 200), replace=False)] *= 8.0
    return orc.from_f32(head, dtype), orc.from_f32(x, dtype)


def _check(orc, dtype, G, rows_in, q8, s8, qp, sp, rot):
    codes, scales = orc.prepare_codes(rows_in, dtype, G)
    assert np.array_equal(from_dev(s8), scales), f"{int((from_dev(s8) != scales).sum())} row scales differ"
    assert np.array_equal(from_dev(sp), scales)
    bad = int((from_dev(q8) != codes).sum())
    assert bad == 0, f"{bad} of {codes.size} int8 codes differ"
    assert np.array_equal(from_dev(qp), orc.pack_signed_int4(codes))
    want = orc.regular_hadamard(rows_in, dtype, G)
    got = from_dev(rot)
    if dtype == "float32":
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    else:
        assert int((got != want).sum()) == 0


CASES = [  # seed, rows, head features, x features, G
    (1, 7, 0, 64, 64),
    (2, 33, 1024, 1664, 64),     # ragged last 1024-feature block, head ends on a block edge
    (3, 5, 48, 80, 64),          # head ends inside a wave's block
    (4, 64, 3072, 12288, 64),    # the FLUX single-block linear2 input (15 waves per row)
    (5, 9, 0, 12288, 256),
    (6, 3, 16, 65520, 16),       # the longest row
]


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("seed,rows,Kh,Kx,G", CASES)
def test_gelu_prepare(orc, dev, dtype, seed, rows, Kh, Kx, G):
    api = _api()
    head, x = _inputs(orc, seed, rows, Kh, Kx, dtype)
    rows_in = orc.gelu_producer_rows(head if Kh else None, x, dtype)
    xd = to_dev(x, dtype, dev)
    hd = to_dev(head, dtype, dev) if Kh else None
    q8, s8 = api.hip_fused_gelu_prepare(xd, G, head=hd, output="int8")
    qp, sp = api.hip_fused_gelu_prepare(xd, G, head=hd, output="packed")
    rot = api.hip_fused_gelu_prepare(xd, G, head=hd, output="rotate")
    torch.cuda.synchronize()
    _check(orc, dtype, G, rows_in, q8, s8, qp, sp, rot)


def test_gelu_prepare_strided_views(orc, dev):
    """x as a column slice of a wider buffer (the FLUX single block's split of linear1's
    output) and head as a slice of another: read in place, same bits as contiguous inputs."""
    api = _api()
    dtype, rows, Kh, Kx, G = "bfloat16", 37, 3072, 12288, 64
    head, x = _inputs(orc, 11, rows, Kh, Kx, dtype)
    wide = np.zeros((rows, 9216 + Kx), np.uint16)
    wide[:, 9216:] = x
    hwide = np.zeros((rows, Kh + 512), np.uint16)
    hwide[:, 256:256 + Kh] = head
    wd, hd = to_dev(wide, dtype, dev), to_dev(hwide, dtype, dev)
    xv, hv = wd[:, 9216:], hd[:, 256:256 + Kh]
    assert xv.stride(0) == 9216 + Kx and not xv.is_contiguous()
    q8, s8 = api.hip_fused_gelu_prepare(xv, G, head=hv)
    qc, sc = api.hip_fused_gelu_prepare(to_dev(x, dtype, dev), G, head=to_dev(head, dtype, dev))
    torch.cuda.synchronize()
    assert torch.equal(q8, qc) and torch.equal(s8, sc)
    codes, scales = orc.prepare_codes(orc.gelu_producer_rows(head, x, dtype), dtype, G)
    assert np.array_equal(from_dev(q8), codes) and np.array_equal(from_dev(s8), scales)


@pytest.mark.parametrize("backend", ["hip-w4a4", "mpp-w4a4", "hip-w4a16"])
def test_forward_gelu(orc, dev, backend):
    """layer.forward_gelu(mlp, head=attn) on [B, L, *] views, against the oracle linear."""
    api = _api()
    dtype, B, L, Kh, Kx, N, G = "bfloat16", 2, 20, 1024, 1664, 70, 64
    K = Kh + Kx
    rng = np.random.default_rng(31)
    head, x = _inputs(orc, 32, B * L, Kh, Kx, dtype)
    dense_w = orc.from_f32(rng.normal(0, 0.02, size=(N, K)).astype(np.float32), dtype)
    dense_b = rng.normal(size=(N,)).astype(np.float32)
    qw, ws = api.quantize_convrot_weight(to_dev(dense_w, dtype, dev), G)
    layer = api.ConvRotLinear(K, N, group_size=G, backend=backend, device=dev).load_nk_weight(
        qw, ws, torch.from_numpy(dense_b).to(dev))
    out = layer.forward_gelu(to_dev(x, dtype, dev).reshape(B, L, Kx), head=to_dev(head, dtype, dev).reshape(B, L, Kh))
    assert tuple(out.shape) == (B, L, N) and out.dtype == torch.bfloat16
    y = orc.gelu_producer_rows(head, x, dtype)
    if backend.endswith("w4a4"):
        w_codes, wsc = orc.prepare_codes(dense_w, dtype, G)
        a_codes, xs = orc.prepare_codes(y, dtype, G)
        want = orc.w4a4_matmul_codes(a_codes, w_codes, xs, wsc, dense_b, dtype)
        assert np.array_equal(from_dev(out).reshape(-1, N), want)
    else:
        # same kernels as forward() on the explicitly formed input
        ref = layer(to_dev(y, dtype, dev).reshape(B, L, K))
        assert torch.equal(out, ref)


def test_forward_gelu_without_head(orc, dev):
    """The double-block MLP form, linear(gelu(h)), through forward_gelu(h)."""
    api = _api()
    dtype, M, K, N, G = "bfloat16", 24, 1024, 40, 64
    rng = np.random.default_rng(41)
    _, x = _inputs(orc, 42, M, 0, K, dtype)
    dense_w = orc.from_f32(rng.normal(0, 0.02, size=(N, K)).astype(np.float32), dtype)
    dense_b = rng.normal(size=(N,)).astype(np.float32)
    qw, ws = api.quantize_convrot_weight(to_dev(dense_w, dtype, dev), G)
    layer = api.ConvRotLinear(K, N, group_size=G, device=dev).load_nk_weight(qw, ws, torch.from_numpy(dense_b).to(dev))
    out = layer.forward_gelu(to_dev(x, dtype, dev))
    w_codes, wsc = orc.prepare_codes(dense_w, dtype, G)
    a_codes, xs = orc.prepare_codes(orc.gelu_tanh(x, dtype), dtype, G)
    assert np.array_equal(from_dev(out), orc.w4a4_matmul_codes(a_codes, w_codes, xs, wsc, dense_b, dtype))


def test_gelu_argument_errors(dev):
    api = _api()
    x = torch.zeros((6, 256), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="rows"):
        api.hip_fused_gelu_prepare(x, 64, head=torch.zeros((5, 64), dtype=torch.bfloat16, device=dev))
    with pytest.raises(ValueError, match="dtype"):
        api.hip_fused_gelu_prepare(x, 64, head=torch.zeros((6, 64), dtype=torch.float16, device=dev))
    with pytest.raises(ValueError, match="divisible"):
        api.hip_fused_gelu_prepare(x, 64, head=torch.zeros((6, 32), dtype=torch.bfloat16, device=dev))
    with pytest.raises(ValueError, match="output"):
        api.hip_fused_gelu_prepare(x, 64, output="fp8")
