"""GPU: convrot_w4a4_gemm_noalloc (the W4A4 GEMM with its stream-K workspace in a static
device array, no allocation) against convrot_w4a4_gemm (no workspace: the data-parallel
plans) through the C ABI, bit for bit.

Two calls in a row on each plan, the second with a smaller input (the array keeps the
first call's contents; the stream-K control block must be left ready by every launch):
a forced stream-K plan (the array's partial tiles and flags are used), the automatic plan
of a config-3 shape, and the gated-residual form.  convrot_w4a4_status(NULL) then reports
no bounded-wait give-up.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _operands(rng, M, K, N, dev):
    a = torch.from_numpy(rng.integers(-8, 8, size=(M, K), dtype=np.int8)).to(dev)
    wq = torch.from_numpy(rng.integers(0, 256, size=(((K + 127) // 128) * ((N + 15) // 16) * 1024,),
                                       dtype=np.uint8)).to(dev)
    xs = torch.from_numpy(rng.uniform(0.01, 0.2, size=(M,)).astype(np.float32)).to(dev)
    ws = torch.from_numpy(rng.uniform(0.01, 0.2, size=(N,)).astype(np.float32)).to(dev)
    b = torch.from_numpy(rng.normal(size=(N,)).astype(np.float32)).to(dev)
    return a, wq, xs, ws, b


def _both(nat, dev, ops, M, K, N, dt, residual=None, gate=None, rows_per_gate=1):
    """(convrot_w4a4_gemm[_residual] output, convrot_w4a4_gemm_noalloc output)."""
    lib, p = nat.load(), nat.ptr
    a, wq, xs, ws, b = ops
    ref = torch.full((M, N), float("nan"), dtype=dt, device=dev)
    got = torch.full((M, N), float("nan"), dtype=dt, device=dev)
    common = (p(a), nat.ACT_INT8, p(xs), p(wq), p(ws), p(b), M, N, K)
    if residual is None:
        nat.check(lib.convrot_w4a4_gemm(*common, p(ref), nat.dtype_code(dt), nat.stream_of(dev)))
        nat.check(lib.convrot_w4a4_gemm_noalloc(*common, None, None, 0, 1, p(got), nat.dtype_code(dt),
                                                nat.stream_of(dev)))
    else:
        stride = N if gate is not None else 0
        nat.check(lib.convrot_w4a4_gemm_residual(*common, p(residual), p(gate), stride, rows_per_gate, p(ref),
                                                 nat.dtype_code(dt), nat.stream_of(dev)))
        nat.check(lib.convrot_w4a4_gemm_noalloc(*common, p(residual), p(gate), stride, rows_per_gate, p(got),
                                                nat.dtype_code(dt), nat.stream_of(dev)))
    torch.cuda.synchronize()
    return ref, got


def _exact(ref, got, label):
    r = ref.view(torch.int16 if ref.element_size() == 2 else torch.int32)
    g = got.view(torch.int16 if got.element_size() == 2 else torch.int32)
    bad = int((r != g).sum())
    assert bad == 0, f"{label}: {bad} of {ref.numel()} outputs differ"
    assert not torch.isnan(got.float()).any(), f"{label}: NaN in the output"


@pytest.mark.parametrize("tile", ["256x256w2x2", "128x256w2x4"])
def test_noalloc_stream_k_matches(dev, tuning, tile):
    """Forced stream-K (one-k-block pieces): the partials and flags live in the static
    array.  Call 1 at 600x2688->600, call 2 at 300x1408->264."""
    from convrot_mlx_amd import _native as nat

    tuning.set("gemm_tile", tile)
    tuning.set("gemm_sk", "1")
    tuning.set("gemm_sk_min", "1")
    rng = np.random.default_rng(91)
    for call, (M, K, N) in enumerate([(600, 2688, 600), (300, 1408, 264)]):
        assert nat.load().convrot_w4a4_gemm_noalloc  # exported
        ref, got = _both(nat, dev, _operands(rng, M, K, N, dev), M, K, N, torch.float32)
        _exact(ref, got, f"tile {tile} call {call} ({M}x{K}->{N})")
    nat.check(nat.load().convrot_w4a4_status(None, nat.stream_of(dev)))


def test_noalloc_automatic_plan_matches(dev):
    """The automatic plan: a config-3 shape (4608x3072->3072), then a smaller one that
    takes a stream-K plan of its own choosing or a data-parallel one (1024x12288->3072)."""
    from convrot_mlx_amd import _native as nat

    rng = np.random.default_rng(92)
    for call, (M, K, N) in enumerate([(4608, 3072, 3072), (1024, 12288, 3072)]):
        ref, got = _both(nat, dev, _operands(rng, M, K, N, dev), M, K, N, torch.bfloat16)
        _exact(ref, got, f"call {call} ({M}x{K}->{N})")
    nat.check(nat.load().convrot_w4a4_status(None, nat.stream_of(dev)))


def test_noalloc_gated_residual_matches(dev, tuning):
    """out = residual + gate * linear, gates per 100 rows, forced stream-K; then a smaller
    plain call."""
    from convrot_mlx_amd import _native as nat

    tuning.set("gemm_tile", "256x256w2x2")
    tuning.set("gemm_sk", "1")
    tuning.set("gemm_sk_min", "2")
    rng = np.random.default_rng(93)
    M, K, N = 700, 1536, 520
    res = torch.from_numpy(rng.normal(size=(M, N)).astype(np.float32)).to(dev).to(torch.bfloat16)
    gate = torch.from_numpy(rng.normal(size=(M // 100, N)).astype(np.float32)).to(dev).to(torch.bfloat16)
    ref, got = _both(nat, dev, _operands(rng, M, K, N, dev), M, K, N, torch.bfloat16, res, gate, 100)
    _exact(ref, got, "gated residual")
    M, K, N = 257, 640, 130
    ref, got = _both(nat, dev, _operands(rng, M, K, N, dev), M, K, N, torch.bfloat16)
    _exact(ref, got, "smaller plain call")
    nat.check(nat.load().convrot_w4a4_status(None, nat.stream_of(dev)))
