"""GPU parity of the W4A16 GEMM's split-K plan (convrot_w4a16_gemm_ws with a workspace).

Few weight tiles and a long K (12288 -> 3072 at M <= 32, config 4) split K over workgroups:
each stores a float32 partial, and the last workgroup of each tile group adds the group's
partials in split order and runs the epilogue.  The product is a float32 sum in another
order than the unsplit kernel's, so it is checked against the oracle within the float32
accumulation bound (as every W4A16 test is, test_core.py:285-309's tolerance argument); the
split's own contract is checked exactly: repeated launches give the same bits, the gated
residual is the oracle's composition of the split's own plain output bit for bit, every
arrival counter is back at zero after a launch, and a W4A4 stream-K launch on the same
workspace in between changes nothing.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import from_dev, normal_input, to_dev

pytestmark = pytest.mark.gpu

COUNTERS = slice(20480, 32768)   # the split's arrival counters in the workspace's control block
PARTIALS = slice(32768, 32768 + (4 << 20))


def _nat():
    from convrot_mlx_amd import _native

    return _native


def _workspace(dev):
    nat = _nat()
    return torch.zeros(int(nat.load().convrot_w4a4_workspace_bytes()), dtype=torch.uint8, device=dev)


def _gemm_ws(dev, x, wq, ws, b, M, N, K, work, out_dtype=torch.bfloat16, residual=None, gate=None, rows_per_gate=1):
    nat = _nat()
    out = torch.empty((M, N), dtype=out_dtype, device=dev)
    nat.check(nat.load().convrot_w4a16_gemm_ws(
        nat.ptr(x), nat.DTYPE_BF16, nat.ptr(wq), nat.ptr(ws), nat.ptr(b), M, N, K,
        nat.ptr(residual), nat.ptr(gate), N if gate is not None else 0, rows_per_gate,
        nat.ptr(work), work.numel() if work is not None else 0, nat.ptr(out), nat.dtype_code(out_dtype),
        nat.stream_of(dev)))
    torch.cuda.synchronize()
    return out


def _case(orc, seed, M, K, N):
    rng = np.random.default_rng(seed)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.01, size=(N,)).astype(np.float32)
    b = rng.normal(0, 0.02, size=(N,)).astype(np.float32)
    act = normal_input(seed + 1, (M, K), "bfloat16", orc)
    return w, ws, b, act


def _check_tolerance(orc, got_bits, act, w, ws, b):
    """|got - ref| <= 2^-22 K sum|terms| |ws| + one bf16 ulp of the output (test_gpu_w4a16_layout_module)."""
    K = w.shape[1]
    got = orc.to_f32(got_bits, "bfloat16")
    ref, _, mag = orc.w4a16_matmul_codes(act, "bfloat16", w, ws, b, "float32")
    tol = 2.0 ** -22 * K * mag * np.abs(ws)[None, :] + np.abs(ref) * (2.0 ** -22 + 2.0 ** -8) + 1e-30
    err = np.abs(got - ref)
    assert (err <= tol).all(), f"max excess {np.max(err - tol)} (max err {err.max()})"


# (M, K, N): config 4's 12288 -> 3072 at every token-tile form (direct loads below 6 rows,
# quad loads, two 16-row halves), a k-range of 30 blocks (a second, partial pass of the
# waves), N = 4096 (86 groups padded to 88), a ragged N (63 tiles) with 11 short splits,
# and a ragged K end (13024 = 101 blocks + 96 features) at M = 32 with N = 530
SHAPES = [(1, 12288, 3072), (5, 12288, 3072), (16, 12288, 3072), (17, 12288, 3072), (32, 12288, 3072),
          (8, 15360, 3072), (3, 6144, 4096), (7, 8192, 1000), (32, 13024, 530)]


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_split_k_matches_oracle(orc, dev, tuning, M, K, N):
    tuning.set("w4a16_cfg", "S")  # below 9 rows the automatic plan does not split
    w, ws, b, act = _case(orc, M * 31 + K + N, M, K, N)
    wq = torch.from_numpy(orc.codes_to_cdna4(w)).to(dev)
    wsd, bd = torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev)
    x = to_dev(act, "bfloat16", dev)
    work = _workspace(dev)
    first = _gemm_ws(dev, x, wq, wsd, bd, M, N, K, work)
    # the split ran (its partials are in the workspace) and left every counter at zero
    assert int(work[PARTIALS].count_nonzero()) > 0, "no split-K partial was written"
    assert int(work[COUNTERS].count_nonzero()) == 0, "arrival counters not rearmed"
    _check_tolerance(orc, from_dev(first), act, w, ws, b)
    again = _gemm_ws(dev, x, wq, wsd, bd, M, N, K, work)
    assert torch.equal(first, again), "repeated split-K launches differ"
    # without a workspace: the unsplit plan, within the same bound of the oracle
    plain = _gemm_ws(dev, x, wq, wsd, bd, M, N, K, None)
    _check_tolerance(orc, from_dev(plain), act, w, ws, b)


@pytest.mark.parametrize("M,K,N", [(4, 12288, 3072), (32, 12288, 3072)])
def test_split_k_gated_residual(orc, dev, tuning, M, K, N):
    """The gated residual in the split's epilogue is the oracle composition of the split's own
    plain output, bit for bit (one gate row per 2 token rows)."""
    tuning.set("w4a16_cfg", "S")
    w, ws, b, act = _case(orc, 7 * M + 3, M, K, N)
    wq = torch.from_numpy(orc.codes_to_cdna4(w)).to(dev)
    wsd, bd = torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev)
    x = to_dev(act, "bfloat16", dev)
    rng = np.random.default_rng(M + 99)
    res = orc.from_f32(rng.normal(size=(M, N)).astype(np.float32), "bfloat16")
    gate = orc.from_f32(rng.normal(size=((M + 1) // 2, N)).astype(np.float32), "bfloat16")
    work = _workspace(dev)
    plain = from_dev(_gemm_ws(dev, x, wq, wsd, bd, M, N, K, work))
    fused = from_dev(_gemm_ws(dev, x, wq, wsd, bd, M, N, K, work, residual=to_dev(res, "bfloat16", dev),
                              gate=to_dev(gate, "bfloat16", dev), rows_per_gate=2))
    want = orc.gated_residual(plain, res, gate, 2, "bfloat16")
    assert np.array_equal(fused, want), f"{int((fused != want).sum())} outputs differ"


def test_split_k_shares_the_stream_k_workspace(orc, dev, tuning):
    """A W4A4 stream-K launch on the same workspace between two split-K launches leaves the
    second one's output unchanged (the split's counters lie outside the stream-K words)."""
    nat = _nat()
    M, K, N = 32, 12288, 3072
    w, ws, b, act = _case(orc, 5, M, K, N)
    wq = torch.from_numpy(orc.codes_to_cdna4(w)).to(dev)
    wsd, bd = torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev)
    x = to_dev(act, "bfloat16", dev)
    work = _workspace(dev)
    first = _gemm_ws(dev, x, wq, wsd, bd, M, N, K, work)
    # a stream-K W4A4 product on the same workspace (partial tiles over the split's partials)
    tuning.set("gemm_sk", "1")
    tuning.set("gemm_sk_min", "1")
    rng = np.random.default_rng(6)
    Ma, Ka, Na = 300, 2688, 530
    a = torch.from_numpy(rng.integers(-8, 8, size=(Ma, Ka), dtype=np.int8)).to(dev)
    wa = rng.integers(-8, 8, size=(Na, Ka), dtype=np.int8)
    wqa = torch.from_numpy(orc.codes_to_cdna4(wa)).to(dev)
    xs = torch.rand(Ma, device=dev) + 0.01
    wsa = torch.rand(Na, device=dev) + 0.01
    out4 = torch.empty((Ma, Na), dtype=torch.bfloat16, device=dev)
    nat.check(nat.load().convrot_w4a4_gemm_ws(
        nat.ptr(a), nat.ACT_INT8, nat.ptr(xs), nat.ptr(wqa), nat.ptr(wsa), None, Ma, Na, Ka, None, None, 0, 1,
        nat.ptr(work), work.numel(), nat.ptr(out4), nat.DTYPE_BF16, nat.stream_of(dev)))
    torch.cuda.synchronize()
    second = _gemm_ws(dev, x, wq, wsd, bd, M, N, K, work)
    assert torch.equal(first, second)


def test_split_k_forced_and_refused(orc, dev, tuning):
    """w4a16_cfg "S" forces the split where a plan exists; a forced letter of another kernel keeps
    the workspace untouched; without a workspace "S" falls back to the automatic plan."""
    M, K, N = 8, 12288, 3072
    w, ws, b, act = _case(orc, 11, M, K, N)
    wq = torch.from_numpy(orc.codes_to_cdna4(w)).to(dev)
    wsd, bd = torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev)
    x = to_dev(act, "bfloat16", dev)
    tuning.set("w4a16_cfg", "B")
    work = _workspace(dev)
    unsplit = _gemm_ws(dev, x, wq, wsd, bd, M, N, K, work)
    assert int(work[PARTIALS].count_nonzero()) == 0, "a forced unsplit kernel wrote partials"
    tuning.set("w4a16_cfg", "S")
    split = _gemm_ws(dev, x, wq, wsd, bd, M, N, K, work)
    assert int(work[PARTIALS].count_nonzero()) > 0
    fallback = _gemm_ws(dev, x, wq, wsd, bd, M, N, K, None)
    for got in (unsplit, split, fallback):
        _check_tolerance(orc, from_dev(got), act, w, ws, b)


@pytest.mark.parametrize("M,split", [(8, False), (9, True), (32, True)])
def test_split_k_automatic_rows(orc, dev, M, split):
    """The automatic plan splits 12288 -> 3072 from 9 token rows on (fewer rows: unsplit)."""
    K, N = 12288, 3072
    w, ws, b, act = _case(orc, 13 + M, M, K, N)
    wq = torch.from_numpy(orc.codes_to_cdna4(w)).to(dev)
    work = _workspace(dev)
    got = _gemm_ws(dev, to_dev(act, "bfloat16", dev), wq, torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev),
                   M, N, K, work)
    assert (int(work[PARTIALS].count_nonzero()) > 0) == split
    _check_tolerance(orc, from_dev(got), act, w, ws, b)
