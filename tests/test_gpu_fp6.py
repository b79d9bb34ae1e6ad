"""GPU parity of the FP6 operand path: the CDNA4 -> FP6 weight conversion, the preparation
kernel's FP6 output and the FP6-operand W4A4 GEMM, each bit for bit against the CPU oracle
(oracle.codes_to_fp6 for the layouts, w4a4_matmul_codes_large for the products), and the
complete FP6 path against the INT8 path.

The FP6 layout and encoding (a code v as the e2m3 value v/8) are this build's own (no reference counterpart); the codes
they carry are the reference's A4 / W4 codes (core.py:149-167, 514-527), and the products
follow reference_w4a4_matmul (core.py:1155-1171) as the INT8 kernels do.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import from_dev, normal_input, outlier_input, to_dev

pytestmark = pytest.mark.gpu


def _nat():
    from convrot_mlx_amd import _native as nat

    return nat


def _u8(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _weight_fp6(nat, wq_dev, N, K, dev):
    out = torch.zeros(int(nat.load().convrot_fp6_bytes(N, K)), dtype=torch.uint8, device=dev)
    nat.check(nat.load().convrot_weight_fp6(nat.ptr(wq_dev), nat.ptr(out), N, K, nat.stream_of(dev)))
    torch.cuda.synchronize()
    return out


def _prep_fp6(nat, xd, G, mode, dev):
    rows, K = xd.shape
    out = torch.zeros(int(nat.load().convrot_fp6_bytes(rows, K)), dtype=torch.uint8, device=dev)
    scales = torch.empty(rows, dtype=torch.float32, device=dev)
    nat.check(nat.load().convrot_prepare(nat.ptr(xd), nat.dtype_code(xd.dtype), rows, K, G, mode, nat.ptr(out),
                                         nat.ptr(scales), nat.stream_of(dev)))
    torch.cuda.synchronize()
    return out, scales


def _gemm_fp6(nat, a6, xs, w6, ws, b, M, N, K, dtype, dev):
    out = torch.empty((M, N), dtype=dtype, device=dev)
    nat.check(nat.load().convrot_w4a4_gemm_fp6(nat.ptr(a6), nat.ptr(xs), nat.ptr(w6), nat.ptr(ws), nat.ptr(b), M, N, K,
                                               nat.ptr(out), nat.dtype_code(dtype), nat.stream_of(dev)))
    torch.cuda.synchronize()
    return out


def _assert_exact(got, want, label):
    if want.dtype == np.float32:
        got, want = got.view(np.uint32), want.view(np.uint32)
    bad = int((got != want).sum())
    assert bad == 0, f"{label}: {bad} of {want.size} differ"


@pytest.mark.parametrize("N,K", [(46, 128), (264, 384), (3072, 3072), (1000, 15360)])
def test_weight_fp6_matches_oracle(orc, dev, N, K):
    """CDNA4 weight -> FP6 blocks: every byte as the oracle's layout of the same codes
    (padding columns included), -8 codes included."""
    nat = _nat()
    rng = np.random.default_rng(N + K)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    got = _weight_fp6(nat, _u8(orc.codes_to_cdna4(w), dev), N, K, dev)
    want = orc.codes_to_fp6(w).reshape(-1)
    _assert_exact(from_dev(got), want, f"weight {N}x{K}")
    assert np.array_equal(orc.fp6_to_codes(from_dev(got).reshape(K // 128, -1, 1536), N, K), w)


def test_weight_fp6_minus8_codes(orc, dev):
    """-8 weight codes (the int4 range's end, never emitted by the quantizers) encode as -1.0
    (v/8) and multiply exactly: the FP6 GEMM on a weight of -8 runs equals the oracle."""
    nat = _nat()
    rng = np.random.default_rng(8)
    M, N, K = 64, 64, 512
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    w[3] = -8
    w[60, 255] = -8
    a = rng.integers(-7, 8, size=(M, K), dtype=np.int8)
    a[5] = -7
    got = _weight_fp6(nat, _u8(orc.codes_to_cdna4(w), dev), N, K, dev)
    _assert_exact(from_dev(got), orc.codes_to_fp6(w).reshape(-1), "weight with -8")
    assert int(orc.codes_to_fp6(np.full((1, 128), -8, np.int8))[0, 0, 0]) & 63 == 0x28
    xs = np.ones(M, np.float32)
    ws = np.ones(N, np.float32)
    b = np.zeros(N, np.float32)
    out = _gemm_fp6(nat, _u8(orc.codes_to_fp6(a), dev), _u8(xs, dev), got, _u8(ws, dev), _u8(b, dev), M, N, K,
                    torch.float16, dev)
    _assert_exact(from_dev(out), orc.w4a4_matmul_codes_large(a, w, xs, ws, b, "float16"), "-8 products")


@pytest.mark.parametrize("dtype,G,rows,K", [
    ("bfloat16", 256, 37, 3072),     # config-3 group, ragged rows
    ("bfloat16", 64, 300, 2688),     # config-2 group, K = 21 k-blocks
    ("float16", 16, 19, 512),
    ("float32", 4, 17, 256),
    ("bfloat16", 1024, 33, 2048),
    ("bfloat16", 256, 1536, 3072),   # the reference tests' route shape (test_core.py:128-137)
    ("bfloat16", 256, 20, 15360),
])
def test_prepare_fp6_matches_oracle(orc, dev, dtype, G, rows, K):
    """Fused preparation with FP6 output: the oracle's A4 codes in the FP6 layout, byte for
    byte (rows padded with zero blocks), and the oracle's row scales."""
    nat = _nat()
    x = outlier_input(rows * 7 + K, (rows, K), dtype, orc)
    codes, scales = orc.prepare_codes(x, dtype, G)
    got, s = _prep_fp6(nat, to_dev(x, dtype, dev), G, nat.PREP_FP6, dev)
    assert np.array_equal(from_dev(s), scales), "scales differ"
    _assert_exact(from_dev(got), orc.codes_to_fp6(codes).reshape(-1), f"{dtype} G={G} {rows}x{K}")


def test_prepare_fp6_without_rotation(orc, dev):
    """CONVROT_PREP_FP6 | NO_ROTATE: quantize_signed_int4_rowwise codes in the FP6 layout."""
    nat = _nat()
    x = normal_input(1234, (21, 384), "bfloat16", orc)
    codes, scales = orc.quantize_rowwise_codes(x, "bfloat16")
    got, s = _prep_fp6(nat, to_dev(x, "bfloat16", dev), 256, nat.PREP_FP6 | nat.PREP_NO_ROTATE, dev)
    assert np.array_equal(from_dev(s), scales)
    _assert_exact(from_dev(got), orc.codes_to_fp6(codes).reshape(-1), "no-rotate")


def test_prepare_fp6_zero_and_tiny_rows(orc, dev):
    """An all-zero row, a row of tiny negative values, and rows whose negative ratios round to
    code 0 next to one large value: every code 0 is +0 (no -0 field)."""
    nat = _nat()
    x = normal_input(77, (18, 1024), "bfloat16", orc)
    x[0] = 0
    x[5] = orc.from_f32(np.full(1024, -1e-30, np.float32), "bfloat16")
    small = -np.abs(np.random.default_rng(5).normal(size=1024)).astype(np.float32) * 0.04
    small[::97] = 0.0
    for r, big in ((7, 40.0), (8, -40.0)):
        row = small.copy()
        row[3] = big
        x[r] = orc.from_f32(row, "bfloat16")
    codes, scales = orc.prepare_codes(x, "bfloat16", 256)
    got, s = _prep_fp6(nat, to_dev(x, "bfloat16", dev), 256, nat.PREP_FP6, dev)
    assert np.array_equal(from_dev(s), scales)
    _assert_exact(from_dev(got), orc.codes_to_fp6(codes).reshape(-1), "zero rows")


def test_modulated_and_gelu_producers_fp6(orc, dev):
    """The fused producers' FP6 output equals their INT8 output in the FP6 layout."""
    nat = _nat()
    from convrot_mlx_amd import core

    rows, K = 48, 3072  # whole 16-row blocks: the library leaves padding rows of a ragged last block unwritten
    x = to_dev(outlier_input(5, (rows, K), "bfloat16", orc), "bfloat16", dev)
    shift = torch.randn(K, device=dev).to(torch.bfloat16)
    scale = torch.randn(K, device=dev).to(torch.bfloat16)
    q8, s8 = core._prepare_modulated(x, shift, scale, 256, nat.PREP_INT8, 1e-6)
    q6, s6 = core._prepare_modulated(x, shift, scale, 256, nat.PREP_FP6, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(s8, s6)
    want = orc.codes_to_fp6(from_dev(q8)).reshape(-1)
    _assert_exact(from_dev(q6).reshape(-1)[: want.size], want, "modulated")
    head = to_dev(outlier_input(6, (rows, 3072), "bfloat16", orc), "bfloat16", dev)
    g8, t8 = core._prepare_gelu(x, head, 256, nat.PREP_INT8)
    g6, t6 = core._prepare_gelu(x, head, 256, nat.PREP_FP6)
    torch.cuda.synchronize()
    assert torch.equal(t8, t6)
    want = orc.codes_to_fp6(from_dev(g8)).reshape(-1)
    _assert_exact(from_dev(g6).reshape(-1)[: want.size], want, "gelu")


@pytest.mark.parametrize("out_dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("M,K,N", [(300, 128, 264), (37, 384, 48), (1000, 640, 1000), (520, 1536, 1000),
                                   (4608, 3072, 3072), (301, 256, 1003), (33, 128, 46)])
def test_fp6_gemm_matches_oracle(orc, dev, out_dtype, M, K, N):
    """FP6-operand GEMM, every output bit-exact against the oracle: ragged tiles (N not a
    multiple of 8 included), one and many k-blocks, all-zero activation rows (+0 sums), a row
    of extreme codes, 16-bit and float32 outputs."""
    nat = _nat()
    rng = np.random.default_rng(M + K + N)
    a = rng.integers(-7, 8, size=(M, K), dtype=np.int8)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    a[1] = 0
    a[2] = 7
    w[3] = -8
    xs = rng.uniform(0.01, 0.2, size=(M,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(N,)).astype(np.float32)
    b = rng.normal(size=(N,)).astype(np.float32)
    b[:4] = 0.0
    dt = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}[out_dtype]
    out = _gemm_fp6(nat, _u8(orc.codes_to_fp6(a), dev), _u8(xs, dev), _u8(orc.codes_to_fp6(w), dev), _u8(ws, dev),
                    _u8(b, dev), M, N, K, dt, dev)
    _assert_exact(from_dev(out), orc.w4a4_matmul_codes_large(a, w, xs, ws, b, out_dtype), f"{M}x{K}x{N}")


def test_fp6_gemm_largest_sums(orc, dev):
    """K = 15360 with runs of +-7 * +-7 and -7 * -8: sums up to 860160 (beyond the largest at
    config 3) stay exact."""
    nat = _nat()
    M, K, N = 64, 15360, 64
    rng = np.random.default_rng(15360)
    a = rng.integers(-7, 8, size=(M, K), dtype=np.int8)
    w = rng.integers(-7, 8, size=(N, K), dtype=np.int8)
    a[:8] = 7
    a[8:16] = -7
    w[:8] = 7
    w[8:16] = -7
    w[16:24] = -8
    xs = np.ones(M, np.float32)
    ws = np.ones(N, np.float32)
    b = np.zeros(N, np.float32)
    out = _gemm_fp6(nat, _u8(orc.codes_to_fp6(a), dev), _u8(xs, dev), _u8(orc.codes_to_fp6(w), dev), _u8(ws, dev),
                    _u8(b, dev), M, N, K, torch.bfloat16, dev)
    _assert_exact(from_dev(out), orc.w4a4_matmul_codes_large(a, w, xs, ws, b, "bfloat16"), "largest sums")


def test_fp6_gemm_near_the_k_limit(orc, dev):
    """K = 262016, the largest multiple of 128 the FP6 entry accepts (K < 262144): rows of 7 x 7,
    7 x -8 and -7 x 7 codes reach |sums| of 14.7 M, within 2^24, so the float32 accumulators
    are still exact.  float32 output with unit scales and no bias compares the accumulators
    themselves with the oracle's int64 dots."""
    nat = _nat()
    M, K, N = 32, 262016, 48
    rng = np.random.default_rng(262016)
    a = rng.integers(-7, 8, size=(M, K), dtype=np.int8)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    a[:4] = 7
    a[4:8] = -7
    w[:4] = 7
    w[4:8] = -8
    xs = np.ones(M, np.float32)
    ws = np.ones(N, np.float32)
    b = np.zeros(N, np.float32)
    out = _gemm_fp6(nat, _u8(orc.codes_to_fp6(a), dev), _u8(xs, dev), _u8(orc.codes_to_fp6(w), dev), _u8(ws, dev),
                    _u8(b, dev), M, N, K, torch.float32, dev)
    want = orc.w4a4_matmul_codes_large(a, w, xs, ws, b, "float32")
    assert np.abs(want[:8, :8]).max() == 8 * 7 * K
    _assert_exact(from_dev(out), want, "K = 262016")


@pytest.mark.parametrize("M,G,K,N", [(1536, 256, 3072, 9216), (4608, 256, 12288, 3072), (1000, 64, 3072, 1000)])
def test_fp6_complete_path_equals_int8_path(orc, dev, M, G, K, N):
    """prep(FP6) -> FP6 GEMM on the FP6 conversion of a quantized weight gives the INT8 path's
    output (prep(INT8) -> convrot_w4a4_gemm) bit for bit."""
    nat = _nat()
    from convrot_mlx_amd import core

    gen = torch.Generator(device=dev)
    gen.manual_seed(M + K + N)
    w = torch.randn((N, K), generator=gen, device=dev) * 0.02
    qw, ws = core.quantize_convrot_weight(w, G)
    wq = core.repack_nk_weight_for_cdna4(qw)
    x = torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16)
    bias = torch.randn(N, generator=gen, device=dev) * 0.02
    q8, xs8 = core._prepare(x, G, nat.PREP_INT8)
    want = core.hip_w4a4_int8_matmul(q8, wq, xs8, ws, bias, output_dtype=torch.bfloat16, out_features=N)
    w6 = _weight_fp6(nat, wq, N, K, dev)
    a6, xs6 = _prep_fp6(nat, x, G, nat.PREP_FP6, dev)
    got = _gemm_fp6(nat, a6, xs6, w6, ws.float().contiguous(), bias.float().contiguous(), M, N, K, torch.bfloat16, dev)
    assert torch.equal(xs6, xs8)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("tile", ["256x256", "256x224", "128x256", "128x128", "128x192"])
@pytest.mark.parametrize("M,K,N", [(300, 384, 1000), (37, 128, 48), (520, 1536, 264), (1000, 640, 232)])
def test_fp6_every_tile(orc, dev, tuning, tile, M, K, N):
    """Each FP6 tile (forced through the fp6_tile tuning override) on ragged M / N tails --
    partial 128-, 192-, 224- and 256-wide column tiles, partial 128- and 256-row tiles -- bit-exact
    against the oracle, in bf16 and f16."""
    nat = _nat()
    tuning.set("fp6_tile", tile)
    assert nat.fp6_tile(M, N) == tuple(int(v) for v in tile.split("x")), "the forced tile is not the one planned"
    rng = np.random.default_rng(M * 3 + K + N)
    a = rng.integers(-7, 8, size=(M, K), dtype=np.int8)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    xs = rng.uniform(0.01, 0.2, size=(M,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(N,)).astype(np.float32)
    b = rng.normal(size=(N,)).astype(np.float32)
    args = (_u8(orc.codes_to_fp6(a), dev), _u8(xs, dev), _u8(orc.codes_to_fp6(w), dev), _u8(ws, dev), _u8(b, dev))
    for out_dtype, dt in (("bfloat16", torch.bfloat16), ("float16", torch.float16)):
        out = _gemm_fp6(nat, *args, M, N, K, dt, dev)
        _assert_exact(from_dev(out), orc.w4a4_matmul_codes_large(a, w, xs, ws, b, out_dtype),
                      f"tile {tile} {M}x{K}x{N} {out_dtype}")


@pytest.mark.parametrize("M", [300, 4600])
@pytest.mark.parametrize("call", ["forward", "forward_modulated", "forward_gelu"])
def test_layer_fp6_ragged_rows(orc, dev, M, call):
    """ConvRotLinear on FP6 operands at a row count that is not a multiple of 16, through each
    forward with a per-image gated residual, on the library's own torch.empty buffers: a freed
    allocation of random bytes sits in torch's cache first, so the padding rows of the FP6
    activation's last 16-row block (never written by the preparation) hold garbage.  Every
    output equals the oracle's -- the producer transform (oracle.modulate / gelu_producer_rows),
    the A4 codes, the exact dots, the epilogue, then oracle.gated_residual -- bit for bit
    (reference: the full-shape route checks of test_core.py:128-137,375-402)."""
    from convrot_mlx_amd import ConvRotLinear, core, quantize_convrot_weight

    B, K, N, G, HEAD = 2, 3072, 1000, 64, 768
    L = M // B
    assert core.fp6_eligible(M, N, K, torch.bfloat16)
    rng = np.random.default_rng(M + len(call))
    w16 = outlier_input(int(rng.integers(1 << 30)), (N, K), "bfloat16", orc, std=0.02, frac=0.01, factor=10.0)
    bias = rng.normal(0, 0.02, size=N).astype(np.float32)
    qw, ws = quantize_convrot_weight(to_dev(w16, "bfloat16", dev), G)
    layer = ConvRotLinear(K, N, group_size=G, device=dev).load_nk_weight(qw, ws, torch.from_numpy(bias).to(dev))
    w_codes, wscales = orc.prepare_codes(w16, "bfloat16", G)
    assert np.array_equal(from_dev(layer.scales), wscales)

    x16 = outlier_input(int(rng.integers(1 << 30)), (M, K), "bfloat16", orc)
    res16 = orc.from_f32((rng.normal(size=(M, N)) * 4).astype(np.float32), "bfloat16")
    gate16 = orc.from_f32(rng.normal(size=(B, N)).astype(np.float32), "bfloat16")
    x = to_dev(x16, "bfloat16", dev).reshape(B, L, K)
    res = to_dev(res16, "bfloat16", dev).reshape(B, L, N)
    gate = to_dev(gate16, "bfloat16", dev).reshape(B, 1, N)
    junk = torch.randint(0, 256, (64 << 20,), dtype=torch.uint8, device=dev)
    del junk
    if call == "forward":
        rows = x16
        got = layer(x, residual=res, gate=gate)
    elif call == "forward_modulated":
        sh16 = orc.from_f32(rng.normal(size=(B, K)).astype(np.float32), "bfloat16")
        sc16 = orc.from_f32(rng.normal(size=(B, K)).astype(np.float32), "bfloat16")
        rows = orc.modulate(x16, "bfloat16", sh16, sc16, L, 1e-6)
        got = layer.forward_modulated(x, to_dev(sh16, "bfloat16", dev).reshape(B, 1, K),
                                      to_dev(sc16, "bfloat16", dev).reshape(B, 1, K), eps=1e-6,
                                      residual=res, gate=gate)
    else:
        rows = orc.gelu_producer_rows(x16[:, :HEAD], np.ascontiguousarray(x16[:, HEAD:]), "bfloat16")
        got = layer.forward_gelu(x[..., HEAD:], head=x[..., :HEAD], residual=res, gate=gate)
    torch.cuda.synchronize()
    a_codes, xs = orc.prepare_codes(rows, "bfloat16", G)
    lin = orc.w4a4_matmul_codes_large(a_codes, w_codes, xs, wscales, bias, "bfloat16")
    want = orc.gated_residual(lin, res16, gate16, L, "bfloat16")
    assert got.shape == (B, L, N)
    _assert_exact(from_dev(got.reshape(M, N)), want, f"{call} M={M}")


@pytest.mark.timeout(300)
def test_video_transfer_shape_bit_exact(orc, dev):
    """The reference's published Wan 2.2 projection (docs/benchmarks/video-transfer.md:15),
    M = 7800, K = N = 5120, through ConvRotLinear (G = 256, FP6 operands, with bias) on
    heavy-tailed operands: weight codes and scales, and every output, equal the oracle's."""
    from convrot_mlx_amd import ConvRotLinear, core, quantize_convrot_weight

    M, K, N, G = 7800, 5120, 5120, 256
    assert core.fp6_eligible(M, N, K, torch.bfloat16)
    w16 = outlier_input(7800, (N, K), "bfloat16", orc, std=0.02, frac=0.01, factor=10.0)
    x16 = outlier_input(5120, (M, K), "bfloat16", orc)
    bias = np.random.default_rng(7).normal(0, 0.02, size=N).astype(np.float32)
    qw, ws = quantize_convrot_weight(to_dev(w16, "bfloat16", dev), G)
    layer = ConvRotLinear(K, N, group_size=G, device=dev).load_nk_weight(qw, ws, torch.from_numpy(bias).to(dev))
    got = layer(to_dev(x16, "bfloat16", dev))
    torch.cuda.synchronize()
    w_codes, wscales = orc.prepare_codes(w16, "bfloat16", G)
    assert np.array_equal(orc.unpack_signed_int4(from_dev(qw)), w_codes)
    assert np.array_equal(from_dev(ws), wscales)
    a_codes, xs = orc.prepare_codes(x16, "bfloat16", G)
    _assert_exact(from_dev(got), orc.w4a4_matmul_codes_large(a_codes, w_codes, xs, wscales, bias, "bfloat16"),
                  "7800x5120->5120")


# ---- compact FP6 weights (the FP6 fields without their exponent bits, 0.5 byte a weight)


def _weight_fp6c(nat, wq_dev, N, K, dev):
    out = torch.zeros(int(nat.load().convrot_cdna4_bytes(N, K)), dtype=torch.uint8, device=dev)
    flag = torch.full((1,), 7, dtype=torch.int32, device=dev)
    nat.check(nat.load().convrot_weight_fp6_compact(nat.ptr(wq_dev), nat.ptr(out), nat.ptr(flag), N, K,
                                                    nat.stream_of(dev)))
    torch.cuda.synchronize()
    return out, int(flag.item())


def _gemm_fp6c(nat, a6, xs, w6c, ws, b, M, N, K, dtype, dev, residual=None, gate=None, gate_stride=0, rpg=1):
    out = torch.empty((M, N), dtype=dtype, device=dev)
    nat.check(nat.load().convrot_w4a4_gemm_fp6_compact(
        nat.ptr(a6), nat.ptr(xs), nat.ptr(w6c), nat.ptr(ws), nat.ptr(b), M, N, K, nat.ptr(residual), nat.ptr(gate),
        gate_stride, rpg, nat.ptr(out), nat.dtype_code(dtype), nat.stream_of(dev)))
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("N,K", [(46, 128), (264, 384), (3072, 3072), (1000, 15360)])
def test_weight_fp6_compact_matches_oracle(orc, dev, N, K):
    """CDNA4 weight -> compact FP6 blocks: every byte as oracle.codes_to_fp6c of the same
    codes (padding included), the -8 flag cleared; a -8 code anywhere raises the flag."""
    nat = _nat()
    rng = np.random.default_rng(N + K + 6)
    w = rng.integers(-7, 8, size=(N, K), dtype=np.int8)
    got, flag = _weight_fp6c(nat, _u8(orc.codes_to_cdna4(w), dev), N, K, dev)
    assert flag == 0
    _assert_exact(from_dev(got), orc.codes_to_fp6c(w).reshape(-1), f"compact weight {N}x{K}")
    assert np.array_equal(orc.fp6c_to_codes(from_dev(got).reshape(K // 128, -1, 1024), N, K), w)
    w[N // 2, K - 1] = -8
    _, flag = _weight_fp6c(nat, _u8(orc.codes_to_cdna4(w), dev), N, K, dev)
    assert flag == 1


@pytest.mark.parametrize("tile", ["256x256", "256x224", "128x256", "128x128", "128x192"])
@pytest.mark.parametrize("M,K,N", [(300, 384, 1000), (37, 128, 48), (520, 1536, 264), (1000, 640, 232)])
def test_fp6_compact_gemm_every_tile(orc, dev, tuning, tile, M, K, N):
    """The FP6 GEMM on compact weights (each fragment expanded in registers), every tile forced,
    ragged M / N: bit-exact against the oracle in bf16, f16 and f32, and a gated residual in
    bf16 against oracle.gated_residual."""
    nat = _nat()
    tuning.set("fp6_tile", tile)
    rng = np.random.default_rng(M * 5 + K + N)
    a = rng.integers(-7, 8, size=(M, K), dtype=np.int8)
    w = rng.integers(-7, 8, size=(N, K), dtype=np.int8)
    a[1] = 0
    w[2] = 7
    w[3] = -7
    xs = rng.uniform(0.01, 0.2, size=(M,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(N,)).astype(np.float32)
    b = rng.normal(size=(N,)).astype(np.float32)
    args = (_u8(orc.codes_to_fp6(a), dev), _u8(xs, dev), _u8(orc.codes_to_fp6c(w), dev), _u8(ws, dev), _u8(b, dev))
    for out_dtype, dt in (("bfloat16", torch.bfloat16), ("float16", torch.float16), ("float32", torch.float32)):
        out = _gemm_fp6c(nat, *args, M, N, K, dt, dev)
        _assert_exact(from_dev(out), orc.w4a4_matmul_codes_large(a, w, xs, ws, b, out_dtype),
                      f"compact tile {tile} {M}x{K}x{N} {out_dtype}")
    res16 = orc.from_f32((rng.normal(size=(M, N)) * 4).astype(np.float32), "bfloat16")
    gate16 = orc.from_f32(rng.normal(size=(2, N)).astype(np.float32), "bfloat16")
    rpg = (M + 1) // 2
    out = _gemm_fp6c(nat, *args, M, N, K, torch.bfloat16, dev, residual=to_dev(res16, "bfloat16", dev),
                     gate=to_dev(gate16, "bfloat16", dev), gate_stride=N, rpg=rpg)
    lin = orc.w4a4_matmul_codes_large(a, w, xs, ws, b, "bfloat16")
    _assert_exact(from_dev(out), orc.gated_residual(lin, res16, gate16, rpg, "bfloat16"), f"compact residual {tile}")


def test_layer_caches_compact_weights_except_minus8(orc, dev, fp6_form):
    """ConvRotLinear caches the compact form for a quantized weight (0.5 byte a weight) and
    the 1536-byte FP6 blocks for a weight holding a -8 code (assigned as raw CDNA4 bytes);
    both layers reproduce the oracle bit for bit."""
    from convrot_mlx_amd import ConvRotLinear, core

    fp6_form("compact")
    M, K, N = 300, 384, 200
    rng = np.random.default_rng(300)
    x16 = orc.from_f32(rng.normal(size=(M, K)).astype(np.float32), "bfloat16")
    a_codes, xs = orc.prepare_codes(x16, "bfloat16", 64)
    for minus8 in (False, True):
        w = rng.integers(-7, 8, size=(N, K), dtype=np.int8)
        if minus8:
            w[7, 100] = -8
        ws = rng.uniform(0.001, 0.01, size=N).astype(np.float32)
        b = rng.normal(size=N).astype(np.float32)
        layer = ConvRotLinear(K, N, group_size=64, device=dev)
        layer.qweight = _u8(orc.codes_to_cdna4(w), dev)
        layer.scales = _u8(ws, dev)
        layer.bias = _u8(b, dev)
        got = layer(to_dev(x16, "bfloat16", dev))
        torch.cuda.synchronize()
        w6 = layer._fp6_cache[1]
        assert w6.shape[-1] == (1536 if minus8 else 1024)
        assert w6.numel() == (core.fp6_bytes(N, K) if minus8 else int(np.prod(core.cdna4_shape(N, K))))
        _assert_exact(from_dev(got), orc.w4a4_matmul_codes_large(a_codes, w, xs, ws, b, "bfloat16"),
                      f"layer, -8 in weight: {minus8}")


def test_fp6_weight_form_policy(orc, dev, fp6_form):
    """The automatic FP6 weight form is the compact one on every tile (256-row tiles at config 3's
    4608 rows, 128-row tiles at 512 rows); a forced form applies everywhere, a bad name raises,
    and a layer rebuilds its cache when the setting changes -- every form giving the same
    output bits."""
    from convrot_mlx_amd import ConvRotLinear, core, quantize_convrot_weight

    assert core.fp6_weight_form(4608, 3072) == "compact" and core.fp6_weight_form(4608, 21504) == "compact"
    assert core.fp6_weight_form(512, 3072) == "compact"
    with pytest.raises(ValueError, match="weight form"):
        core.set_fp6_weight_form("tiny")
    M, K, N, G = 512, 1024, 768, 64
    gen = torch.Generator(device=dev).manual_seed(6)
    qw, ws = quantize_convrot_weight((torch.randn((N, K), generator=gen, device=dev) * 0.02).to(torch.bfloat16), G)
    layer = ConvRotLinear(K, N, group_size=G, device=dev).load_nk_weight(qw, ws)
    x = torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16)
    outs = {}
    for form, block in (("auto", 1024), ("compact", 1024), ("full", 1536)):
        fp6_form(form)
        outs[form] = layer(x)
        torch.cuda.synchronize()
        assert layer._fp6_cache[1].shape[-1] == block, form
    assert torch.equal(outs["compact"], outs["full"]) and torch.equal(outs["auto"], outs["full"])


def test_layer_under_graph_capture_without_fp6_cache(orc, dev, fp6_form):
    """A layer whose FP6 weight form is not cached yet, first called under HIP-graph capture,
    runs on INT8 operands (the compact conversion reads a flag back and cannot run there);
    every replay equals the eager FP6 result bit for bit, and the cache appears on the next
    eager call."""
    from convrot_mlx_amd import ConvRotLinear, core, quantize_convrot_weight

    fp6_form("compact")
    M, K, N, G = 512, 1024, 768, 64
    gen = torch.Generator(device=dev).manual_seed(5)
    w = (torch.randn((N, K), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
    qw, ws = quantize_convrot_weight(w, G)
    layer = ConvRotLinear(K, N, group_size=G, device=dev).load_nk_weight(qw, ws)
    x = torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        layer(x[:16])  # the few-row path: workspace-free, no FP6 form
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            static = layer(x)
        assert layer._fp6_cache is None
        eager = layer(x)
        torch.cuda.synchronize()
        assert layer._fp6_cache is not None and layer._fp6_cache[1].shape[-1] == 1024
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(static, eager)
            layer(x[:300])
    torch.cuda.current_stream().wait_stream(stream)
