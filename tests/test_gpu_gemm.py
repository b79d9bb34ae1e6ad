"""GPU parity: INT8-MFMA W4A4 GEMM + fused epilogue vs the CPU oracle.

Integer accumulators must be exact (unit scales, zero bias, float32 output),
and every output must equal the oracle's bit for bit (the epilogue is the
same sequence of float32 roundings).  Seeds and shapes follow
/root/reference/tests/test_core.py:139-175,213-283,329-373.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import from_dev, normal_input, outlier_input, to_dev

pytestmark = pytest.mark.gpu


def _api():
    import convrot_mlx_amd as api

    return api


def _dev_u8(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


# Output names of _run_both, in order: the C ABI's packed-activation kernel (register-staged,
# reads the packed codes itself), the packed Python entry point (unpacks to int8, then the
# int8 kernels) and the int8 entry point.
_BOTH = ("packed-kernel", "packed-api", "int8")


def _run_both(orc, dev, a_codes, w_codes, xs, ws, bias, out_dtype):
    """Run the packed-A kernel, the packed-A and the int8-A entry points with a CDNA4 weight."""
    from convrot_mlx_amd import _native as nat

    api = _api()
    N, K = w_codes.shape
    wq = _dev_u8(orc.codes_to_cdna4(w_codes), dev)
    qact = _dev_u8(orc.pack_signed_int4(a_codes), dev)
    a8 = torch.from_numpy(np.ascontiguousarray(a_codes)).to(dev)
    xs_d, ws_d = torch.from_numpy(xs).to(dev), torch.from_numpy(ws).to(dev)
    b_d = torch.from_numpy(bias).to(dev)
    dt = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}[out_dtype]
    M = a_codes.shape[0]
    out_k = torch.empty((M, N), dtype=dt, device=dev)
    nat.check(nat.load().convrot_w4a4_gemm(nat.ptr(qact), nat.ACT_PACKED, nat.ptr(xs_d), nat.ptr(wq), nat.ptr(ws_d),
                                           nat.ptr(b_d), M, N, K, nat.ptr(out_k), nat.dtype_code(dt),
                                           nat.stream_of(dev)))
    out_p = api.hip_w4a4_matmul(qact, wq, xs_d, ws_d, b_d, output_dtype=dt, out_features=N)
    out_8 = api.hip_w4a4_int8_matmul(a8, wq, xs_d, ws_d, b_d, output_dtype=dt, out_features=N)
    torch.cuda.synchronize()
    return from_dev(out_k), from_dev(out_p), from_dev(out_8)


def _assert_exact(got, expected, label):
    if got.dtype == np.float32:
        bad = int((got.view(np.uint32) != expected.view(np.uint32)).sum())
    else:
        bad = int((got != expected).sum())
    assert bad == 0, f"{label}: {bad} of {expected.size} outputs differ"


@pytest.mark.parametrize("out_dtype", ["float32", "bfloat16", "float16"])
def test_edges_37x64x46(orc, dev, out_dtype):
    """test_core.py:213-283: seed 2026082302, M=37, K=64, N=46, codes in [-7, 7]."""
    rng = np.random.default_rng(2026082302)
    a = rng.integers(-7, 8, size=(37, 64), dtype=np.int8)
    w = rng.integers(-7, 8, size=(46, 64), dtype=np.int8)
    xs = rng.uniform(0.01, 0.2, size=(37,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(46,)).astype(np.float32)
    b = rng.normal(size=(46,)).astype(np.float32)
    expected = orc.w4a4_matmul_codes(a, w, xs, ws, b, out_dtype)
    for got, name in zip(_run_both(orc, dev, a, w, xs, ws, b, out_dtype), _BOTH):
        _assert_exact(got, expected, f"{name} {out_dtype}")


def test_exact_integer_dots(orc, dev):
    """Unit scales and zero bias: the float32 output is the exact integer dot (test_core.py:244-264)."""
    rng = np.random.default_rng(2026082302)
    a = rng.integers(-8, 8, size=(37, 320), dtype=np.int8)  # -8 included: unpack covers [-8, 7]
    w = rng.integers(-8, 8, size=(46, 320), dtype=np.int8)
    ones_m, ones_n, zeros_n = np.ones(37, np.float32), np.ones(46, np.float32), np.zeros(46, np.float32)
    dots = a.astype(np.int64) @ w.astype(np.int64).T
    for got, name in zip(_run_both(orc, dev, a, w, ones_m, ones_n, zeros_n, "float32"), _BOTH):
        assert np.array_equal(got, dots.astype(np.float32)), name


def test_max_magnitude_accumulators(orc, dev):
    """|acc| at its largest: every code -8/7 at K=15360 stays exact."""
    K = 15360
    a = np.full((16, K), -8, np.int8)
    a[1::2] = 7
    w = np.full((32, K), -8, np.int8)
    w[::3] = 7
    ones_m, ones_n, zeros_n = np.ones(16, np.float32), np.ones(32, np.float32), np.zeros(32, np.float32)
    dots = a.astype(np.int64) @ w.astype(np.int64).T
    for got, name in zip(_run_both(orc, dev, a, w, ones_m, ones_n, zeros_n, "float32"), _BOTH):
        assert np.array_equal(got, dots.astype(np.float32)), name


@pytest.mark.parametrize(
    "seed,M,K,N", [(29, 17, 512, 39), (27, 31, 1024, 61), (2026082300, 14, 256, 33), (5, 1, 3072, 64),
                   (6, 130, 2688, 272), (8, 257, 128, 129)]
)
def test_odd_shapes_bf16(orc, dev, seed, M, K, N):
    """test_core.py:139-175,329-355 shapes and ragged tails on every tile edge, bf16 output."""
    rng = np.random.default_rng(seed)
    a = rng.integers(-7, 8, size=(M, K), dtype=np.int8)
    w = rng.integers(-7, 8, size=(N, K), dtype=np.int8)
    xs = rng.uniform(0.01, 0.2, size=(M,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(N,)).astype(np.float32)
    b = rng.normal(size=(N,)).astype(np.float32)
    expected = orc.w4a4_matmul_codes(a, w, xs, ws, b, "bfloat16")
    for got, name in zip(_run_both(orc, dev, a, w, xs, ws, b, "bfloat16"), _BOTH):
        _assert_exact(got, expected, f"{name} seed {seed}")


# Tiles the automatic choice picks (BMxBN, waves WMxWN), plus 2x2-wave register-staged
# variants that are only reached through the override.
_TILES = ["256x256w2x4", "256x128w4x2", "128x256w2x4", "128x128w2x2", "192x128w4x2", "256x256w2x2",
          "288x192w2x2", "256x128w2x2", "128x256w2x2", "256x256w4x2"]


@pytest.mark.parametrize("no_dma", [False, True], ids=["dma", "regstaged"])
@pytest.mark.parametrize("tile", _TILES)
@pytest.mark.parametrize("seed,M,K,N", [(41, 300, 384, 530), (42, 17, 2688, 46), (43, 520, 256, 264)])
def test_every_tile_config(orc, dev, tuning, tile, no_dma, seed, M, K, N):
    """Each GEMM tile variant (forced through the gemm_tile tuning override; gemm_no_dma selects
    the register-staged int8 kernel) on ragged M/N/K tails."""
    tuning.set("gemm_tile", tile)
    if no_dma:
        tuning.set("gemm_no_dma", "1")
    else:
        tuning.set("gemm_no_dma", None)
    rng = np.random.default_rng(seed)
    a = rng.integers(-8, 8, size=(M, K), dtype=np.int8)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    xs = rng.uniform(0.01, 0.2, size=(M,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(N,)).astype(np.float32)
    b = rng.normal(size=(N,)).astype(np.float32)
    expected = orc.w4a4_matmul_codes(a, w, xs, ws, b, "bfloat16")
    for got, name in zip(_run_both(orc, dev, a, w, xs, ws, b, "bfloat16"), _BOTH):
        _assert_exact(got, expected, f"{name} tile {tile}")


@pytest.mark.parametrize("tile", ["256x256w2x4", "256x256w2x2", "256x128w4x2", "128x256w2x4", "128x128w2x2",
                                  "192x128w4x2"])
@pytest.mark.parametrize(
    "seed,M,K,N,sk_min",
    [(51, 300, 2688, 530, 1),    # tiles split into up to 21 one-k-block pieces
     (52, 37, 64, 46, 1),        # a single k-block: pieces are whole tiles
     (53, 2100, 384, 16384, 4)],  # whole-tile rounds followed by a stream-K remainder
)
def test_stream_k(orc, dev, tuning, tile, seed, M, K, N, sk_min):
    """Stream-K kernel forced on: partial tiles summed across workgroups must give the
    single-pass result bit for bit; two launches in a row check the re-armed counters."""
    api = _api()
    tuning.set("gemm_tile", tile)
    tuning.set("gemm_sk", "1")
    tuning.set("gemm_sk_min", str(sk_min))
    tuning.set("gemm_no_dma", None)
    rng = np.random.default_rng(seed)
    a = rng.integers(-8, 8, size=(M, K), dtype=np.int8)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    xs = rng.uniform(0.01, 0.2, size=(M,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(N,)).astype(np.float32)
    b = rng.normal(size=(N,)).astype(np.float32)
    rows = np.arange(M) if M * N <= 200_000 else np.sort(rng.choice(M, size=64, replace=False))
    expected = orc.w4a4_matmul_codes(a[rows], w, xs[rows], ws, b, "bfloat16")
    wq = _dev_u8(orc.codes_to_cdna4(w), dev)
    a8 = torch.from_numpy(a).to(dev)
    args = (torch.from_numpy(xs).to(dev), torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev))
    for call in range(2):
        out = api.hip_w4a4_int8_matmul(a8, wq, *args, output_dtype=torch.bfloat16, out_features=N)
        torch.cuda.synchronize()
        _assert_exact(from_dev(out)[rows], expected, f"tile {tile} call {call}")


@pytest.mark.parametrize("sk", [False, True], ids=["dp", "sk"])
@pytest.mark.parametrize("tile", ["256x256w2x4", "256x256w2x2", "256x128w4x2", "128x256w2x4", "128x128w2x2",
                                  "192x128w4x2", "288x192w2x2"])
@pytest.mark.parametrize("out_dtype", ["float32", "float16"])
def test_epilogue_operands_without_bias(orc, dev, tuning, tile, sk, out_dtype):
    """The DMA kernels stage xs / ws / bias of each tile in LDS: ragged M and N that are not
    multiples of 4 (the staged copies end mid-vector) and a missing bias (read as zeros)."""
    api = _api()
    tuning.set("gemm_tile", tile)
    tuning.set("gemm_sk", "1" if sk else "0")
    tuning.set("gemm_sk_min", "1")
    tuning.set("gemm_no_dma", None)
    M, K, N = 301, 384, 531
    rng = np.random.default_rng(61)
    a = rng.integers(-8, 8, size=(M, K), dtype=np.int8)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    xs = rng.uniform(0.01, 0.2, size=(M,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(N,)).astype(np.float32)
    dt = {"float16": torch.float16, "float32": torch.float32}[out_dtype]
    out = api.hip_w4a4_int8_matmul(torch.from_numpy(a).to(dev), _dev_u8(orc.codes_to_cdna4(w), dev),
                                   torch.from_numpy(xs).to(dev), torch.from_numpy(ws).to(dev), None,
                                   output_dtype=dt, out_features=N)
    torch.cuda.synchronize()
    expected = orc.w4a4_matmul_codes(a, w, xs, ws, np.zeros(N, np.float32), out_dtype)
    _assert_exact(from_dev(out), expected, f"tile {tile} sk={sk} {out_dtype}")


def test_kn_layout_entry_matches(orc, dev):
    """mpp_w4a4_matmul with the reference's K x packed-N weight (repacked on device)."""
    api = _api()
    rng = np.random.default_rng(2026082302)
    a = rng.integers(-7, 8, size=(37, 64), dtype=np.int8)
    w = rng.integers(-7, 8, size=(46, 64), dtype=np.int8)
    xs = rng.uniform(0.01, 0.2, size=(37,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(46,)).astype(np.float32)
    b = rng.normal(size=(46,)).astype(np.float32)
    kn = orc.repack_nk_weight_for_mpp(orc.pack_signed_int4(w))
    out = api.mpp_w4a4_matmul(
        _dev_u8(orc.pack_signed_int4(a), dev), _dev_u8(kn, dev), torch.from_numpy(xs).to(dev),
        torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev), output_dtype=torch.float32,
    )
    _assert_exact(from_dev(out), orc.w4a4_matmul_codes(a, w, xs, ws, b, "float32"), "kn entry")


# Benchmark configs 2 (M = 1536, G = 64) and 3 (M = 4608, G = 256, the four FLUX double-block
# shapes plus the fused single-block linears 3072->21504 and 15360->3072).
FLUX_SHAPES = [(1536, 64, 3072, 9216), (1536, 64, 3072, 3072), (1536, 64, 3072, 12288), (1536, 64, 12288, 3072),
               (1536, 64, 3072, 21504), (1536, 64, 15360, 3072),
               (4608, 256, 3072, 9216), (4608, 256, 3072, 3072), (4608, 256, 3072, 12288), (4608, 256, 12288, 3072),
               (4608, 256, 3072, 21504), (4608, 256, 15360, 3072)]


@pytest.mark.parametrize("operands", ["fp6", "int8"])
@pytest.mark.parametrize("M,G,K,N", FLUX_SHAPES)
def test_flux_shapes_complete_path(orc, dev, M, G, K, N, operands):
    """benchmark configs 2/3 at full size through ConvRotLinear (prep kernel -> GEMM kernel),
    on the configs' heavy-tailed inputs, on FP6 operands (the default at these sizes) and on
    INT8 operands.  Every weight code and scale, every activation code and scale (and, on
    FP6, every byte of the FP6 activation blocks), and every output must equal the oracle's
    bit for bit (the oracle's dots come from w4a4_dots_exact, its epilogue from the C
    restatement)."""
    api = _api()
    x = outlier_input(K + N, (M, K), "bfloat16", orc)
    w = outlier_input(K * 3 + N, (N, K), "bfloat16", orc, std=0.02, frac=0.01, factor=10.0)
    bias = np.random.default_rng(N).normal(0.0, 0.02, size=N).astype(np.float32)
    xd, wd = to_dev(x, "bfloat16", dev), to_dev(w, "bfloat16", dev)
    qw, ws = api.quantize_convrot_weight(wd, G)
    layer = api.ConvRotLinear(K, N, group_size=G, backend="hip-w4a4", device=dev)
    layer.load_nk_weight(qw, ws, torch.from_numpy(bias).to(dev))
    was = api.fp6_operands_enabled()
    api.set_fp6_operands(operands == "fp6")
    try:
        assert api.fp6_eligible(M, N, K, torch.bfloat16) == (operands == "fp6")
        y = from_dev(layer(xd))
    finally:
        api.set_fp6_operands(was)
    a_dev, xs_dev = api.hip_fused_prepare_convrot_activation_i8(xd, G)
    w_codes, wscales = orc.prepare_codes(w, "bfloat16", G)
    assert np.array_equal(from_dev(ws), wscales), "weight scales"
    assert np.array_equal(orc.unpack_signed_int4(from_dev(qw)), w_codes), "weight codes"
    a_codes, xs = orc.prepare_codes(x, "bfloat16", G)
    assert np.array_equal(from_dev(xs_dev), xs), "activation scales"
    assert np.array_equal(from_dev(a_dev), a_codes), "activation codes"
    if operands == "fp6":
        a6, xs6 = api.hip_fused_prepare_convrot_activation_fp6(xd, G)
        assert np.array_equal(from_dev(xs6), xs), "activation scales (FP6 preparation)"
        assert np.array_equal(from_dev(a6), orc.codes_to_fp6(a_codes)), "FP6 activation blocks"
    expected = orc.w4a4_matmul_codes_large(a_codes, w_codes, xs, wscales, bias, "bfloat16")
    _assert_exact(y, expected, f"{M}x{K}->{N} {operands}")


@pytest.mark.parametrize("cfg", ["A", "B", "C", "F"])
@pytest.mark.parametrize("out_dtype", ["bfloat16", "float32", "float16"])
@pytest.mark.parametrize("seed,M,K,N", [(61, 1, 3072, 530), (62, 5, 64, 46), (63, 16, 2688, 18432 // 8),
                                        (64, 17, 384, 100), (65, 32, 1024, 1024), (66, 47, 256, 33)])
def test_small_m_kernel(orc, dev, tuning, cfg, out_dtype, seed, M, K, N):
    """The few-row W4A4 kernel (every work split, forced) against the oracle bit for bit,
    on ragged N and K tails, one to three token tiles."""
    api = _api()
    tuning.set("gemm_smallm_max", "64")
    tuning.set("w4a4_smallm_cfg", cfg)
    rng = np.random.default_rng(seed)
    a = rng.integers(-7, 8, size=(M, K), dtype=np.int8)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    xs = rng.uniform(0.01, 0.2, size=(M,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(N,)).astype(np.float32)
    b = rng.normal(size=(N,)).astype(np.float32)
    expected = orc.w4a4_matmul_codes(a, w, xs, ws, b, out_dtype)
    wq = _dev_u8(orc.codes_to_cdna4(w), dev)
    a8 = torch.from_numpy(a).to(dev)
    dt = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}[out_dtype]
    args = (torch.from_numpy(xs).to(dev), torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev))
    for _ in range(2):
        out = api.hip_w4a4_int8_matmul(a8, wq, *args, output_dtype=dt, out_features=N)
        _assert_exact(from_dev(out), expected, f"small-M cfg {cfg}")
    no_bias = api.hip_w4a4_int8_matmul(a8, wq, args[0], args[1], None, output_dtype=dt, out_features=N)
    _assert_exact(from_dev(no_bias), orc.w4a4_matmul_codes(a, w, xs, ws, np.zeros(N, np.float32), out_dtype),
                  f"small-M cfg {cfg} without bias")


@pytest.mark.parametrize("tile", ["256x256w2x4", "256x256w2x2", "288x192w2x2"])
@pytest.mark.parametrize("M,K,N", [(4608, 3072, 3072), (1536, 12288, 3072), (520, 15360, 1000), (300, 128, 264)])
def test_large_tiles_full_output(orc, dev, tuning, tile, M, K, N):
    """The large tiles (256x256 with 8 waves and the accumulator in VGPRs; 256x256 and 288x192
    with 4 waves and the accumulator in the AGPRs, software-pipelined k-steps) forced on
    full-size and ragged shapes, every output compared bit for bit: one and many k-blocks, a
    ragged last tile row and column."""
    api = _api()
    tuning.set("gemm_tile", tile)
    tuning.set("gemm_sk", "0")
    rng = np.random.default_rng(M + K + N)
    a = rng.integers(-8, 8, size=(M, K), dtype=np.int8)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    xs = rng.uniform(0.01, 0.2, size=(M,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(N,)).astype(np.float32)
    b = rng.normal(size=(N,)).astype(np.float32)
    out = api.hip_w4a4_int8_matmul(torch.from_numpy(a).to(dev), _dev_u8(orc.codes_to_cdna4(w), dev),
                                   torch.from_numpy(xs).to(dev), torch.from_numpy(ws).to(dev),
                                   torch.from_numpy(b).to(dev), output_dtype=torch.bfloat16, out_features=N)
    _assert_exact(from_dev(out), orc.w4a4_matmul_codes_large(a, w, xs, ws, b, "bfloat16"), f"tile {tile}")


@pytest.mark.parametrize("tile", ["256x256w2x2", "128x256w2x4"])
def test_stream_k_wait_timeout_is_reported(orc, dev, tuning, tile):
    """A stream-K owner whose bounded wait for a partial tile gives up -- forced from the host
    with zero polls, so every kernel still runs to its end -- writes NaN over its tile instead
    of a silently wrong value and sets the workspace's error word: w4a4_status raises once and
    clears it.  The next launch (normal bounded wait) is exact again: flags left by the failed
    launch carry an older generation and never match.

    600x2688->600 has 21 k-blocks per tile; with stream-K ranges of at least 14 k-blocks, the
    XCD groups that hold two tiles split them into three pieces (their owners wait), while
    the groups that hold one tile run it as a single piece (no wait, never poisoned)."""
    api = _api()
    from convrot_mlx_amd import _native as nat

    tuning.set("gemm_tile", tile)
    tuning.set("gemm_sk", "1")
    tuning.set("gemm_sk_min", "14")
    M, K, N = 600, 2688, 600
    rng = np.random.default_rng(71)
    a = rng.integers(-8, 8, size=(M, K), dtype=np.int8)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    xs = rng.uniform(0.01, 0.2, size=(M,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(N,)).astype(np.float32)
    b = rng.normal(size=(N,)).astype(np.float32)
    expected = orc.w4a4_matmul_codes(a, w, xs, ws, b, "float32")
    args = (torch.from_numpy(a).to(dev), _dev_u8(orc.codes_to_cdna4(w), dev), torch.from_numpy(xs).to(dev),
            torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev))

    def run():
        out = api.hip_w4a4_int8_matmul(*args, output_dtype=torch.float32, out_features=N)
        torch.cuda.synchronize()
        return from_dev(out)

    api.w4a4_status(dev)  # nothing pending from earlier tests
    tuning.set("sk_spin_limit", "0")
    got = run()
    nan = np.isnan(got)
    assert nan.any(), "no owner waited: the forced give-up did not happen"
    assert not nan.all(), "whole tiles and single-piece tiles must not be poisoned"
    assert np.array_equal(got[~nan].view(np.uint32), expected[~nan].view(np.uint32))
    with pytest.raises(nat.ConvRotNativeError, match="gave up"):
        api.w4a4_status(dev)
    api.w4a4_status(dev)  # the error word was cleared
    tuning.set("sk_spin_limit", None)
    for _ in range(2):
        _assert_exact(run(), expected, f"tile {tile} after a failed launch")
    api.w4a4_status(dev)


@pytest.mark.parametrize("tile", ["288x192w2x2", "256x256w2x2"])
@pytest.mark.parametrize("out_dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("grid,M,K,N", [(8, 1000, 640, 1000),   # 4 x 6 / 4 x 4 tiles, ragged edges, 3 per workgroup
                                        (16, 600, 384, 776),    # more workgroups than tiles
                                        (8, 300, 128, 264),     # one k-block
                                        (8, 2000, 1408, 1536)])  # 7 x 8 / 8 x 6 tiles, 11 k-blocks
def test_persistent_kernel(orc, dev, tuning, tile, out_dtype, grid, M, K, N):
    """The persistent 4-wave kernel (which the automatic plan runs when a 4-wave tile's grid
    exceeds one round) forced on a small grid through the gemm_persist override, so every
    workgroup runs several tiles: every output bit-exact against the oracle and equal to the
    one-tile-per-workgroup kernel's."""
    api = _api()
    tuning.set("gemm_tile", tile)
    tuning.set("gemm_sk", "0")
    tuning.set("gemm_smallm_max", "0")
    rng = np.random.default_rng(M + K + N + grid)
    a = rng.integers(-8, 8, size=(M, K), dtype=np.int8)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    xs = rng.uniform(0.01, 0.2, size=(M,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(N,)).astype(np.float32)
    b = rng.normal(size=(N,)).astype(np.float32)
    want = orc.w4a4_matmul_codes_large(a, w, xs, ws, b, out_dtype)
    args = (torch.from_numpy(a).to(dev), _dev_u8(orc.codes_to_cdna4(w), dev), torch.from_numpy(xs).to(dev),
            torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev))
    dt = {"bfloat16": torch.bfloat16, "float16": torch.float16}[out_dtype]
    outs = {}
    for mode in (str(grid), "0"):
        tuning.set("gemm_persist", mode)
        for call in range(2):
            out = api.hip_w4a4_int8_matmul(*args, output_dtype=dt, out_features=N)
            torch.cuda.synchronize()
            got = from_dev(out)
            _assert_exact(got, want, f"tile {tile} gemm_persist={mode} call {call}")
        outs[mode] = got
    assert np.array_equal(outs[str(grid)], outs["0"])


@pytest.mark.parametrize("out_dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("M,K,N", [(300, 128, 264), (1000, 640, 1000), (520, 15360, 1000), (4608, 3072, 3072)])
def test_mfma32_tile(orc, dev, tuning, out_dtype, M, K, N):
    """The 4-wave 256x256 tile on 32x32x32 MFMAs (which the automatic plan runs when the
    tile's grid leaves CUs idle) forced on and off through gemm_mfma32: ragged edges, one and
    many k-blocks, every output bit-exact against the oracle both ways."""
    api = _api()
    tuning.set("gemm_tile", "256x256w2x2")
    tuning.set("gemm_sk", "0")
    tuning.set("gemm_smallm_max", "0")
    rng = np.random.default_rng(M + K + N + 32)
    a = rng.integers(-8, 8, size=(M, K), dtype=np.int8)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    xs = rng.uniform(0.01, 0.2, size=(M,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(N,)).astype(np.float32)
    b = rng.normal(size=(N,)).astype(np.float32)
    want = orc.w4a4_matmul_codes_large(a, w, xs, ws, b, out_dtype)
    args = (torch.from_numpy(a).to(dev), _dev_u8(orc.codes_to_cdna4(w), dev), torch.from_numpy(xs).to(dev),
            torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev))
    dt = {"bfloat16": torch.bfloat16, "float16": torch.float16}[out_dtype]
    for mode in ("1", "0"):
        tuning.set("gemm_mfma32", mode)
        out = api.hip_w4a4_int8_matmul(*args, output_dtype=dt, out_features=N)
        torch.cuda.synchronize()
        _assert_exact(from_dev(out), want, f"gemm_mfma32={mode}")
