"""GPU parity: W4A16 GEMM (tolerance), layout kernels (bit-exact) and the module contract."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import from_dev, normal_input, outlier_input, to_dev

pytestmark = pytest.mark.gpu


def _api():
    import convrot_mlx_amd as api

    return api


def _u8(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


# ---------------------------------------------------------------- W4A16

def _w4a16_check(orc, dev, act, act_dtype, w_codes, ws, b, out_dtype="float32"):
    """Float32 sums in any order: |got - ref| <= 2^-22 * K * sum|terms| * |ws| + 1 ulp of the output.

    The rigorous bound for any summation order is (K-1) * 2^-24 * sum_k |a_k w_k|; the factor
    used here is 4x that.  Outputs in bf16/f16 additionally allow one output ulp."""
    api = _api()
    N, K = w_codes.shape
    wq = _u8(orc.codes_to_cdna4(w_codes), dev)
    dt = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}[out_dtype]
    got = api.hip_w4a16_matmul(to_dev(act, act_dtype, dev), wq, torch.from_numpy(ws).to(dev),
                               torch.from_numpy(b).to(dev), output_dtype=dt, out_features=N)
    got = orc.to_f32(from_dev(got), out_dtype)
    ref, dots, mag = orc.w4a16_matmul_codes(act, act_dtype, w_codes, ws, b, "float32")
    tol = 2.0 ** -22 * K * mag * np.abs(ws)[None, :] + np.abs(ref) * 2.0 ** -22 + 1e-30
    if out_dtype != "float32":
        ulp = 2.0 ** -8 if out_dtype == "bfloat16" else 2.0 ** -11
        tol = tol + np.abs(ref) * ulp
    err = np.abs(got - ref)
    assert (err <= tol).all(), f"max excess {np.max(err - tol)} (max err {err.max()})"


@pytest.mark.parametrize("act_dtype", ["float16", "bfloat16"])
def test_w4a16_edges(orc, dev, act_dtype):
    """test_core.py:285-309: seed 2026082303, 37x64 activations, 46 outputs."""
    rng = np.random.default_rng(2026082303)
    w = rng.integers(-7, 8, size=(46, 64), dtype=np.int8)
    ws = rng.uniform(0.01, 0.2, size=(46,)).astype(np.float32)
    b = rng.normal(size=(46,)).astype(np.float32)
    act = orc.from_f32(rng.normal(size=(37, 64)).astype(np.float32), act_dtype)
    _w4a16_check(orc, dev, act, act_dtype, w, ws, b)


@pytest.mark.parametrize("M", [1, 8, 32])
@pytest.mark.parametrize("K,N", [(3072, 12288), (12288, 3072)])
def test_w4a16_config4(orc, dev, M, K, N):
    """benchmark config 4 shapes: small M, int4 weights with per-row scales, bf16 output."""
    rng = np.random.default_rng(M * 7 + K)
    w = rng.integers(-7, 8, size=(N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.01, size=(N,)).astype(np.float32)
    b = rng.normal(0, 0.02, size=(N,)).astype(np.float32)
    act = normal_input(M + K, (M, K), "bfloat16", orc)
    _w4a16_check(orc, dev, act, "bfloat16", w, ws, b, "bfloat16")


@pytest.mark.parametrize("M", [1, 8, 32])
@pytest.mark.parametrize("K,N", [(3072, 12288), (12288, 3072)])
def test_w4a16_config4_complete_path(orc, dev, M, K, N):
    """benchmark config 4 end to end through ConvRotLinear(backend="hip-w4a16"), G = 256:
    the weight quantized by the prep kernel (codes and scales bit-exact), the activations
    rotated by it (bit-exact against regular_hadamard), then the W4A16 GEMM within the
    float32-order tolerance of the oracle product of the oracle's rotation."""
    api = _api()
    G = 256
    x = outlier_input(M * 5 + K, (M, K), "bfloat16", orc)
    w = outlier_input(K + N, (N, K), "bfloat16", orc, std=0.02, frac=0.01, factor=10.0)
    bias = np.random.default_rng(K + N).normal(0.0, 0.02, size=N).astype(np.float32)
    xd = to_dev(x, "bfloat16", dev)
    qw, ws = api.quantize_convrot_weight(to_dev(w, "bfloat16", dev), G)
    layer = api.ConvRotLinear(K, N, group_size=G, backend="hip-w4a16", device=dev)
    layer.load_nk_weight(qw, ws, torch.from_numpy(bias).to(dev))
    got = orc.to_f32(from_dev(layer(xd)), "bfloat16")
    w_codes, wscales = orc.prepare_codes(w, "bfloat16", G)
    assert np.array_equal(orc.unpack_signed_int4(from_dev(qw)), w_codes)
    assert np.array_equal(from_dev(ws), wscales)
    rot = orc.regular_hadamard(x, "bfloat16", G)
    assert np.array_equal(from_dev(api.hip_fused_rotate_convrot_activation(xd, G)), rot)
    ref, _, mag = orc.w4a16_matmul_codes(rot, "bfloat16", w_codes, wscales, bias, "float32")
    tol = 2.0 ** -22 * K * mag * np.abs(wscales)[None, :] + np.abs(ref) * (2.0 ** -22 + 2.0 ** -8) + 1e-30
    err = np.abs(got - ref)
    assert (err <= tol).all(), f"max excess {np.max(err - tol)} (max err {err.max()})"


@pytest.mark.parametrize("cfg", ["A", "B", "C", "D", "E", "F", "T"])
@pytest.mark.parametrize("M,K,N", [(17, 96, 46), (37, 2688, 530), (1, 4000, 33), (5, 12288, 3072), (32, 3072, 1000)])
def test_w4a16_every_split(orc, dev, tuning, cfg, M, K, N):
    """Each W4A16 work split (forced through the w4a16_cfg tuning override) on ragged M/N and on K that is
    not a multiple of the 128-feature block (the tail features must read as zero)."""
    tuning.set("w4a16_cfg", cfg)
    rng = np.random.default_rng(M * 131 + K + N)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.01, size=(N,)).astype(np.float32)
    b = rng.normal(0, 0.02, size=(N,)).astype(np.float32)
    act = normal_input(M + K + N, (M, K), "bfloat16", orc)
    _w4a16_check(orc, dev, act, "bfloat16", w, ws, b, "bfloat16")


@pytest.mark.parametrize("cfg", ["A", "B", "D"])
@pytest.mark.parametrize("act_dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("K,N", [(3072, 12288), (2720, 530), (12288, 3072)])
def test_w4a16_load_orders_agree(orc, dev, tuning, cfg, act_dtype, K, N):
    """Splits A and B load activations in two orders: from 6 rows on, quad-coalesced reads that
    are transposed through LDS; below that, each lane reads its MFMA fragment directly.  Both
    feed the same MFMAs in the same order, so rows 0..3 of a 40-row launch (quad order, two
    token tiles) equal a 4-row launch (direct order) bit for bit; on the ragged shape the 40-row
    launch is also checked against the oracle (the config-4 shapes are, at M = 8 and 32, by
    test_w4a16_config4)."""
    api = _api()
    tuning.set("w4a16_cfg", cfg)
    rng = np.random.default_rng(K * 3 + N)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.01, size=(N,)).astype(np.float32)
    b = rng.normal(0, 0.02, size=(N,)).astype(np.float32)
    act = normal_input(K + N + 1, (40, K), act_dtype, orc)
    wq = _u8(orc.codes_to_cdna4(w), dev)
    wsd, bd = torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev)
    xd = to_dev(act, act_dtype, dev)
    many = api.hip_w4a16_matmul(xd, wq, wsd, bd, output_dtype=torch.float32, out_features=N)
    few = api.hip_w4a16_matmul(xd[:4].contiguous(), wq, wsd, bd, output_dtype=torch.float32, out_features=N)
    assert torch.equal(many[:4].view(torch.int32), few.view(torch.int32))
    if N < 1000:
        _w4a16_check(orc, dev, act, act_dtype, w, ws, b)


def _w4a16_tiled_case(orc, dev, act_dtype, out_dtype, M, K, N):
    rng = np.random.default_rng(M * 17 + K * 3 + N)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.01, size=(N,)).astype(np.float32)
    b = rng.normal(0, 0.02, size=(N,)).astype(np.float32)
    act = outlier_input(M + K + N, (M, K), act_dtype, orc)
    _w4a16_check(orc, dev, act, act_dtype, w, ws, b, out_dtype)


@pytest.mark.parametrize("tile", ["256x256", "256x128", "128x256", "128x128"])
@pytest.mark.parametrize("M,K,N", [(256, 128, 256), (300, 2688, 530), (1100, 4000, 2100), (129, 96, 8)])
def test_w4a16_tiled(orc, dev, tuning, tile, M, K, N):
    """Every tile of the tiled kernel (M >= 128, forced through the w4a16_tile tuning override): partial
    tiles in M and N, K ending inside a 128-feature block, more tiles than the eight-way XCD
    interleave covers, and an incomplete group of four tile rows."""
    tuning.set("w4a16_cfg", "T")
    tuning.set("w4a16_tile", tile)
    _w4a16_tiled_case(orc, dev, "bfloat16", "bfloat16", M, K, N)


@pytest.mark.parametrize("tile", ["256x256", "128x128"])
@pytest.mark.parametrize("act_dtype,out_dtype", [("bfloat16", "float32"), ("float16", "float16"),
                                                  ("float16", "bfloat16"), ("float16", "float32")])
def test_w4a16_tiled_dtypes(orc, dev, tuning, tile, act_dtype, out_dtype):
    """Activation and output dtypes of the tiled kernel on a ragged shape."""
    tuning.set("w4a16_cfg", "T")
    tuning.set("w4a16_tile", tile)
    _w4a16_tiled_case(orc, dev, act_dtype, out_dtype, 300, 2688, 530)


# ---------------------------------------------------------------- layouts

def test_pack_literal_bytes(orc, dev):
    """test_core.py:186-192."""
    api = _api()
    v = torch.tensor([[-8, -7, -1, 0, 1, 7, 3, -4]], dtype=torch.int8, device=dev)
    p = api.pack_signed_int4(v)
    assert p.cpu().tolist() == [[0x98, 0x0F, 0x71, 0xC3]]
    assert api.unpack_signed_int4(p).cpu().tolist() == v.cpu().tolist()


def test_unpack_matches_oracle(orc, dev):
    """test_core.py:194-201: seed 2026082300, 37x64 values in [-8, 8)."""
    api = _api()
    rng = np.random.default_rng(2026082300)
    v = rng.integers(-8, 8, size=(37, 64), dtype=np.int8)
    packed = orc.pack_signed_int4(v)
    assert np.array_equal(from_dev(api.pack_signed_int4(torch.from_numpy(v).to(dev))), packed)
    assert np.array_equal(from_dev(api.metal_unpack_signed_int4(_u8(packed, dev))), orc.unpack_signed_int4(packed))


@pytest.mark.parametrize("rows,cols,offset", [(4608, 1536, 0), (3, 16, 0), (5, 7, 0), (2, 32, 1)])
def test_unpack_kernels(orc, dev, rows, cols, offset):
    """Both unpack kernels: 16 packed bytes per thread (size a multiple of 16, aligned) and one
    byte per thread (ragged size, or a buffer starting off a 16-byte boundary), every byte
    value included."""
    api = _api()
    rng = np.random.default_rng(rows * 7 + cols)
    packed = rng.integers(0, 256, size=rows * cols + offset, dtype=np.uint8)
    packed[offset:offset + 256] = np.arange(256, dtype=np.uint8)[: min(256, rows * cols)]
    dev_buf = _u8(packed, dev)
    view = dev_buf[offset:].view(rows, cols)
    want = orc.unpack_signed_int4(packed[offset:].reshape(rows, cols))
    assert np.array_equal(from_dev(api.unpack_signed_int4(view)), want)


def test_mpp_repack_round_trip(orc, dev):
    """test_core.py:203-211: (46, 64) codes -> KN (64, 23) and back, bit-exact."""
    api = _api()
    rng = np.random.default_rng(2026082301)
    v = rng.integers(-7, 8, size=(46, 64), dtype=np.int8)
    nk = orc.pack_signed_int4(v)
    kn = api.repack_nk_weight_for_mpp(_u8(nk, dev))
    assert tuple(kn.shape) == (64, 23)
    assert np.array_equal(from_dev(kn), orc.repack_nk_weight_for_mpp(nk))
    assert np.array_equal(from_dev(api.repack_mpp_weight_to_nk(kn)), nk)


@pytest.mark.parametrize("N,K", [(46, 64), (33, 256), (3072, 3072), (21504, 3072), (17, 2688)])
def test_cdna4_repack_round_trips(orc, dev, N, K):
    api = _api()
    rng = np.random.default_rng(N + K)
    v = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    nk = orc.pack_signed_int4(v)
    c4 = api.repack_nk_weight_for_cdna4(_u8(nk, dev))
    assert np.array_equal(from_dev(c4), orc.codes_to_cdna4(v))
    assert np.array_equal(from_dev(api.repack_cdna4_weight_to_nk(c4, N, K)), nk)
    if N % 2 == 0:
        kn = orc.repack_nk_weight_for_mpp(nk)
        c4b = api.repack_mpp_weight_for_cdna4(_u8(kn, dev))
        assert np.array_equal(from_dev(c4b), from_dev(c4))
        assert np.array_equal(from_dev(api.repack_cdna4_weight_to_mpp(c4, N, K)), kn)


# ---------------------------------------------------------------- module

def _layer_reference(orc, x, dense_w, dense_b, G, dtype="bfloat16"):
    w_codes, wscales = orc.prepare_codes(dense_w, dtype, G)
    a_codes, xscales = orc.prepare_codes(x, dtype, G)
    return orc.w4a4_matmul_codes(a_codes, w_codes, xscales, wscales, dense_b, dtype)


@pytest.mark.parametrize("backend", ["hip-w4a4", "hip-w4a16"])
def test_default_backend_takes_reference_assignment(orc, dev, backend):
    """Reference code assigns a K x packed-N qweight (test_core.py:375-402's layer set-up); on the
    hip-* backends that runs on a cached CDNA4 repack, with the same output bits as load_nk_weight."""
    api = _api()
    rng = np.random.default_rng(31)
    n = 34
    dense_w = orc.from_f32(rng.normal(size=(n, 256)).astype(np.float32), "bfloat16")
    dense_b = torch.from_numpy(rng.normal(size=(n,)).astype(np.float32)).to(dev)
    values = to_dev(orc.from_f32(rng.normal(size=(2, 7, 256)).astype(np.float32), "bfloat16"), "bfloat16", dev)
    qweight, wscales = api.quantize_convrot_weight(to_dev(dense_w, "bfloat16", dev))
    ref_layer = api.ConvRotLinear(256, n, backend=backend, device=dev)
    ref_layer.load_nk_weight(qweight, wscales, dense_b)
    layer = api.ConvRotLinear(256, n, backend=backend, device=dev)
    layer.qweight = api.repack_nk_weight_for_mpp(qweight)
    layer.scales = wscales
    layer.bias = dense_b
    assert layer.qweight.ndim == 2 and layer.backend == backend
    assert torch.equal(layer(values), ref_layer(values))
    layer.qweight = api.repack_nk_weight_for_mpp(torch.zeros_like(qweight))  # a new tensor: the repack follows
    out = layer(values)
    assert torch.equal(out, dense_b.to(torch.bfloat16).expand_as(out))  # zero codes: bias alone


@pytest.mark.parametrize("backend", ["hip-w4a4", "mpp-w4a4"])
def test_layer_matches_contract_bf16(orc, dev, backend):
    """test_core.py:375-402: (2,7,256) -> 33 (34 for the even-N mpp layout), seed 29, bit-exact."""
    api = _api()
    n = 33 if backend == "hip-w4a4" else 34
    rng = np.random.default_rng(29)
    dense_w = orc.from_f32(rng.normal(size=(n, 256)).astype(np.float32), "bfloat16")
    dense_b = rng.normal(size=(n,)).astype(np.float32)
    values = orc.from_f32(rng.normal(size=(2, 7, 256)).astype(np.float32), "bfloat16")
    qweight, wscales = api.quantize_convrot_weight(to_dev(dense_w, "bfloat16", dev))
    layer = api.ConvRotLinear(256, n, backend=backend, device=dev)
    if backend == "mpp-w4a4":
        layer.qweight = api.repack_nk_weight_for_mpp(qweight)  # the reference's assignment style
        layer.scales = wscales
        layer.bias = torch.from_numpy(dense_b).to(dev)
    else:
        layer.load_nk_weight(qweight, wscales, torch.from_numpy(dense_b).to(dev))
    out = layer(to_dev(values, "bfloat16", dev))
    assert tuple(out.shape) == (2, 7, n) and out.dtype == torch.bfloat16
    expected = _layer_reference(orc, values.reshape(-1, 256), dense_w, dense_b, 256)
    assert np.array_equal(from_dev(out).reshape(-1, n), expected)


@pytest.mark.parametrize("backend", ["hip-w4a16", "mpp-w4a16"])
def test_w4a16_layer_group64_k2688(orc, dev, backend):
    """test_core.py:427-448: G=64 at K=2688, (2,7,2688) -> 34; checked against the oracle."""
    api = _api()
    rng = np.random.default_rng(2026082306)
    dense_w = orc.from_f32(rng.normal(size=(34, 2688)).astype(np.float32), "bfloat16")
    dense_b = rng.normal(size=(34,)).astype(np.float32)
    values = orc.from_f32(rng.normal(size=(2, 7, 2688)).astype(np.float32), "bfloat16")
    qweight, wscales = api.quantize_convrot_weight(to_dev(dense_w, "bfloat16", dev), 64)
    layer = api.ConvRotLinear(2688, 34, group_size=64, backend=backend, device=dev)
    layer.load_nk_weight(qweight, wscales, torch.from_numpy(dense_b).to(dev))
    out = layer(to_dev(values, "bfloat16", dev))
    assert tuple(out.shape) == (2, 7, 34)
    rot = orc.regular_hadamard(values.reshape(-1, 2688), "bfloat16", 64)
    w_codes, ws = orc.prepare_codes(dense_w, "bfloat16", 64)
    ref, _, mag = orc.w4a16_matmul_codes(rot, "bfloat16", w_codes, ws, dense_b, "float32")
    got = orc.to_f32(from_dev(out).reshape(-1, 34), "bfloat16")
    tol = 2.0 ** -22 * 2688 * mag * ws[None, :] + np.abs(ref) * 2.0 ** -8
    assert (np.abs(got - ref) <= tol).all()


_MANY_TOKENS = {}


def _many_tokens_case(orc, K, N):
    """Inputs and oracle of the many-token layer test (computed once per session)."""
    if (K, N) not in _MANY_TOKENS:
        rng = np.random.default_rng(20260823)
        dense_w = orc.from_f32((rng.normal(size=(N, K)) * 0.02).astype(np.float32), "bfloat16")
        dense_b = (rng.normal(size=(N,)) * 0.02).astype(np.float32)
        values = outlier_input(31, (2, 256, K), "bfloat16", orc)
        rot = orc.regular_hadamard(values.reshape(-1, K), "bfloat16", 64)
        w_codes, ws = orc.prepare_codes(dense_w, "bfloat16", 64)
        ref, _, mag = orc.w4a16_matmul_codes(rot, "bfloat16", w_codes, ws, dense_b, "float32")
        _MANY_TOKENS[(K, N)] = (dense_w, dense_b, values, ws, ref, mag)
    return _MANY_TOKENS[(K, N)]


@pytest.mark.parametrize("cfg", [None, "T", "F"], ids=["auto", "tiled", "split"])
def test_w4a16_layer_many_tokens(orc, dev, tuning, cfg):
    """ConvRotLinear (hip-w4a16) at 512 tokens, 1024 -> 3072, G=64: the automatic dispatch
    (the tiled kernel at this size) and each kernel forced, against the oracle."""
    api = _api()
    if cfg is None:
        tuning.set("w4a16_cfg", None)
    else:
        tuning.set("w4a16_cfg", cfg)
    tuning.set("w4a16_tile", None)
    K, N = 1024, 3072
    dense_w, dense_b, values, ws, ref, mag = _many_tokens_case(orc, K, N)
    qweight, wscales = api.quantize_convrot_weight(to_dev(dense_w, "bfloat16", dev), 64)
    layer = api.ConvRotLinear(K, N, group_size=64, backend="hip-w4a16", device=dev)
    layer.load_nk_weight(qweight, wscales, torch.from_numpy(dense_b).to(dev))
    out = layer(to_dev(values, "bfloat16", dev))
    assert tuple(out.shape) == (2, 256, N) and out.dtype == torch.bfloat16
    got = orc.to_f32(from_dev(out).reshape(-1, N), "bfloat16")
    tol = 2.0 ** -22 * K * mag * ws[None, :] + np.abs(ref) * 2.0 ** -8
    assert (np.abs(got - ref) <= tol).all(), f"max excess {np.max(np.abs(got - ref) - tol)}"


def test_w4a4_layer_group64_k2688(orc, dev):
    api = _api()
    rng = np.random.default_rng(2026082306)
    dense_w = orc.from_f32(rng.normal(size=(34, 2688)).astype(np.float32), "bfloat16")
    dense_b = rng.normal(size=(34,)).astype(np.float32)
    values = orc.from_f32(rng.normal(size=(2, 7, 2688)).astype(np.float32), "bfloat16")
    qweight, wscales = api.quantize_convrot_weight(to_dev(dense_w, "bfloat16", dev), 64)
    layer = api.ConvRotLinear(2688, 34, group_size=64, backend="mpp-w4a4", device=dev)
    layer.qweight = api.repack_nk_weight_for_mpp(qweight)
    layer.scales = wscales
    layer.bias = torch.from_numpy(dense_b).to(dev)
    out = layer(to_dev(values, "bfloat16", dev))
    expected = _layer_reference(orc, values.reshape(-1, 2688), dense_w, dense_b, 64)
    assert np.array_equal(from_dev(out).reshape(-1, 34), expected)


def test_config1_end_to_end(orc, dev):
    """benchmark config 1: K=N=1024, M=64, G=64, W~N(0,0.02^2), X~N(0,1), no bias, seed 0."""
    api = _api()
    rng = np.random.default_rng(0)
    w = orc.from_f32(rng.normal(0.0, 0.02, size=(1024, 1024)).astype(np.float32), "bfloat16")
    x = orc.from_f32(rng.normal(size=(64, 1024)).astype(np.float32), "bfloat16")
    qw, ws = api.quantize_convrot_weight(to_dev(w, "bfloat16", dev), 64)
    layer = api.ConvRotLinear(1024, 1024, bias=False, group_size=64, device=dev).load_nk_weight(qw, ws)
    out = layer(to_dev(x, "bfloat16", dev))
    expected = _layer_reference(orc, x, w, np.zeros(1024, np.float32), 64)
    assert np.array_equal(from_dev(out), expected)
