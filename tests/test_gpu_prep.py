"""GPU parity: fused preparation kernel vs the CPU oracle, bit for bit.

Seeds and shapes follow /root/reference/tests/test_core.py (:54-137), plus
the benchmark FLUX shapes, every supported group size and dtype, and edge rows.
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


def _check_prepare(orc, dev, x, dtype, G, label):
    api = _api()
    xd = to_dev(x, dtype, dev)
    codes, scales = orc.prepare_codes(x, dtype, G)
    q, s = api.hip_fused_prepare_convrot_activation(xd, G)
    q8, s8 = api.hip_fused_prepare_convrot_activation_i8(xd, G)
    torch.cuda.synchronize()
    got_codes = orc.unpack_signed_int4(from_dev(q))
    assert np.array_equal(from_dev(s), scales), f"{label}: scales differ ({int((from_dev(s) != scales).sum())} rows)"
    assert np.array_equal(from_dev(s8), scales), f"{label}: int8-mode scales differ"
    bad = int((got_codes != codes).sum())
    assert bad == 0, f"{label}: {bad} packed codes differ of {codes.size}"
    bad8 = int((from_dev(q8) != codes).sum())
    assert bad8 == 0, f"{label}: {bad8} int8 codes differ of {codes.size}"
    assert np.array_equal(from_dev(q), orc.pack_signed_int4(codes)), f"{label}: packed bytes differ"


def _check_rotate(orc, dev, x, dtype, G, label):
    api = _api()
    expected = orc.regular_hadamard(x, dtype, G)
    got = from_dev(api.hip_fused_rotate_convrot_activation(to_dev(x, dtype, dev), G))
    if dtype == "float32":
        assert np.array_equal(got.view(np.uint32), expected.view(np.uint32)), label
    else:
        bad = int((got != expected).sum())
        assert bad == 0, f"{label}: {bad} rotated values differ"


@pytest.mark.parametrize("seed", [18, 1801, 1802, 17])
def test_reference_seeds_19x512_g256(orc, dev, seed):
    x = normal_input(seed, (19, 512), "bfloat16", orc)
    _check_prepare(orc, dev, x, "bfloat16", 256, f"seed {seed}")
    _check_rotate(orc, dev, x, "bfloat16", 256, f"seed {seed}")


def test_group64_h3_k2688(orc, dev):
    """test_core.py:98-126: G=64 at K=2688, M=17, seed 2026082305."""
    x = normal_input(2026082305, (17, 2688), "bfloat16", orc)
    _check_prepare(orc, dev, x, "bfloat16", 64, "h3 k2688")
    _check_rotate(orc, dev, x, "bfloat16", 64, "h3 k2688")


def test_route_shape_1536x3072(orc, dev):
    """test_core.py:128-137: route shape 1536x3072, G=256, seed 20260823."""
    x = normal_input(20260823, (1536, 3072), "bfloat16", orc)
    _check_prepare(orc, dev, x, "bfloat16", 256, "route shape")


@pytest.mark.parametrize("G", [4, 16, 64, 256, 1024])
@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_groups_and_dtypes(orc, dev, G, dtype):
    x = normal_input(7000 + G, (23, 2048), dtype, orc)
    _check_prepare(orc, dev, x, dtype, G, f"G={G} {dtype}")
    _check_rotate(orc, dev, x, dtype, G, f"G={G} {dtype}")


@pytest.mark.parametrize(
    "M,K,G",
    [(64, 1024, 64), (37, 3072, 64), (29, 3072, 256), (11, 12288, 64), (9, 12288, 256), (13, 15360, 256),
     (5, 64, 64), (3, 256, 256), (4, 65536, 256), (6, 21504 - 21504 % 256, 256)],
)
def test_baseline_feature_counts(orc, dev, M, K, G):
    """Every K of the benchmark configs (single- and multi-wave rows), heavy-tailed inputs."""
    x = outlier_input(M * 131 + K, (M, K), "bfloat16", orc)
    _check_prepare(orc, dev, x, "bfloat16", G, f"M={M} K={K} G={G}")


def test_flux_m4608_k3072_g256(orc, dev):
    """Config 3 activation shape at full size, outlier channels x20."""
    x = outlier_input(3, (4608, 3072), "bfloat16", orc)
    _check_prepare(orc, dev, x, "bfloat16", 256, "4608x3072")


def test_zero_and_constant_rows(orc, dev):
    x = normal_input(5, (8, 512), "bfloat16", orc)
    x[0] = 0  # all-zero row: scale = bf16(1e-10)/7, codes 0
    x[1] = orc.from_f32(np.full(512, 3.0, np.float32), "bfloat16")
    x[2, ::2] = orc.from_f32(np.full(256, -1e-3, np.float32), "bfloat16")
    _check_prepare(orc, dev, x, "bfloat16", 256, "edge rows")
    _check_prepare(orc, dev, x, "bfloat16", 64, "edge rows g64")


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_quantize_without_rotation(orc, dev, dtype):
    """quantize_signed_int4_rowwise (core.py:149-158), as test_core.py:311-327 uses it."""
    api = _api()
    x = normal_input(23, (19, 256), dtype, orc)
    q, s = api.quantize_signed_int4_rowwise(to_dev(x, dtype, dev))
    codes, scales = orc.quantize_rowwise_codes(x, dtype)
    assert np.array_equal(from_dev(s), scales)
    assert np.array_equal(orc.unpack_signed_int4(from_dev(q)), codes)


@pytest.mark.parametrize("features", [2, 6, 34, 250])
def test_quantize_without_rotation_any_even_features(orc, dev, features):
    """quantize_signed_int4_rowwise accepts any even row length, as the reference does
    (core.py:97-100,149-158): rows not a multiple of 16 long are padded with zeros on the
    device; codes and scales equal the oracle's bit for bit, with extreme rows (all zero, one
    outlier) included."""
    api = _api()
    x = normal_input(29 + features, (7, features), "bfloat16", orc)
    x[0] = 0
    x[1, -1] = orc.from_f32(np.array([300.0], np.float32), "bfloat16")[0]
    q, s = api.quantize_signed_int4_rowwise(to_dev(x, "bfloat16", dev))
    codes, scales = orc.quantize_rowwise_codes(x, "bfloat16")
    assert q.shape == (7, features // 2)
    assert np.array_equal(from_dev(s), scales)
    assert np.array_equal(orc.unpack_signed_int4(from_dev(q)), codes)


def test_regular_hadamard_any_leading_shape(orc, dev):
    api = _api()
    x = normal_input(9, (2, 3, 7, 256), "bfloat16", orc)
    got = from_dev(api.regular_hadamard(to_dev(x, "bfloat16", dev), 64))
    assert np.array_equal(got.reshape(-1, 256), orc.regular_hadamard(x.reshape(-1, 256), "bfloat16", 64))


def test_weight_quantization_matches_oracle(orc, dev):
    """quantize_convrot_weight (core.py:514-527) on a FLUX-sized weight slice with outlier inputs."""
    api = _api()
    w = outlier_input(11, (512, 3072), "bfloat16", orc, std=0.02, frac=0.01, factor=10.0)
    q, s = api.quantize_convrot_weight(to_dev(w, "bfloat16", dev), 64)
    codes, scales = orc.prepare_codes(w, "bfloat16", 64)
    assert np.array_equal(from_dev(s), scales)
    assert np.array_equal(orc.unpack_signed_int4(from_dev(q)), codes)
