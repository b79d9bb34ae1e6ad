"""CPU: the Python API mirrors the reference's contract (names, defaults, attributes,
validation messages of /root/reference/src/convrot_mlx/core.py) and refuses to compute
anywhere but on a ROCm device -- there is no CPU fallback."""

from __future__ import annotations

import pytest
import torch

import convrot_mlx_amd as api


def test_public_names_cover_the_reference_api():
    ref_names = {  # /root/reference/src/convrot_mlx/__init__.py:41-75, minus oracle/legacy/expanded backends
        "CONVROT_GROUP_SIZE", "INT4_MAX", "SUPPORTED_BACKENDS", "SUPPORTED_FUSED_GROUP_SIZES",
        "SUPPORTED_PREPROCESSORS", "ConvRotLinear", "compiled_prepare_convrot_activation",
        "compiled_regular_hadamard", "eligible_linear", "metal_fused_prepare_convrot_activation",
        "metal_fused_prepare_convrot_activation_i8", "metal_fused_rotate_convrot_activation",
        "metal_unpack_signed_int4", "mpp_w4a4_int8_matmul", "mpp_w4a4_matmul", "mpp_w4a16_matmul",
        "pack_signed_int4", "prepare_convrot_activation", "quantize_convrot_weight",
        "quantize_signed_int4_rowwise", "regular_hadamard", "repack_mpp_weight_to_nk",
        "repack_nk_weight_for_mpp", "unpack_signed_int4",
    }
    assert ref_names <= set(api.__all__)
    assert api.CONVROT_GROUP_SIZE == 256 and api.INT4_MAX == 7
    assert {64, 256} <= api.SUPPORTED_FUSED_GROUP_SIZES


def test_layer_defaults_and_attributes(monkeypatch):
    monkeypatch.delenv("CONVROT_BACKEND", raising=False)
    monkeypatch.delenv("CONVROT_MLX_BACKEND", raising=False)
    layer = api.ConvRotLinear(512, 33, device="meta")
    assert layer.backend == "hip-w4a4" and layer.group_size == 256 and layer.source_has_bias
    assert layer.weight_layout == api.WEIGHT_LAYOUT_CDNA4
    assert tuple(layer.qweight.shape) == (4, 3, 1024) and layer.qweight.dtype == torch.uint8
    assert layer.scales.dtype == torch.float32 and tuple(layer.scales.shape) == (33,)
    assert layer.bias.dtype == torch.float32 and tuple(layer.bias.shape) == (33,)
    assert set(layer.state_dict()) == {"qweight", "scales", "bias"}
    mpp = api.ConvRotLinear(256, 34, bias=False, backend="mpp-w4a4", device="meta")
    assert tuple(mpp.qweight.shape) == (256, 17) and mpp.weight_layout == "packed-kn-low-nibble-even-output"
    assert not mpp.source_has_bias


def test_reference_env_var_selects_backend(monkeypatch):
    monkeypatch.delenv("CONVROT_BACKEND", raising=False)
    monkeypatch.setenv("CONVROT_MLX_BACKEND", "mpp-w4a16")
    assert api.ConvRotLinear(256, 8, device="meta").backend == "mpp-w4a16"
    monkeypatch.setenv("CONVROT_MLX_BACKEND", "bogus")
    with pytest.raises(ValueError, match=r"Unknown ConvRot backend 'bogus'; expected one of"):
        api.ConvRotLinear(256, 8, device="meta")


@pytest.mark.parametrize(
    "kwargs,msg",
    [
        (dict(in_features=100, out_features=8), "in_features 100 not divisible by ConvRot group size 256"),
        (dict(in_features=256, out_features=8, backend="metal"), "Unknown ConvRot backend 'metal'"),
        (dict(in_features=256, out_features=8, preprocessor="x"), "Unknown ConvRot preprocessor 'x'"),
        (dict(in_features=256, out_features=33, backend="mpp-w4a4"), "MPP packed weights require even out_features, got 33"),
        (dict(in_features=256, out_features=8, group_size=128), "Regular Hadamard size must be a power of 4, got 128"),
    ],
)
def test_layer_constructor_validation(kwargs, msg):
    with pytest.raises(ValueError, match=msg.replace("[", r"\[")):
        api.ConvRotLinear(device="meta", **kwargs)


def test_forward_checks_features_first():
    layer = api.ConvRotLinear(256, 8, device="meta")
    with pytest.raises(ValueError, match="ConvRotLinear expected K=256, got 128"):
        layer(torch.empty(3, 128, device="meta"))


def test_no_cpu_fallback():
    layer = api.ConvRotLinear(256, 8)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        layer(torch.zeros(2, 256, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        api.hip_fused_prepare_convrot_activation(torch.zeros(2, 256, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        api.pack_signed_int4(torch.zeros(2, 8, dtype=torch.int8))


def test_functional_validation_messages():
    x = torch.empty(4, 512, dtype=torch.bfloat16, device="meta")
    with pytest.raises(ValueError, match=r"expects 2D input, got \(512,\)"):
        api.hip_fused_prepare_convrot_activation(torch.empty(512, device="meta"))
    with pytest.raises(ValueError, match="features 512 not divisible by ConvRot group size 1024"):
        api.hip_fused_prepare_convrot_activation(x, 1024)
    with pytest.raises(ValueError, match="Regular Hadamard size must be a power of 4, got 32"):
        api.regular_hadamard(x, 32)
    with pytest.raises(ValueError, match="last dimension must be even, got 7"):
        api.pack_signed_int4(torch.empty(2, 7, dtype=torch.int8, device="meta"))
    with pytest.raises(ValueError, match="MPP int4 packing requires even out_features, got 5"):
        api.repack_nk_weight_for_mpp(torch.empty(5, 8, dtype=torch.uint8, device="meta"))
    with pytest.raises(ValueError, match=r"MPP W4 weight must use K x packed-N layout; activation K=64"):
        api.mpp_w4a4_int8_matmul(torch.empty(3, 64, dtype=torch.int8, device="meta"),
                                 torch.empty(32, 23, dtype=torch.uint8, device="meta"),
                                 None, None, None, output_dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="MPP W4A4 requires a 2D int8 activation"):
        api.mpp_w4a4_int8_matmul(torch.empty(3, 64, dtype=torch.uint8, device="meta"), None, None, None, None,
                                 output_dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="MPP W4A16 requires float16 or bfloat16 activation"):
        api.mpp_w4a16_matmul(torch.empty(3, 64, device="meta"), None, None, None, output_dtype=torch.bfloat16)
    with pytest.raises(ValueError, match=r"MPP weight scales must have shape \(46,\)"):
        api.mpp_w4a16_matmul(torch.empty(3, 64, dtype=torch.bfloat16, device="meta"),
                             torch.empty(64, 23, dtype=torch.uint8, device="meta"),
                             torch.empty(45, device="meta"), torch.empty(46, device="meta"),
                             output_dtype=torch.bfloat16)


def test_eligible_linear():
    assert api.eligible_linear(torch.nn.Linear(512, 8))
    assert not api.eligible_linear(torch.nn.Linear(500, 8))
    assert api.eligible_linear(torch.nn.Linear(192, 8), 64)
    assert not api.eligible_linear(torch.nn.Conv1d(4, 4, 1))


def test_fp6_operand_policy():
    """FP6 operands (same bits as INT8, twice the MFMA rate) are used by ConvRotLinear at
    FP6_MIN_ROWS rows and above with in_features % 128 == 0 (below 262144); set_fp6_operands
    switches the path off and on."""
    was = api.fp6_operands_enabled()
    try:
        api.set_fp6_operands(True)
        m = api.core.FP6_MIN_ROWS
        assert api.fp6_eligible(4608, 12288, 3072, torch.bfloat16)
        assert api.fp6_eligible(m, 3076, 3072, torch.float16)  # any N
        assert api.fp6_eligible(m, 3072, 3072, torch.float32)
        assert not api.fp6_eligible(m - 1, 3072, 3072, torch.bfloat16)  # few rows: INT8 weight streaming
        assert not api.fp6_eligible(4608, 3072, 3072 + 64, torch.bfloat16)  # K % 128
        assert not api.fp6_eligible(4608, 3072, 262144, torch.bfloat16)  # sums no longer exact in float32
        api.set_fp6_operands(False)
        assert not api.fp6_eligible(4608, 12288, 3072, torch.bfloat16)
    finally:
        api.set_fp6_operands(was)


def test_fp6_functional_validation():
    """The FP6 entry points check shapes before any launch (and never compute on the CPU)."""
    a6 = torch.zeros(api.core.fp6_shape(300, 256), dtype=torch.uint8)
    w6 = torch.zeros(api.core.fp6_shape(64, 256), dtype=torch.uint8)
    xs, ws, b = torch.ones(300), torch.ones(64), torch.zeros(64)
    with pytest.raises(ValueError, match="K % 128"):
        api.hip_w4a4_fp6_matmul(a6, w6, xs, ws, b, output_dtype=torch.bfloat16, rows=300, out_features=64,
                                in_features=192)
    with pytest.raises(ValueError, match="float32, float16 or bfloat16"):
        api.hip_w4a4_fp6_matmul(a6, w6, xs, ws, b, output_dtype=torch.float64, rows=300, out_features=64,
                                in_features=256)
    with pytest.raises(ValueError, match="gate and inplace need a residual"):
        api.hip_w4a4_fp6_matmul(a6, w6, xs, ws, b, output_dtype=torch.bfloat16, rows=300, out_features=64,
                                in_features=256, inplace=True)
    with pytest.raises(ValueError, match="FP6 operands must be"):
        api.hip_w4a4_fp6_matmul(a6, w6, xs, ws, b, output_dtype=torch.bfloat16, rows=400, out_features=64,
                                in_features=256)
    with pytest.raises(ValueError, match="divisible by 128"):
        api.hip_fused_prepare_convrot_activation_fp6(torch.zeros(4, 64, dtype=torch.bfloat16), 64)
    with pytest.raises(ValueError, match="divisible by 128"):
        api.fp6_weight(torch.zeros((1, 4, 1024), dtype=torch.uint8), 64, 192)
    with pytest.raises(Exception):
        api.hip_w4a4_fp6_matmul(a6, w6, xs, ws, b, output_dtype=torch.bfloat16, rows=300, out_features=64,
                                in_features=256)  # CPU tensors: no fallback
