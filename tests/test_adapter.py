"""Model integration on the CPU: the torch FLUX DiT topology and `replace_convrot_linears`.

Covers what needs no kernel: which Linears are eligible, how many are replaced
(the reference FLUX adapter's count, /root/reference/docs/benchmarks/m4-pro.md:40
reports 313 at group 256), that replacement keeps the module tree loadable, and
the dense forward's shapes.  Numerics of the converted model run under the
`gpu` marker (test_gpu_adapter.py).
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

from examples.flux1_dev.dit import Flux, FluxParams, build, make_inputs


def _tiny(**kw) -> FluxParams:
    base = dict(in_channels=64, vec_in_dim=64, context_in_dim=128, hidden_size=128, mlp_ratio=4.0,
                num_heads=2, depth=2, depth_single_blocks=3, axes_dim=(8, 28, 28))
    base.update(kw)
    return FluxParams(**base)


def _linears(model: nn.Module) -> list[tuple[str, nn.Linear]]:
    return [(n, m) for n, m in model.named_modules() if isinstance(m, nn.Linear)]


def test_flux_dev_linear_census():
    """The full FLUX.1-dev topology on the meta device: 314 Linears, 313 of them with in_features
    divisible by 256 (img_in's 64 is the one exception), all 314 at group 64."""
    with torch.device("meta"):
        model = Flux(FluxParams())
    linears = _linears(model)
    assert len(linears) == 314
    g256 = [n for n, m in linears if m.in_features % 256 == 0]
    assert len(g256) == 313 and "img_in" not in g256
    assert all(m.in_features % 64 == 0 for _, m in linears)
    shapes = {(m.in_features, m.out_features) for _, m in linears}
    # the benchmark FLUX linear shapes all occur in the model
    for shape in [(3072, 9216), (3072, 3072), (3072, 12288), (12288, 3072), (3072, 21504), (15360, 3072)]:
        assert shape in shapes
    params = sum(p.numel() for p in model.parameters())
    assert 11.8e9 < params < 12.0e9


@pytest.mark.parametrize("group_size", [64, 256])
def test_replace_counts_and_names(group_size):
    from convrot_mlx_amd import ConvRotLinear, eligible_linear, replace_convrot_linears

    model = build(_tiny(hidden_size=256, context_in_dim=256, vec_in_dim=256, axes_dim=(16, 56, 56)), "cpu")
    before = _linears(model)
    want = [n for n, m in before if eligible_linear(m, group_size)]
    names = replace_convrot_linears(model, group_size=group_size, convert=False)
    assert names == want
    assert len(names) == (len(before) if group_size == 64 else len(before) - 1)
    after = dict(model.named_modules())
    for name, dense in before:
        layer = after[name]
        if name in names:
            assert isinstance(layer, ConvRotLinear)
            assert (layer.in_features, layer.out_features) == (dense.in_features, dense.out_features)
            assert layer.source_has_bias == (dense.bias is not None)
            assert layer.group_size == group_size
        else:
            assert layer is dense
    # convert=False leaves the reference's initial parameters: ones scales, zero bias
    layer = after[names[0]]
    assert torch.equal(layer.scales, torch.ones_like(layer.scales))
    assert torch.equal(layer.bias, torch.zeros_like(layer.bias))
    # state-dict keys follow the reference's checkpoint naming: {name}.qweight/.scales/.bias
    keys = model.state_dict().keys()
    for name in names:
        assert {f"{name}.qweight", f"{name}.scales", f"{name}.bias"} <= keys


def test_replace_sequential_children_in_place():
    from convrot_mlx_amd import ConvRotLinear, replace_convrot_linears

    model = nn.Sequential(nn.Linear(128, 64), nn.GELU(), nn.Sequential(nn.Linear(64, 32, bias=False)),
                          nn.Linear(48, 16))
    names = replace_convrot_linears(model, group_size=64, convert=False, backend="hip-w4a16")
    assert names == ["0", "2.0"]
    assert isinstance(model[0], ConvRotLinear) and isinstance(model[2][0], ConvRotLinear)
    assert isinstance(model[3], nn.Linear) and not isinstance(model[3], ConvRotLinear)
    assert model[0].backend == "hip-w4a16" and not model[2][0].source_has_bias


def test_tiny_dense_forward_shapes():
    p = _tiny()
    model = build(p, "cpu")
    inputs = make_inputs(p, img_tokens=16, txt_tokens=8, device="cpu")
    with torch.no_grad():
        out = model(**inputs)
    assert out.shape == (1, 16, p.in_channels) and out.dtype == torch.bfloat16
    assert torch.isfinite(out.float()).all()
