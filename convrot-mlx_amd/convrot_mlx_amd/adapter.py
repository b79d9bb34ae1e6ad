"""Model integration: swap eligible torch Linears for ConvRotLinear.

torch counterpart of the reference's FLUX adapter and converter
(/root/reference/examples/flux1_dev/adapter.py:45-70 `replace_convrot_linears`,
convert.py:111-141 per-linear quantization): every `nn.Linear` whose
in_features divide into ConvRot groups (`eligible_linear`, core.py:1316-1321)
becomes a `ConvRotLinear` of the same shape.  With `convert=True` the dense
weight is quantized on the GPU by the fused prep kernel
(`quantize_convrot_weight`, the same rotation + A4 contract as the
activations) and the bias is stored as float32 (zeros when the source had
none), as convert.py:126-134 writes them; ineligible Linears keep their
source weights.
"""

from __future__ import annotations

import torch
from torch import nn

from .core import CONVROT_GROUP_SIZE, ConvRotLinear, eligible_linear, quantize_convrot_weight


def _set_submodule(root: nn.Module, name: str, module: nn.Module) -> None:
    parent_name, _, child = name.rpartition(".")
    parent = root.get_submodule(parent_name) if parent_name else root
    setattr(parent, child, module)


def replace_convrot_linears(
    model: nn.Module,
    *,
    backend: str | None = None,
    preprocessor: str | None = None,
    group_size: int = CONVROT_GROUP_SIZE,
    convert: bool = True,
) -> list[str]:
    """Replace every eligible Linear of `model` in place; return the replaced names in
    `named_modules` order (adapter.py:45-70).

    convert=False installs layers with the reference's initial parameters (zero weights,
    unit scales, zero bias) for loading a converted checkpoint afterwards; convert=True
    quantizes each dense weight on its device (which must be a GPU: there is no CPU path).
    """
    selected = [(name, module) for name, module in model.named_modules()
                if name and eligible_linear(module, group_size)]
    names = []
    for name, dense in selected:
        out_features, in_features = dense.weight.shape
        layer = ConvRotLinear(in_features, out_features, bias=dense.bias is not None, group_size=group_size,
                              backend=backend, preprocessor=preprocessor, device=dense.weight.device)
        if convert:
            with torch.no_grad():
                qweight, scales = quantize_convrot_weight(dense.weight.detach(), group_size)
                bias = (dense.bias.detach().to(torch.float32) if dense.bias is not None
                        else torch.zeros(out_features, dtype=torch.float32, device=dense.weight.device))
                layer.load_nk_weight(qweight, scales, bias)
        _set_submodule(model, name, layer)
        names.append(name)
    return names
