"""Benchmark config 5 at full size on the GPU: the random-init FLUX.1-dev DiT (19 double-stream +
38 single-stream blocks, hidden 3072, 24 heads x 128, MLP ratio 4) with every eligible Linear
replaced by a W4A4 ConvRotLinear at G = 64, one step on 1024 image + 512 text tokens.

The reference pins its route at full shape (/root/reference/tests/test_core.py:128-137,375-402):
here a sample of the converted layers -- the M = 1 modulation and embedder rows, the text and
image streams' projections, both single-block linears and the final layer -- must reproduce the
oracle's W4A4 linear bit for bit on the activations the model feeds them (every weight code and
scale, every output), the whole step must stay within a relative-L2 / cosine bound of the dense
bf16 step, and repeated steps must be bit-identical.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch import nn

from _util import from_dev
from examples.flux1_dev.dit import FluxParams, build, make_inputs

pytestmark = pytest.mark.gpu

G = 64
# (module name, rows the model feeds it at 1024 image + 512 text tokens)
SAMPLED = {
    "time_in.in_layer": 1,
    "guidance_in.out_layer": 1,
    "double_blocks.0.img_mod.lin": 1,
    "double_blocks.0.txt_qkv": 512,
    "double_blocks.0.img_qkv": 1024,
    "double_blocks.9.img_proj": 1024,
    "double_blocks.18.txt_mlp.0": 512,
    "double_blocks.18.img_mlp.2": 1024,
    "txt_in": 512,
    "img_in": 1024,
    "single_blocks.0.linear1": 1536,
    "single_blocks.37.linear2": 1536,
    "single_blocks.20.modulation.lin": 1,
    "final_adaln": 1,
    "final_linear": 1024,
}


@pytest.mark.timeout(600)
def test_full_size_dit_step(orc, dev):
    from convrot_mlx_amd import ConvRotLinear, replace_convrot_linears

    p = FluxParams()
    model = build(p, dev, seed=11)
    inputs = make_inputs(p, img_tokens=1024, txt_tokens=512, device=dev, seed=12)
    modules = dict(model.named_modules())
    assert all(isinstance(modules[n], nn.Linear) for n in SAMPLED)
    dense_w = {n: (from_dev(modules[n].weight), from_dev(modules[n].bias.float())) for n in SAMPLED}
    with torch.no_grad():
        ref = model(**inputs).float()
    linears = sum(1 for m in model.modules() if isinstance(m, nn.Linear))
    names = replace_convrot_linears(model, group_size=G)
    assert linears == 314 and len(names) == 314

    seen: dict[str, tuple[np.ndarray, np.ndarray]] = {}

    def hook(name):
        def fn(mod, args, out):
            seen[name] = (from_dev(args[0].reshape(-1, mod.in_features)),
                          from_dev(out.reshape(-1, mod.out_features)))
        return fn

    mods = dict(model.named_modules())
    handles = [mods[n].register_forward_hook(hook(n)) for n in SAMPLED]
    with torch.no_grad():
        got = model(**inputs)
    for h in handles:
        h.remove()
    with torch.no_grad():
        again = model(**inputs)
    assert torch.equal(got, again), "repeated steps differ"

    for name, rows in SAMPLED.items():
        layer = mods[name]
        assert isinstance(layer, ConvRotLinear) and layer.backend == "hip-w4a4"
        x, out = seen[name]
        assert x.shape[0] == rows, (name, x.shape)
        w, b = dense_w[name]
        w_codes, wscales = orc.prepare_codes(w, "bfloat16", G)
        n_out, k_in = w.shape
        assert np.array_equal(orc.cdna4_to_codes(from_dev(layer.qweight), n_out, k_in), w_codes), name
        assert np.array_equal(from_dev(layer.scales), wscales), name
        a_codes, xs = orc.prepare_codes(x, "bfloat16", G)
        want = orc.w4a4_matmul_codes_large(a_codes, w_codes, xs, wscales, b, "bfloat16")
        bad = int((out != want).sum())
        assert bad == 0, f"{name}: {bad} of {want.size} outputs differ from the oracle"

    got = got.float()
    assert torch.isfinite(got).all()
    rel = ((got - ref).norm() / ref.norm()).item()
    cos = F.cosine_similarity(got.flatten(), ref.flatten(), dim=0).item()
    print(f"full-size config 5: rel_l2={rel:.4f} cosine={cos:.5f}")
    # measured on MI355X at this size: relative L2 ~0.29, cosine ~0.96 (bench seed); a dropped
    # scale or a transposed weight decorrelates the output (relative L2 near 1)
    assert rel < 0.35 and cos > 0.93
