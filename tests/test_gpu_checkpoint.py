"""Offline conversion and repack on the GPU, end to end through the files.

A tiny random-init FLUX DiT's dense weights are written as a safetensors source,
converted (GPU quantization), repacked to the MPP and CDNA4 layouts behind the
round-trip gate, and loaded into fresh models for every backend.  The NK bytes and
scales are checked against the oracle; every loaded model must reproduce the
in-place converted model bit for bit.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch
from torch import nn

from _util import from_dev
from examples.flux1_dev.dit import FluxParams, build, make_inputs

pytestmark = pytest.mark.gpu

G = 64


def _tiny() -> FluxParams:
    return FluxParams(in_channels=64, vec_in_dim=256, context_in_dim=256, hidden_size=256, mlp_ratio=2.0,
                      num_heads=2, depth=1, depth_single_blocks=2, axes_dim=(16, 56, 56))


def test_convert_repack_load(orc, dev, tmp_path):
    import convrot_mlx_amd as api
    from convrot_mlx_amd import checkpoint as ck

    p = _tiny()
    dense = build(p, dev, seed=11)
    src = tmp_path / "dense.safetensors"
    ck._write_safetensors(src, dense.state_dict(), {"format": "pt"})
    topology = build(p, "meta")
    nk = tmp_path / "nk" / "model.safetensors"
    receipt = api.convert_checkpoint(src, nk, topology, group_size=G, device=dev)

    linears = [(n, m) for n, m in dense.named_modules() if isinstance(m, nn.Linear)]
    assert receipt["algorithm"]["converted_linear_count"] == str(len(linears))
    assert receipt["output"]["sha256"] == ck.sha256(nk)
    assert json.loads((nk.parent / "conversion.json").read_text())["output"]["sha256"] == ck.sha256(nk)
    tensors, meta = ck._read_safetensors(nk)
    assert meta["schema"] == ck.CONVROT_SCHEMA and api.inspect_checkpoint(nk, group_size=G)
    # every source tensor exactly once: converted weights became qweight/scales(/bias), the rest copied
    source = dense.state_dict()
    conv = {n for n, _ in linears}
    want = {k for k in source if k.rsplit(".", 1)[0] not in conv}
    for n in conv:
        want |= {f"{n}.qweight", f"{n}.scales", f"{n}.bias"}
    assert set(tensors) == want
    for k in source:
        if k.rsplit(".", 1)[0] not in conv:
            assert torch.equal(tensors[k], source[k].cpu()), k
    # NK bytes and scales of two layers against the oracle
    for name in ("double_blocks.0.img_qkv", "single_blocks.1.linear2"):
        w = from_dev(dict(dense.named_modules())[name].weight)
        codes, scales = orc.prepare_codes(w, "bfloat16", G)
        assert np.array_equal(tensors[f"{name}.qweight"].numpy(), orc.pack_signed_int4(codes)), name
        assert np.array_equal(tensors[f"{name}.scales"].numpy(), scales), name

    inputs = make_inputs(p, img_tokens=64, txt_tokens=16, device=dev, seed=12)
    api.replace_convrot_linears(dense, group_size=G)
    with torch.no_grad():
        ref = dense(**inputs)

    def run(path, backend):
        model, m, names = api.load_convrot_checkpoint(build(p, dev, seed=99), path, backend=backend,
                                                      group_size=G, device=dev)
        assert len(names) == len(linears)
        with torch.no_grad():
            return model(**inputs)

    assert torch.equal(run(nk, "hip-w4a4"), ref)
    for target, backend in (("mpp", "mpp-w4a4"), ("cdna4", "hip-w4a4")):
        out = tmp_path / target / "model.safetensors"
        rec = api.repack_checkpoint(nk, out, target=target, device=dev)
        assert rec["bitExactRoundTrip"] and rec["repackedLinearCount"] == len(linears)
        api.inspect_checkpoint(out, group_size=G)
        assert torch.equal(run(out, backend), ref), target
        with pytest.raises(FileExistsError):
            api.repack_checkpoint(nk, out, target=target, device=dev)
    with pytest.raises(FileExistsError):
        api.convert_checkpoint(src, nk, topology, group_size=G, device=dev)
