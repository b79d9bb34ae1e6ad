"""Checkpoint format, loader gates and conversion refusals on the CPU.

Files are fabricated from `replace_convrot_linears(convert=False)` state dicts with
random bytes, so every check here runs without a kernel: schema / layout / group-size /
layer-count / digest gates of the loader (adapter.py:81-106), strict key loading,
metadata gates (convert.py:42-59, repack_mpp.py:67-83), and the refusals that come
before any quantization (convert.py:70-88,103-109; repack_mpp.py:86-109).  Conversion
and repacks themselves run under the `gpu` marker (test_gpu_checkpoint.py).
"""

from __future__ import annotations

import os

import pytest
import torch

from examples.flux1_dev.dit import FluxParams, build

G = 64


def _tiny() -> FluxParams:
    return FluxParams(in_channels=64, vec_in_dim=128, context_in_dim=128, hidden_size=128, mlp_ratio=2.0,
                      num_heads=2, depth=1, depth_single_blocks=1, axes_dim=(8, 28, 28))


def _api():
    import convrot_mlx_amd as api
    from convrot_mlx_amd import checkpoint as ck

    return api, ck


def _fabricate(tmp_path, backend, schema, extra_meta=None, drop_key=None, name="ck.safetensors"):
    """A converted model with random qweight bytes / scales / biases, written as a checkpoint."""
    api, ck = _api()
    model = build(_tiny(), "cpu", seed=1)
    names = api.replace_convrot_linears(model, backend=backend, group_size=G, convert=False)
    gen = torch.Generator().manual_seed(7)
    modules = dict(model.named_modules())
    for n in names:
        layer = modules[n]
        layer.qweight = torch.randint(0, 256, layer.qweight.shape, dtype=torch.uint8, generator=gen)
        layer.scales = torch.rand(layer.scales.shape, generator=gen)
        layer.bias = torch.randn(layer.bias.shape, generator=gen)
    state = model.state_dict()
    if drop_key:
        state.pop(drop_key)
    meta = {"schema": schema, "convrot_group_size": str(G), "converted_linear_count": str(len(names)),
            "weight_bits": "4", "source_sha256": "abc", "lossless_layout_repack": "true"}
    if schema == ck.CONVROT_MPP_SCHEMA:
        meta["weight_layout"] = ck.CONVROT_MPP_WEIGHT_LAYOUT
    if schema == ck.CONVROT_CDNA4_SCHEMA:
        meta["weight_layout"] = api.WEIGHT_LAYOUT_CDNA4
    meta.update(extra_meta or {})
    path = tmp_path / name
    ck._write_safetensors(path, state, meta)
    return path, state, names


@pytest.mark.parametrize("backend,schema_name", [("hip-w4a4", "CONVROT_CDNA4_SCHEMA"),
                                                 ("hip-w4a16", "CONVROT_CDNA4_SCHEMA"),
                                                 ("mpp-w4a4", "CONVROT_MPP_SCHEMA"),
                                                 ("mpp-w4a16", "CONVROT_MPP_SCHEMA")])
def test_load_round_trips_every_tensor(tmp_path, backend, schema_name):
    api, ck = _api()
    path, state, names = _fabricate(tmp_path, backend, getattr(ck, schema_name))
    fresh = build(_tiny(), "cpu", seed=2)
    model, meta, converted = api.load_convrot_checkpoint(fresh, path, backend=backend, group_size=G)
    assert converted == names and meta["schema"] == getattr(ck, schema_name)
    loaded = model.state_dict()
    assert loaded.keys() == state.keys()
    for k, v in state.items():
        assert torch.equal(loaded[k], v), k
    assert api.inspect_checkpoint(path, group_size=G)["schema"] == getattr(ck, schema_name)


def test_loader_gates(tmp_path):
    api, ck = _api()
    mpp, _, _ = _fabricate(tmp_path, "mpp-w4a4", ck.CONVROT_MPP_SCHEMA, name="mpp.safetensors")
    cdna4, _, _ = _fabricate(tmp_path, "hip-w4a4", ck.CONVROT_CDNA4_SCHEMA, name="c.safetensors")
    fresh = lambda: build(_tiny(), "cpu", seed=2)  # noqa: E731
    with pytest.raises(ValueError, match="requires checkpoint schema"):
        api.load_convrot_checkpoint(fresh(), mpp, backend="hip-w4a4", group_size=G)
    with pytest.raises(ValueError, match="requires checkpoint schema"):
        api.load_convrot_checkpoint(fresh(), cdna4, backend="mpp-w4a4", group_size=G)
    with pytest.raises(ValueError, match="group size"):
        api.load_convrot_checkpoint(fresh(), cdna4, backend="hip-w4a4", group_size=256)
    with pytest.raises(ValueError, match="source digest"):
        api.load_convrot_checkpoint(fresh(), cdna4, backend="hip-w4a4", group_size=G, expected_source_sha256="x")
    bad_layout, _, _ = _fabricate(tmp_path, "mpp-w4a4", ck.CONVROT_MPP_SCHEMA, {"weight_layout": "nk"},
                                  name="bl.safetensors")
    with pytest.raises(ValueError, match="weight layout"):
        api.load_convrot_checkpoint(fresh(), bad_layout, backend="mpp-w4a4", group_size=G)
    bad_count, _, _ = _fabricate(tmp_path, "hip-w4a4", ck.CONVROT_CDNA4_SCHEMA,
                                 {"converted_linear_count": "3"}, name="bc.safetensors")
    with pytest.raises(ValueError, match="layer count"):
        api.load_convrot_checkpoint(fresh(), bad_count, backend="hip-w4a4", group_size=G)
    _, _, names = _fabricate(tmp_path, "hip-w4a4", ck.CONVROT_CDNA4_SCHEMA, name="ok.safetensors")
    dropped, _, names = _fabricate(tmp_path, "hip-w4a4", ck.CONVROT_CDNA4_SCHEMA,
                                   drop_key=f"{names[0]}.scales", name="dropped.safetensors")
    with pytest.raises(RuntimeError, match="Missing key"):
        api.load_convrot_checkpoint(fresh(), dropped, backend="hip-w4a4", group_size=G)


def test_inspect_gates(tmp_path):
    api, ck = _api()
    path, _, _ = _fabricate(tmp_path, "mpp-w4a4", ck.CONVROT_MPP_SCHEMA, {"lossless_layout_repack": "false"})
    with pytest.raises(ValueError, match="lossless_layout_repack"):
        api.inspect_checkpoint(path, group_size=G)
    other, _, _ = _fabricate(tmp_path, "hip-w4a4", "something-else", name="o.safetensors")
    with pytest.raises(ValueError, match="no ConvRot schema"):
        api.inspect_checkpoint(other, group_size=G)


def test_convert_and_repack_refusals(tmp_path):
    """Everything convert/repack refuse before quantizing: existing output or receipt,
    symlinked or missing source, a source whose keys differ from the model, a source of the
    wrong schema, a qweight count that disagrees with the metadata."""
    api, ck = _api()
    model = build(_tiny(), "cpu", seed=1)
    state = {k: v for k, v in model.state_dict().items()}
    src = tmp_path / "dense.safetensors"
    ck._write_safetensors(src, state, {})
    out = tmp_path / "out.safetensors"
    out.write_bytes(b"")
    with pytest.raises(FileExistsError, match="Refusing to overwrite"):
        api.convert_checkpoint(src, out, model, group_size=G)
    out.unlink()
    (tmp_path / "conversion.json").write_text("{}")
    with pytest.raises(FileExistsError, match="receipt"):
        api.convert_checkpoint(src, out, model, group_size=G)
    (tmp_path / "conversion.json").unlink()
    link = tmp_path / "link.safetensors"
    os.symlink(src, link)
    with pytest.raises(FileNotFoundError, match="non-symlinked"):
        api.convert_checkpoint(link, out, model, group_size=G)
    with pytest.raises(FileNotFoundError):
        api.convert_checkpoint(tmp_path / "absent.safetensors", out, model, group_size=G)
    partial = dict(state)
    partial.pop(next(iter(partial)))
    with pytest.raises(ValueError, match="topology differs"):
        api.convert_checkpoint(partial, out, model, group_size=G)
    with pytest.raises(ValueError, match="Source SHA-256 mismatch"):
        api.convert_checkpoint(src, out, model, group_size=G, expected_source_sha256="0" * 64)
    assert not out.exists()

    wrong, _, _ = _fabricate(tmp_path, "hip-w4a4", ck.CONVROT_CDNA4_SCHEMA, name="w.safetensors")
    with pytest.raises(ValueError, match="schema"):
        api.repack_checkpoint(wrong, tmp_path / "r.safetensors", target="mpp")
    nk_bad, _, _ = _fabricate(tmp_path, "hip-w4a4", ck.CONVROT_SCHEMA,
                              {"packing": ck.NK_PACKING, "converted_linear_count": "1"}, name="nk.safetensors")
    with pytest.raises(ValueError, match="metadata expects 1"):
        api.repack_checkpoint(nk_bad, tmp_path / "r.safetensors", target="cdna4")
    with pytest.raises(ValueError, match="target"):
        api.repack_checkpoint(nk_bad, tmp_path / "r2.safetensors", target="kn")
    (tmp_path / "r3.safetensors").write_bytes(b"")
    with pytest.raises(FileExistsError):
        api.repack_checkpoint(nk_bad, tmp_path / "r3.safetensors", target="mpp")
    assert not (tmp_path / "r.safetensors").exists()


def test_receipt_schema_names():
    _, ck = _api()
    # the reference's checkpoint schemas are kept verbatim so its files identify the same way
    assert ck.CONVROT_SCHEMA == "convrot-mlx.flux1-convrot-w4a4.v1"
    assert ck.CONVROT_MPP_SCHEMA == "convrot-mlx.flux1-convrot-w4-mpp.v1"
    assert ck.CONVROT_MPP_WEIGHT_LAYOUT == "signed_twos_complement_low_nibble_even_output_k_by_packed_n"
