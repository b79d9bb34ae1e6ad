"""Offline conversion, lossless repack and loading of ConvRot checkpoints (safetensors).

torch counterpart of the reference's FLUX checkpoint tooling:
  - `convert_checkpoint`  convert.py:62-177  dense source -> NK-packed ConvRot W4A4 file;
  - `repack_checkpoint`   repack_mpp.py:86-190  NK -> MPP (K x packed-N) or -> CDNA4 tiles,
                          behind a bit-exact round-trip gate;
  - `load_convrot_checkpoint`  adapter.py:73-106  swap the model's Linears, check the schema,
                          layout, group size and layer count, then load strictly;
  - `inspect_checkpoint`  convert.py:42-59 / repack_mpp.py:67-83 metadata gates.

Formats.  Keys are `{name}.qweight`, `{name}.scales` (float32 [N]) and `{name}.bias`
(float32 [N], zeros when the source Linear had none) for every converted Linear; every
other source tensor is copied unchanged, and each source tensor is consumed exactly once
(convert.py:147-149).  Metadata values are strings.  Three schemas:
  - CONVROT_SCHEMA (the reference's, NK: qweight uint8 [N, K/2]);
  - CONVROT_MPP_SCHEMA with CONVROT_MPP_WEIGHT_LAYOUT (the reference's, qweight [K, N/2]);
  - CONVROT_CDNA4_SCHEMA with WEIGHT_LAYOUT_CDNA4 (this library's, qweight in the CDNA4
    tile layout [ceil(K/128), ceil(N/16), 1024]); metadata `linear_shapes` records each
    layer's (N, K), since the padded tile shape does not.

The reference pins its checks to one FLUX.1 Dev source digest and topology; here the
digest is recorded (and checked when the caller passes one) and the topology is the
model the caller passes.  Quantization and repacks run on the GPU (the HIP kernels);
there is no CPU path.  Outputs and receipts are never overwritten.
"""

from __future__ import annotations

import os

import hashlib
import json
import time
from datetime import datetime, timezone
from pathlib import Path
from typing import Mapping

import torch
from torch import nn

from .adapter import replace_convrot_linears
from .core import (
    CONVROT_GROUP_SIZE,
    WEIGHT_LAYOUT_CDNA4,
    ConvRotLinear,
    eligible_linear,
    quantize_convrot_weight,
    repack_cdna4_weight_to_nk,
    repack_mpp_weight_to_nk,
    repack_nk_weight_for_cdna4,
    repack_nk_weight_for_mpp,
)

CONVROT_SCHEMA = "convrot-mlx.flux1-convrot-w4a4.v1"  # adapter.py:25
CONVROT_MPP_SCHEMA = "convrot-mlx.flux1-convrot-w4-mpp.v1"  # adapter.py:26
CONVROT_MPP_WEIGHT_LAYOUT = "signed_twos_complement_low_nibble_even_output_k_by_packed_n"  # adapter.py:27-29
CONVROT_CDNA4_SCHEMA = "convrot-mlx-amd.convrot-w4-cdna4.v1"
CONVERSION_RECEIPT_SCHEMA = "convrot-mlx-amd.conversion.v1"
REPACK_RECEIPT_SCHEMA = "convrot-mlx-amd.repack.v1"

NK_PACKING = "signed_twos_complement_low_nibble_even_column"  # convert.py:169
_COMMON_REQUIRED = {"weight_bits": "4"}


def sha256(path: Path) -> str:
    """convert.py:29-34: streamed SHA-256 of a file."""
    digest = hashlib.sha256()
    with Path(path).open("rb") as handle:
        while chunk := handle.read(16 * 1024 * 1024):
            digest.update(chunk)
    return digest.hexdigest()


def _now() -> str:
    return datetime.now(timezone.utc).isoformat()


def _refuse_existing(path: Path, what: str) -> None:
    if path.exists() or path.is_symlink():
        raise FileExistsError(f"Refusing to overwrite existing {what}: {path}")


def _read_safetensors(path: Path) -> tuple[dict[str, torch.Tensor], dict[str, str]]:
    from safetensors import safe_open

    tensors = {}
    with safe_open(str(path), framework="pt", device="cpu") as handle:
        metadata = dict(handle.metadata() or {})
        for key in handle.keys():
            tensors[key] = handle.get_tensor(key)
    return tensors, metadata


def _write_safetensors(path: Path, tensors: Mapping[str, torch.Tensor], metadata: Mapping[str, str]) -> None:
    from safetensors.torch import save_file

    path.parent.mkdir(parents=True, exist_ok=True)
    save_file({k: v.detach().contiguous().cpu() for k, v in tensors.items()}, str(path),
              metadata={k: str(v) for k, v in metadata.items()})


def read_metadata(path: str | Path) -> dict[str, str]:
    from safetensors import safe_open

    with safe_open(str(path), framework="pt", device="cpu") as handle:
        return dict(handle.metadata() or {})


def _check_required(metadata: Mapping[str, str], required: Mapping[str, str], where: str) -> None:
    for name, expected in required.items():
        if metadata.get(name) != expected:
            raise ValueError(f"{where} metadata {name!r} is {metadata.get(name)!r}; expected {expected!r}")


def _selected_linears(model: nn.Module, group_size: int) -> list[tuple[str, nn.Linear]]:
    return [(name, m) for name, m in model.named_modules() if name and eligible_linear(m, group_size)]


# ------------------------------------------------------------------ convert


def convert_checkpoint(
    source: str | Path | Mapping[str, torch.Tensor],
    output: str | Path,
    model: nn.Module,
    *,
    receipt: str | Path | None = None,
    group_size: int = CONVROT_GROUP_SIZE,
    device: str | torch.device = "cuda",
    skip_source_hash: bool = False,
    expected_source_sha256: str | None = None,
) -> dict:
    """Quantize every eligible Linear of `model`'s topology from a dense source checkpoint.

    `source` is a safetensors file (or an in-memory state dict) whose keys are exactly
    `model`'s parameter names; `model` only supplies the topology (it may live on the meta
    device).  Writes the NK-packed CONVROT_SCHEMA file and a JSON receipt (default
    `conversion.json` beside the output) and returns the receipt.  convert.py:62-177.
    """
    output = Path(output)
    receipt_path = Path(receipt) if receipt is not None else output.with_name("conversion.json")
    _refuse_existing(output, "ConvRot checkpoint")
    _refuse_existing(receipt_path, "conversion receipt")
    started_at, started = _now(), time.perf_counter()

    if isinstance(source, Mapping):
        source_weights = dict(source)
        source_info = {"path": None, "bytes": None, "sha256": "in-memory"}
    else:
        src = Path(source)
        if not src.is_file() or src.is_symlink():
            raise FileNotFoundError(f"Expected a regular, non-symlinked source checkpoint: {src}")
        digest = "skipped" if skip_source_hash else sha256(src)
        if expected_source_sha256 is not None and digest != expected_source_sha256:
            raise ValueError(f"Source SHA-256 mismatch: {digest}")
        source_weights, _ = _read_safetensors(src)
        source_info = {"path": str(src), "bytes": src.stat().st_size, "sha256": digest}

    expected = {name for name, _ in model.named_parameters()}
    missing = sorted(expected - source_weights.keys())
    unexpected = sorted(source_weights.keys() - expected)
    if missing or unexpected:
        raise ValueError(f"Source topology differs from the model; missing={missing[:8]}, unexpected={unexpected[:8]}")

    linears = [(n, m) for n, m in model.named_modules() if isinstance(m, nn.Linear)]
    selected = _selected_linears(model, group_size)
    out: dict[str, torch.Tensor] = {}
    shapes: dict[str, list[int]] = {}
    dev = torch.device(device)
    for name, _ in selected:
        weight = source_weights.pop(f"{name}.weight")
        with torch.no_grad():
            qweight, scales = quantize_convrot_weight(weight.to(dev), group_size)
        out[f"{name}.qweight"] = qweight.cpu()
        out[f"{name}.scales"] = scales.cpu()
        bias_key = f"{name}.bias"
        if bias_key in source_weights:
            out[bias_key] = source_weights.pop(bias_key).to(torch.float32)
        else:
            out[bias_key] = torch.zeros((weight.shape[0],), dtype=torch.float32)
        shapes[name] = [int(weight.shape[0]), int(weight.shape[1])]
        del weight, qweight, scales
    # Ineligible Linears and every other tensor stay in their source dtype; each source key
    # is written exactly once.
    overlap = source_weights.keys() & out.keys()
    if overlap:
        raise ValueError(f"Source tensors collide with converted keys: {sorted(overlap)[:8]}")
    out.update(source_weights)

    metadata = {
        "schema": CONVROT_SCHEMA,
        "source_sha256": source_info["sha256"],
        "convrot_group_size": str(group_size),
        "quant_group_size": str(group_size),
        "weight_bits": "4",
        "activation_bits": "4",
        "weight_scale": "rowwise_absmax_div_7",
        "activation_scale": "rowwise_absmax_div_7",
        "packing": NK_PACKING,
        "converted_linear_count": str(len(selected)),
        "linear_count": str(len(linears)),
        "reference_algorithm": "plain ConvRot W4A4 eager contract",
        "quantizer": "convrot_prepare (gfx950 HIP)",
    }
    _write_safetensors(output, out, metadata)
    evidence = {
        "schema": CONVERSION_RECEIPT_SCHEMA,
        "source": source_info,
        "output": {"path": str(output), "bytes": output.stat().st_size, "sha256": sha256(output)},
        "algorithm": metadata,
        "convertedLayers": shapes,
        "startedAt": started_at,
        "completedAt": _now(),
        "elapsedSeconds": round(time.perf_counter() - started, 3),
    }
    receipt_path.parent.mkdir(parents=True, exist_ok=True)
    receipt_path.write_text(json.dumps(evidence, indent=2, sort_keys=True) + "\n")
    return evidence


# ------------------------------------------------------------------ repack


def repack_checkpoint(
    source: str | Path,
    output: str | Path,
    *,
    target: str = "mpp",
    receipt: str | Path | None = None,
    device: str | torch.device = "cuda",
    skip_source_hash: bool = False,
) -> dict:
    """Losslessly repack an NK ConvRot checkpoint to the MPP (`target="mpp"`) or CDNA4
    (`target="cdna4"`) weight layout.  Every qweight passes a bit-exact round trip back to
    NK before it is written; scales, biases and unconverted tensors are copied unchanged.
    repack_mpp.py:86-190."""
    if target not in ("mpp", "cdna4"):
        raise ValueError(f"repack target must be 'mpp' or 'cdna4', got {target!r}")
    source, output = Path(source), Path(output)
    receipt_path = Path(receipt) if receipt is not None else output.with_name("repack.json")
    _refuse_existing(output, f"{target.upper()} checkpoint")
    _refuse_existing(receipt_path, "repack receipt")
    if not source.is_file() or source.is_symlink():
        raise FileNotFoundError(f"Expected a regular, non-symlinked ConvRot checkpoint: {source}")
    started_at, started = _now(), time.perf_counter()
    weights, src_meta = _read_safetensors(source)
    _check_required(src_meta, {"schema": CONVROT_SCHEMA, "packing": NK_PACKING, **_COMMON_REQUIRED}, "Source")
    source_hash = "skipped" if skip_source_hash else sha256(source)

    qweight_keys = sorted(k for k in weights if k.endswith(".qweight"))
    expected_count = int(src_meta.get("converted_linear_count", "-1"))
    if len(qweight_keys) != expected_count:
        raise ValueError(f"Found {len(qweight_keys)} qweights; metadata expects {expected_count}")
    dev = torch.device(device)
    out: dict[str, torch.Tensor] = {}
    shapes: dict[str, dict[str, list[int]]] = {}
    linear_shapes: dict[str, list[int]] = {}
    for key in qweight_keys:
        nk = weights.pop(key).to(dev)
        n, k = int(nk.shape[0]), int(nk.shape[1]) * 2
        if target == "mpp":
            packed = repack_nk_weight_for_mpp(nk)
            back = repack_mpp_weight_to_nk(packed)
        else:
            packed = repack_nk_weight_for_cdna4(nk)
            back = repack_cdna4_weight_to_nk(packed, n, k)
        if not torch.equal(back, nk):
            raise RuntimeError(f"Bit-exact {target.upper()} repack gate failed for {key}")
        out[key] = packed.cpu()
        name = key[: -len(".qweight")]
        shapes[key] = {"sourcePackedNK": [n, k // 2], "repacked": [int(v) for v in packed.shape]}
        linear_shapes[name] = [n, k]
        del nk, packed, back
    out.update(weights)
    metadata = dict(src_meta)
    metadata["source_convrot_sha256"] = source_hash
    metadata["lossless_layout_repack"] = "true"
    if target == "mpp":
        metadata.update({
            "schema": CONVROT_MPP_SCHEMA,
            "weight_layout": CONVROT_MPP_WEIGHT_LAYOUT,
            "packing": "signed_twos_complement_low_nibble_even_output",
            "activation_bits": "4-or-16-runtime-selected",
            "supported_activation_modes": "a4-values-in-int8,bfloat16,float16",
        })
    else:
        metadata.update({
            "schema": CONVROT_CDNA4_SCHEMA,
            "weight_layout": WEIGHT_LAYOUT_CDNA4,
            "packing": "cdna4_16x128_tiles_split_nibble",
            "activation_bits": "4-or-16-runtime-selected",
            "supported_activation_modes": "a4-values-in-int8,bfloat16,float16",
            "linear_shapes": json.dumps(linear_shapes, sort_keys=True),
        })
    _write_safetensors(output, out, metadata)
    evidence = {
        "schema": REPACK_RECEIPT_SCHEMA,
        "target": target,
        "source": {"path": str(source), "bytes": source.stat().st_size, "sha256": source_hash},
        "output": {"path": str(output), "bytes": output.stat().st_size, "sha256": sha256(output)},
        "algorithm": metadata,
        "repackedLinearCount": len(qweight_keys),
        "bitExactRoundTrip": True,
        "repackedShapes": shapes,
        "startedAt": started_at,
        "completedAt": _now(),
        "elapsedSeconds": round(time.perf_counter() - started, 3),
    }
    receipt_path.parent.mkdir(parents=True, exist_ok=True)
    receipt_path.write_text(json.dumps(evidence, indent=2, sort_keys=True) + "\n")
    return evidence


# ------------------------------------------------------------------ inspect / load


def inspect_checkpoint(path: str | Path, group_size: int = CONVROT_GROUP_SIZE) -> dict[str, str]:
    """Check a checkpoint's metadata against its schema's required values and return it
    (convert.py:42-59, repack_mpp.py:67-83)."""
    metadata = read_metadata(path)
    schema = metadata.get("schema")
    required = {"convrot_group_size": str(group_size), **_COMMON_REQUIRED}
    if schema == CONVROT_SCHEMA:
        required.update({"activation_bits": "4", "weight_scale": "rowwise_absmax_div_7",
                         "activation_scale": "rowwise_absmax_div_7", "packing": NK_PACKING})
    elif schema == CONVROT_MPP_SCHEMA:
        required.update({"weight_layout": CONVROT_MPP_WEIGHT_LAYOUT, "lossless_layout_repack": "true"})
    elif schema == CONVROT_CDNA4_SCHEMA:
        required.update({"weight_layout": WEIGHT_LAYOUT_CDNA4, "lossless_layout_repack": "true"})
    else:
        raise ValueError(f"{path} has no ConvRot schema (found {schema!r})")
    _check_required(metadata, required, str(path))
    return metadata


def load_convrot_checkpoint(
    model: nn.Module,
    path: str | Path,
    *,
    backend: str | None = None,
    preprocessor: str | None = None,
    group_size: int = CONVROT_GROUP_SIZE,
    expected_source_sha256: str | None = None,
    device: str | torch.device | None = None,
) -> tuple[nn.Module, dict[str, str], list[str]]:
    """Swap `model`'s eligible Linears for ConvRotLinear and load a converted checkpoint into
    it strictly; returns (model, metadata, converted names).  adapter.py:73-106.

    Schemas by backend: `mpp-*` needs CONVROT_MPP_SCHEMA with the MPP weight layout;
    `hip-*` takes CONVROT_CDNA4_SCHEMA as stored, or the NK CONVROT_SCHEMA repacked to the
    CDNA4 layout on `device` while loading."""
    metadata = read_metadata(path)
    # the same default as ConvRotLinear: $CONVROT_BACKEND, then the reference's variable
    backend = backend or os.getenv("CONVROT_BACKEND") or os.getenv("CONVROT_MLX_BACKEND") or "hip-w4a4"
    uses_mpp = backend.startswith("mpp-")
    allowed = (CONVROT_MPP_SCHEMA,) if uses_mpp else (CONVROT_CDNA4_SCHEMA, CONVROT_SCHEMA)
    schema = metadata.get("schema")
    if schema not in allowed:
        raise ValueError(f"ConvRot backend {backend!r} requires checkpoint schema "
                         f"{' or '.join(repr(s) for s in allowed)}; found {schema!r}")
    if uses_mpp and metadata.get("weight_layout") != CONVROT_MPP_WEIGHT_LAYOUT:
        raise ValueError(f"MPP ConvRot checkpoint has unsupported weight layout: {metadata.get('weight_layout')!r}")
    if schema == CONVROT_CDNA4_SCHEMA and metadata.get("weight_layout") != WEIGHT_LAYOUT_CDNA4:
        raise ValueError(f"CDNA4 ConvRot checkpoint has unsupported weight layout: {metadata.get('weight_layout')!r}")
    if expected_source_sha256 is not None and metadata.get("source_sha256") != expected_source_sha256:
        raise ValueError("ConvRot checkpoint does not derive from the expected source digest.")
    if int(metadata.get("convrot_group_size", "0")) != group_size:
        raise ValueError("ConvRot checkpoint group size does not match this runtime.")

    converted = replace_convrot_linears(model, backend=backend, preprocessor=preprocessor,
                                        group_size=group_size, convert=False)
    if int(metadata.get("converted_linear_count", "-1")) != len(converted):
        raise ValueError("ConvRot checkpoint layer count does not match the model topology.")
    weights, _ = _read_safetensors(Path(path))
    if schema == CONVROT_SCHEMA:
        modules = dict(model.named_modules())
        dev = torch.device(device) if device is not None else None
        for name in converted:
            key = f"{name}.qweight"
            if key not in weights:
                continue  # reported by the strict load below
            layer: ConvRotLinear = modules[name]
            nk = weights[key].to(dev or layer.qweight.device)
            if tuple(nk.shape) != (layer.out_features, layer.in_features // 2):
                raise ValueError(f"{key} has shape {tuple(nk.shape)}; expected "
                                 f"{(layer.out_features, layer.in_features // 2)}")
            weights[key] = repack_nk_weight_for_cdna4(nk)
    model.load_state_dict(weights, strict=True)
    return model, metadata, converted
