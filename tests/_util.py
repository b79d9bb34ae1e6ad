"""Test helpers: numpy <-> torch transfers of bf16/f16 bit patterns, seeded inputs."""

from __future__ import annotations

import numpy as np
import torch

TORCH_DT = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def to_dev(arr: np.ndarray, dtype: str, dev) -> torch.Tensor:
    """Oracle-side storage (uint16 bits or float32) -> device tensor of `dtype`."""
    if dtype == "float32":
        return torch.from_numpy(np.ascontiguousarray(arr, dtype=np.float32)).to(dev)
    bits = np.ascontiguousarray(arr, dtype=np.uint16).view(np.int16)
    return torch.from_numpy(bits).view(TORCH_DT[dtype]).to(dev)


def from_dev(t: torch.Tensor) -> np.ndarray:
    """Device tensor -> oracle-side storage (uint16 bits for 16-bit floats)."""
    t = t.detach().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def normal_input(seed: int, shape, dtype: str, orc) -> np.ndarray:
    """rng.normal(size).astype(float32) then an RNE cast, as test_core.py builds inputs (e.g. :55-58)."""
    rng = np.random.default_rng(seed)
    return orc.from_f32(rng.normal(size=shape).astype(np.float32), dtype)


def outlier_input(seed: int, shape, dtype: str, orc, std=1.0, frac=0.005, factor=20.0) -> np.ndarray:
    """Heavy-tailed activations/weights of the benchmark configs: a fixed seeded subset of
    channels (columns) scaled by `factor`."""
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, std, size=shape).astype(np.float32)
    k = shape[-1]
    cols = rng.choice(k, size=max(1, int(round(frac * k))), replace=False)
    x[..., cols] *= factor
    return orc.from_f32(x, dtype)
