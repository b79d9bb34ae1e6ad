#!/usr/bin/env python3
"""W4A4 or W4A16 for the M = 1 modulation Linears of a DiT: complete-path time and deviation.

A FLUX-style DiT runs its adaLN modulation Linears (3072 -> 18432 / 9216 / 6144) on one
row per image.  At that M both ConvRot backends stream the same int4 weights, so the
choice is between W4A4 (int8 A4 codes: rotate + quantize, few-row INT8 GEMM) and W4A16
(rotated bf16 activations, bf16 GEMM).  For each shape and M in {1, 2} this times
`ConvRotLinear.forward` under both backends (HIP-graph replays of 64 calls cycling through
weight sets > 512 MB) and torch's dense bf16 `linear`, and reports each backend's relative
L2 deviation from the float32 product with the dense bf16 weights.

Weights ~ N(0, 0.02^2), bias ~ N(0, 0.02^2), input silu(N(0, 1)) in bf16, group 64.

    python benchmarks/small_m_policy.py
"""

from __future__ import annotations

import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT / "convrot-mlx_amd") not in sys.path:
    sys.path.insert(0, str(ROOT / "convrot-mlx_amd"))

import torch  # noqa: E402
import torch.nn as nn  # noqa: E402
import torch.nn.functional as F  # noqa: E402

import convrot_mlx_amd as api  # noqa: E402

SHAPES = [(3072, 18432), (3072, 9216), (3072, 6144)]
BACKENDS = ("hip-w4a4", "hip-w4a16")
CALLS = 64


def graph_us(fn, stream: torch.cuda.Stream) -> float:
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for i in range(3):
            fn(i)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(CALLS):
                fn(i)
        graph.replay()
        torch.cuda.synchronize()
        best = 1e30
        for _ in range(5):
            t0 = time.perf_counter()
            graph.replay()
            torch.cuda.synchronize()
            best = min(best, (time.perf_counter() - t0) * 1e6 / CALLS)
    torch.cuda.current_stream().wait_stream(stream)
    return best


def main() -> int:
    if not torch.cuda.is_available():
        raise SystemExit("this benchmark needs a GPU")
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    stream = torch.cuda.Stream()
    print("| M | K -> N | W4A4 us | W4A16 us | dense bf16 us | W4A4 rel L2 | W4A16 rel L2 |")
    print("|---:|---|---:|---:|---:|---:|---:|")
    for K, N in SHAPES:
        sets = max(2, (600 << 20) // (N * K // 2) + 1)
        dense = []
        for _ in range(sets):
            d = nn.Linear(K, N).to(dev, torch.bfloat16)
            nn.init.normal_(d.weight, 0.0, 0.02)
            nn.init.normal_(d.bias, 0.0, 0.02)
            dense.append(d)
        layers = {}
        for backend in BACKENDS:
            converted = []
            for d in dense:
                holder = nn.Sequential(nn.Linear(K, N).to(dev, torch.bfloat16))
                holder[0].load_state_dict(d.state_dict())
                api.replace_convrot_linears(holder, backend=backend, group_size=64)
                converted.append(holder[0])
            layers[backend] = converted
        for M in (1, 2):
            x = F.silu(torch.randn(M, K, device=dev)).to(torch.bfloat16)
            ref = F.linear(x.float(), dense[0].weight.float(), dense[0].bias.float())
            us, rel = {}, {}
            for backend in BACKENDS:
                us[backend] = graph_us(lambda i, b=backend: layers[b][i % sets](x), stream)
                y = layers[backend][0](x).float()
                rel[backend] = ((y - ref).norm() / ref.norm()).item()
            dense_us = graph_us(lambda i: F.linear(x, dense[i % sets].weight, dense[i % sets].bias), stream)
            print(f"| {M} | {K} -> {N} | {us['hip-w4a4']:.1f} | {us['hip-w4a16']:.1f} | {dense_us:.1f} | "
                  f"{rel['hip-w4a4']:.4f} | {rel['hip-w4a16']:.4f} |", flush=True)
        del dense, layers
    return 0


if __name__ == "__main__":
    sys.exit(main())
