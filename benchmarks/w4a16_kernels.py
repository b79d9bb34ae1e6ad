#!/usr/bin/env python3
"""W4A16 GEMM kernel sweep on MI355X: each kernel of `convrot_w4a16_gemm` against dense bf16.

The W4A16 entry point (the counterpart of the reference's mpp_w4a16_matmul,
/root/reference/src/convrot_mlx/core.py:1123-1152) has two kernels: a weight-streaming
split kernel for few token rows and an LDS-tiled MFMA kernel with 256/128-row and -column
tiles for many.  This script forces each one (CONVROT_W4A16_CFG / CONVROT_W4A16_TILE),
also runs the default dispatch, and times torch's dense bf16 `linear` on the same shape.

Timing: HIP-graph replays of 16 launches that cycle through 4 weight sets (so that the
weights are not all L2/MALL-resident), one replay after a warm-up replay, on a side
stream; microseconds per launch.  Activations are bf16, the output bf16.

    python benchmarks/w4a16_kernels.py [--shape MxKxN ...] [--variants F,T256x256,...,auto]
"""

from __future__ import annotations

import argparse
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT / "convrot-mlx_amd") not in sys.path:
    sys.path.insert(0, str(ROOT / "convrot-mlx_amd"))

import torch  # noqa: E402
import torch.nn.functional as F  # noqa: E402

import convrot_mlx_amd as api  # noqa: E402
from convrot_mlx_amd import core  # noqa: E402

DEFAULT_SHAPES = ["1536x3072x21504", "1536x15360x3072", "1024x3072x3072", "1024x3072x12288",
                  "1024x12288x3072", "512x3072x3072", "4096x3072x3072", "4096x4096x4096",
                  "256x3072x12288", "128x3072x12288", "128x3072x3072", "64x3072x12288"]
DEFAULT_VARIANTS = "A,F,T256x256,T256x128,T128x256,T128x128,auto"
WEIGHT_SETS = 4
LAUNCHES = 16


def _set_variant(v: str) -> None:
    os.environ.pop("CONVROT_W4A16_CFG", None)
    os.environ.pop("CONVROT_W4A16_TILE", None)
    if v == "auto":
        return
    if v.startswith("T") and len(v) > 1:
        os.environ["CONVROT_W4A16_CFG"] = "T"
        os.environ["CONVROT_W4A16_TILE"] = v[1:]
    else:
        os.environ["CONVROT_W4A16_CFG"] = v


def _graph_us(run, stream: torch.cuda.Stream) -> float:
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for i in range(3):
            run(i)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(LAUNCHES):
                run(i)
        graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        graph.replay()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    torch.cuda.current_stream().wait_stream(stream)
    return (t1 - t0) * 1e6 / LAUNCHES


def sweep(shape: str, variants: list[str], stream: torch.cuda.Stream) -> dict:
    M, K, N = (int(v) for v in shape.split("x"))
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(M * 31 + K * 7 + N)
    wq = [torch.randint(0, 256, core.cdna4_shape(N, K), dtype=torch.uint8, device=dev, generator=gen)
          for _ in range(WEIGHT_SETS)]
    wd = [torch.randn(N, K, device=dev, generator=gen).to(torch.bfloat16) for _ in range(WEIGHT_SETS)]
    x = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
    ws = torch.rand(N, device=dev, generator=gen) * 0.01
    b = torch.rand(N, device=dev, generator=gen)
    row = {"shape": shape}
    outs = []
    for v in variants:
        _set_variant(v)
        holder = {}

        def run(i, holder=holder):
            holder["out"] = api.hip_w4a16_matmul(x, wq[i % WEIGHT_SETS], ws, b, output_dtype=torch.bfloat16,
                                                 out_features=N)

        row[v] = _graph_us(run, stream)
        outs.append(api.hip_w4a16_matmul(x, wq[0], ws, b, output_dtype=torch.bfloat16, out_features=N).float())
    _set_variant("auto")
    row["dense"] = _graph_us(lambda i: F.linear(x, wd[i % WEIGHT_SETS]), stream)
    ref = outs[0]
    row["max_rel_diff"] = max(((o - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item() for o in outs)
    return row


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--shape", action="append", help="MxKxN (repeatable)")
    ap.add_argument("--variants", default=DEFAULT_VARIANTS)
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("this sweep needs a GPU")
    variants = args.variants.split(",")
    stream = torch.cuda.Stream()
    head = "| M x K x N | " + " | ".join(variants) + " | dense bf16 | best W4A16 / dense | max rel diff |"
    print(head)
    print("|" + "---|" * (len(variants) + 4))
    for shape in args.shape or DEFAULT_SHAPES:
        r = sweep(shape, variants, stream)
        best = min(r[v] for v in variants)
        cells = " | ".join(f"{r[v]:.1f}" for v in variants)
        print(f"| {shape} | {cells} | {r['dense']:.1f} | {r['dense'] / best:.2f}x | {r['max_rel_diff']:.1e} |",
              flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
