#!/usr/bin/env python3
"""W4A4 GEMM plan sweep on MI355X: every tile / kernel-kind plan of `convrot_w4a4_gemm`
against the automatic choice, over M and the FLUX linear shapes.

The W4A4 entry point (the counterpart of mpp_w4a4_int8_matmul,
/root/reference/src/convrot_mlx/core.py:1088-1120) picks a tile (256x256, 128x256,
256x128, 128x128 or 192x128) and a kernel kind (one workgroup per tile, or the
persistent stream-K kernel) from a cost model.  This script forces each plan through
CONVROT_GEMM_TILE / CONVROT_GEMM_SK, times it, and times the automatic choice, so the
model's regret (its time over the best plan's) can be read per shape.

Timing: 4 warm-up launches, then 24 launches cycling through 3 operand sets (so that not
every operand is L2-resident), bracketed by HIP events on the library's stream;
microseconds per launch.  int8 activation codes, bf16 output, few-row kernel disabled
(CONVROT_GEMM_SMALLM_MAX=0) so that every M runs the tiled kernels.

    python benchmarks/w4a4_plans.py [--m 256,512,...] [--out plans.jsonl]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT / "convrot-mlx_amd") not in sys.path:
    sys.path.insert(0, str(ROOT / "convrot-mlx_amd"))

import torch  # noqa: E402

from convrot_mlx_amd import _native as nat, core  # noqa: E402

KN = [(3072, 3072), (3072, 9216), (3072, 12288), (12288, 3072), (3072, 21504), (15360, 3072)]
PLANS = [("256x256w2x4", "0"), ("128x256w2x4", "0"), ("256x128w4x2", "0"), ("128x128w2x2", "0"),
         ("192x128w4x2", "0"), ("128x256w2x4", "1"), ("256x128w4x2", "1"), ("128x128w2x2", "1"),
         ("192x128w4x2", "1"), ("auto", "")]
SETS, WARMUP, LAUNCHES = 3, 4, 24


def _operands(M, K, N, dev):
    sets = []
    for s in range(SETS):
        g = torch.Generator(device=dev)
        g.manual_seed(s)
        wq = torch.randint(0, 256, core.cdna4_shape(N, K), dtype=torch.uint8, device=dev, generator=g)
        a = torch.randint(-7, 8, (M, K), dtype=torch.int8, device=dev, generator=g)
        xs, ws, b = torch.rand(M, device=dev), torch.rand(N, device=dev), torch.rand(N, device=dev)
        sets.append((a, xs, wq, ws, b, torch.empty((M, N), dtype=torch.bfloat16, device=dev)))
    return sets


def _time_plan(lib, stream, M, K, N, sets) -> float:
    def run(ops):
        a, xs, wq, ws, b, o = ops
        nat.check(lib.convrot_w4a4_gemm(nat.ptr(a), nat.ACT_INT8, nat.ptr(xs), nat.ptr(wq), nat.ptr(ws),
                                        nat.ptr(b), M, N, K, nat.ptr(o), nat.DTYPE_BF16, stream))

    for i in range(WARMUP):
        run(sets[i % SETS])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(LAUNCHES):
        run(sets[i % SETS])
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / LAUNCHES


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--m", default="256,512,1024,1536,2048,3072,4608")
    ap.add_argument("--out", default=None, help="also append one JSON line per shape here")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("this sweep needs a GPU")
    dev = torch.device("cuda:0")
    lib, stream = nat.load(), nat.stream_of(dev)
    os.environ["CONVROT_GEMM_SMALLM_MAX"] = "0"
    names = [f"{t}/{'sk' if k == '1' else 'dp'}" if t != "auto" else "auto" for t, k in PLANS]
    print("| M | K | N | " + " | ".join(names) + " | auto / best |")
    print("|" + "---:|" * (len(names) + 4))
    out = open(args.out, "a") if args.out else None
    total_auto = total_best = 0.0
    for M in (int(v) for v in args.m.split(",")):
        for K, N in KN:
            sets = _operands(M, K, N, dev)
            row = {"M": M, "K": K, "N": N}
            for (tile, sk), name in zip(PLANS, names):
                if tile == "auto":
                    os.environ.pop("CONVROT_GEMM_TILE", None)
                    os.environ.pop("CONVROT_GEMM_SK", None)
                else:
                    os.environ["CONVROT_GEMM_TILE"], os.environ["CONVROT_GEMM_SK"] = tile, sk
                row[name] = round(_time_plan(lib, stream, M, K, N, sets), 2)
            best = min(v for k, v in row.items() if "/" in k)
            total_auto += row["auto"]
            total_best += best
            cells = " | ".join(f"**{row[n]:.1f}**" if row[n] == best else f"{row[n]:.1f}" for n in names)
            print(f"| {M} | {K} | {N} | {cells} | {row['auto'] / best:.3f} |", flush=True)
            if out:
                out.write(json.dumps(row) + "\n")
                out.flush()
            del sets
    print(f"\nsum of auto times / sum of best-plan times: {total_auto / total_best:.4f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
