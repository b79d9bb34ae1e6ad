"""Per-step kernel time of the DiT, by category, from a rocprofv3 kernel trace.

`dit.py --variant dense|convrot` launches a marker kernel (torch's spin kernel)
right before its timed steps; this script keeps the dispatches after the last
marker, divides by the step count and groups kernels into ConvRot GEMM / prep,
dense GEMM, attention, layer norm and the remaining elementwise work.

    rocprofv3 --kernel-trace -f csv -d OUT/dense -o run -- python3 examples/flux1_dev/dit.py --variant dense --steps 3
    rocprofv3 --kernel-trace -f csv -d OUT/convrot -o run -- python3 examples/flux1_dev/dit.py --variant convrot --steps 3
    python3 examples/flux1_dev/trace_summary.py OUT/dense OUT/convrot --steps 3
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import sys


def category(name: str) -> str:
    low = name.lower()
    if "w4a4_gemm" in name or "w4a4_smallm" in name:
        return "convrot_gemm"
    if "prep_kernel" in name:
        return "convrot_prep"
    if "convrot" in name:
        return "convrot_other"
    if "attn" in low or "flash" in low or "fmha" in low:
        return "attention"
    if name.startswith(("Cijk", "Custom_Cijk")) or "gemm" in low:
        return "dense_gemm"
    if "norm" in low:
        return "layernorm"
    return "elementwise"


def summarize(trace_dir: str, steps: int, top: int = 12) -> dict:
    files = glob.glob(f"{trace_dir}/**/*kernel_trace.csv", recursive=True)
    if not files:
        raise SystemExit(f"no kernel_trace.csv under {trace_dir}")
    rows = sorted(csv.DictReader(open(files[0])), key=lambda r: int(r["Start_Timestamp"]))
    marks = [i for i, r in enumerate(rows) if "sleep" in r["Kernel_Name"].lower() or "spin" in r["Kernel_Name"].lower()]
    if not marks:
        raise SystemExit(f"no marker kernel in {files[0]}")
    rows = rows[marks[-1] + 1:]
    cats: dict[str, float] = {}
    names: dict[str, list] = {}
    for r in rows:
        ms = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e6 / steps
        name = r["Kernel_Name"]
        cats[category(name)] = cats.get(category(name), 0.0) + ms
        acc = names.setdefault(name, [0.0, 0])
        acc[0] += ms
        acc[1] += 1
    kernels = sorted(names.items(), key=lambda kv: -kv[1][0])[:top]
    return {
        "dispatches_per_step": len(rows) // steps,
        "kernel_ms_per_step": round(sum(cats.values()), 3),
        "categories_ms": {c: round(t, 3) for c, t in sorted(cats.items(), key=lambda kv: -kv[1])},
        "top_kernels": [{"name": n[:120], "ms": round(t, 3), "calls": c // steps,
                         "avg_us": round(t * 1e3 * steps / c, 1)} for n, (t, c) in kernels],
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("dirs", nargs="+", help="rocprofv3 -d directories, one per variant")
    ap.add_argument("--steps", type=int, default=3)
    args = ap.parse_args()
    out = {d: summarize(d, args.steps) for d in args.dirs}
    json.dump(out, sys.stdout, indent=1)
    print()
    return 0


if __name__ == "__main__":
    sys.exit(main())
