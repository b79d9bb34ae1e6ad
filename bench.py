#!/usr/bin/env python3
"""Benchmark of the complete ConvRot W4A4 linear path on one MI355X.

Workload (the north-star configuration): the six FLUX
linears at M=4608 tokens (4096 image + 512 text), group 256, bf16, with bias --
QKV 3072->9216, attention out 3072->3072, MLP 3072->12288 and 12288->3072, and
the fused single-block linears 3072->21504 and 15360->3072.  Weights
~N(0, 0.02^2) with 1% of input channels x10, activations ~N(0, 1) with 0.5% of
channels x20, bias ~N(0, 0.02^2) (synthetic, seeded).  One step = the complete
path ConvRotLinear runs at these sizes (fused prep kernel writing FP6 operands
-> FP6-MFMA GEMM with the fused scale/bias epilogue; the A4/W4 codes as FP6
values give the INT8 path's outputs bit for bit) over all six linears, inputs
and weights already resident in HBM.  A step
touches ~1.2 GB of distinct buffers, over four times the 256 MB Infinity
Cache, so no linear finds its operands cached from its previous step.

`value` comes from K steps launched back to back with no event markers in the
queue; per-kernel durations come from HIP events recorded on the launch stream
around every launch, over a pass of max(K, 30) steps run between the warm-up
and the timed region.

Prints ONE JSON line (the driver's contract).  Extra keys:
  roofline        the W4A4 GEMM (dominant kernel) vs the FP6 MFMA peak it runs on (and the
                  INT8 peak the metric is quoted against), per shape too
  int8_operands   the same step on INT8 operands (prep int8 codes -> INT8-MFMA GEMM)
  prep_roofline   the prep kernel vs the HBM peak, per shape too
  per_shape       complete-path latency and TOPS of each linear
  dense_bf16_control  torch bf16 linear (hipBLASLt) on the same six shapes
  cpu_baseline    the CPU oracle (C restatement of the eager path) on every host thread,
                  median of 3, over a bounded row sample of the same six linears
  config2_m1536   configs[1] (M=1536, G=64, four double-block shapes), complete path
  flux_m4608_column_shard_8  4608x3072->1536, one GPU's share of an 8-way column split
  w4a16_config4   configs[3] (W4A16, M in {1, 8, 32}): int4-weight GB/s, HIP-graph replays
  flux_dit_config5  configs[4]: one step of a random-init FLUX.1-dev DiT, dense vs W4A4, with the
                  Linears' weight bytes and the step's peak device memory
  video_transfer_shapes  the reference's published projection shapes (M = 7800 / 8800), complete
                  path on MI355X beside its M4 Pro latencies (context, other hardware)
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT / "convrot-mlx_amd"), str(ROOT)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

INT8_PEAK_TOPS = 5000.0  # MI355X dense INT8 MFMA (TOPS)
FP6_PEAK_TOPS = 10100.0  # MI355X dense FP6 MFMA
BF16_PEAK_TFLOPS = 2500.0
HBM_PEAK_GBPS = 8000.0

CONFIG3 = {"M": 4608, "G": 256,
           "shapes": [(3072, 9216), (3072, 3072), (3072, 12288), (12288, 3072), (3072, 21504), (15360, 3072)]}
CONFIG2 = {"M": 1536, "G": 64, "shapes": [(3072, 9216), (3072, 3072), (3072, 12288), (12288, 3072)]}
CONFIG4 = {"G": 256, "Ms": (1, 8, 32), "shapes": [(3072, 12288), (12288, 3072)]}
# The reference's only published single-projection timings (docs/benchmarks/video-transfer.md:15-20):
# (model, M, K, N, median complete-projection seconds of its MPP W4A4 path on an M4 Pro).
VIDEO_SHAPES = [("Wan 2.2 A14B", 7800, 5120, 5120, 0.103394), ("Wan expansion", 7800, 5120, 13824, 0.290321),
                ("Wan contraction", 7800, 13824, 5120, 0.352751), ("LTX 2.5", 8800, 4096, 4096, 0.075218),
                ("LTX expansion", 8800, 4096, 16384, 0.297969), ("LTX contraction", 8800, 16384, 4096, 0.408371)]
TRAFFIC_FILE = ROOT / "profiles" / "gemm_w4a4_fp6_flux_m4608_traffic.json"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--sets", type=int, default=1, help="buffer sets cycled (one set is ~1.2 GB already)")
    ap.add_argument("--cpu-rows-per-thread", type=int, default=48,
                    help="rows of each linear per host thread in the CPU-baseline sample (~4 s a repetition)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the dense control and the config-2/4/5 figures")
    ap.add_argument("--no-config5", action="store_true", help="skip the FLUX DiT step (config 5)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run one 256 MiB device copy first (counter calibration for rocprofv3 --pmc)")
    ap.add_argument("--operands", choices=("fp6", "int8"), default="fp6",
                    help="operands of the measured path: FP6 (what ConvRotLinear runs at these sizes) or INT8")
    ap.add_argument("--workload", choices=("config3", "config2"), default="config3",
                    help="the measured workload: configs[2] (the headline, M=4608 G=256) or configs[1] (M=1536 "
                         "G=64, for profiling); the extras are the same either way")
    return ap.parse_args()


def outliers(torch, gen, dev, shape, std, frac, factor):
    x = torch.randn(shape, generator=gen, device=dev, dtype=torch.float32) * std
    k = shape[-1]
    idx = torch.randperm(k, generator=gen, device=dev)[: max(1, round(frac * k))]
    x[:, idx] *= factor
    return x.to(torch.bfloat16)


def make_layers(torch, core, dev, M, G, shapes, seed, sets=1, fp6=True):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    out = []
    for _ in range(sets):
        layers = []
        for K, N in shapes:
            w = outliers(torch, gen, dev, (N, K), 0.02, 0.01, 10.0)
            qw, ws = core.quantize_convrot_weight(w, G)
            wq = core.repack_nk_weight_for_cdna4(qw)
            layers.append(dict(
                K=K, N=N, w=w, qw=qw, wq=wq, ws=ws,
                w6=core.fp6_weight(wq, N, K) if fp6 else None,
                w6c=core.fp6_weight_compact(wq, N, K) if fp6 else None,
                form=core.fp6_weight_form(M, N) if fp6 else None,  # the form ConvRotLinear caches
                a6=torch.empty(core.fp6_shape(M, K), dtype=torch.uint8, device=dev) if fp6 else None,
                bias=(torch.randn(N, generator=gen, device=dev) * 0.02).float(),
                x=outliers(torch, gen, dev, (M, K), 1.0, 0.005, 20.0),
                out=torch.empty((M, N), dtype=torch.bfloat16, device=dev),
                qact=torch.empty((M, K), dtype=torch.int8, device=dev),
                xs=torch.empty((M,), dtype=torch.float32, device=dev)))
        out.append(layers)
    return out


class PathRunner:
    """Launches of the complete path (prep -> GEMM) of one set of linears on one stream,
    on FP6 or INT8 operands, with optional HIP events around every launch.  FP6 weights are
    the form ConvRotLinear caches for the shape (core.fp6_weight_form: the compact 0.5-byte
    form unless a setting asks for the 0.75-byte operand blocks), or with
    full_weights the operand blocks everywhere."""

    def __init__(self, nat, dev, M, G, fp6=True, full_weights=False):
        import torch

        self.nat, self.lib, self.stream, self.M, self.G = nat, nat.load(), nat.stream_of(dev), M, G
        self.fp6, self.full = fp6, full_weights
        self.work = torch.zeros(int(self.lib.convrot_w4a4_workspace_bytes()), dtype=torch.uint8, device=dev)

    def prep(self, L):
        nat = self.nat
        mode, out = (nat.PREP_FP6, L["a6"]) if self.fp6 else (nat.PREP_INT8, L["qact"])
        nat.check(self.lib.convrot_prepare(nat.ptr(L["x"]), nat.DTYPE_BF16, self.M, L["K"], self.G, mode,
                                           nat.ptr(out), nat.ptr(L["xs"]), self.stream))

    def gemm(self, L):
        nat = self.nat
        if self.fp6 and not self.full and L["form"] == "compact":
            nat.check(self.lib.convrot_w4a4_gemm_fp6_compact(
                nat.ptr(L["a6"]), nat.ptr(L["xs"]), nat.ptr(L["w6c"]), nat.ptr(L["ws"]), nat.ptr(L["bias"]), self.M,
                L["N"], L["K"], None, None, 0, 1, nat.ptr(L["out"]), nat.DTYPE_BF16, self.stream))
        elif self.fp6:
            nat.check(self.lib.convrot_w4a4_gemm_fp6(nat.ptr(L["a6"]), nat.ptr(L["xs"]), nat.ptr(L["w6"]),
                                                     nat.ptr(L["ws"]), nat.ptr(L["bias"]), self.M, L["N"], L["K"],
                                                     nat.ptr(L["out"]), nat.DTYPE_BF16, self.stream))
        else:  # with the stream-K workspace, as ConvRotLinear calls it
            nat.check(self.lib.convrot_w4a4_gemm_ws(nat.ptr(L["qact"]), nat.ACT_INT8, nat.ptr(L["xs"]),
                                                    nat.ptr(L["wq"]), nat.ptr(L["ws"]), nat.ptr(L["bias"]), self.M,
                                                    L["N"], L["K"], None, None, 0, 1, nat.ptr(self.work),
                                                    self.work.numel(), nat.ptr(L["out"]), nat.DTYPE_BF16,
                                                    self.stream))

    def step(self, layers, events=None):
        for j, L in enumerate(layers):
            if events is None:
                self.prep(L)
                self.gemm(L)
            else:
                e = events[j]
                e[0].record()
                self.prep(L)
                e[1].record()
                self.gemm(L)
                e[2].record()


def measure_path(torch, np, runner, sets, shapes, M, steps, warmup, ev_min=30):
    """(ms per step from `steps` marker-free steps, per-shape prep and GEMM ms from a pass of
    max(steps, ev_min) steps with HIP events around each launch, that pass's ms per step)."""
    for i in range(warmup):
        runner.step(sets[i % len(sets)])
    torch.cuda.synchronize()
    ev_steps = max(steps, ev_min)
    ev = [[[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in shapes] for _ in range(ev_steps)]
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    for i in range(ev_steps):
        runner.step(sets[i % len(sets)], ev[i])
    torch.cuda.synchronize()
    ms_events = (time.perf_counter() - t2) * 1e3 / ev_steps
    # Timed region: K steps back to back, no event markers in the queue (each marker is a
    # separate queue packet with a few microseconds of dispatch gap).
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        runner.step(sets[i % len(sets)])
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / steps
    prep_ms = np.zeros(len(shapes))
    gemm_ms = np.zeros(len(shapes))
    for i in range(ev_steps):
        for j in range(len(shapes)):
            prep_ms[j] += ev[i][j][0].elapsed_time(ev[i][j][1])
            gemm_ms[j] += ev[i][j][1].elapsed_time(ev[i][j][2])
    return ms_per_step, prep_ms / ev_steps, gemm_ms / ev_steps, ms_events, ev_steps


def prep_back_to_back(torch, nat, dev, M, G, shapes, fp6, reps=20, cold_bytes=600 << 20):
    """Per-shape prep duration without event markers between launches: `reps` launches of one
    shape back to back between two HIP events, their inputs (and outputs) cycled through more
    than `cold_bytes` of distinct bf16 rows (so no launch finds its rows in the 256 MB
    Infinity Cache, and each writes a buffer of its own, as each linear of a step does).  The
    markers of measure_path's pass each add a dispatch gap of a few microseconds to the launch
    they bracket."""
    lib, stream = nat.load(), nat.stream_of(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    mode = nat.PREP_FP6 if fp6 else nat.PREP_INT8
    out_us = []
    for K, _ in shapes:
        nbuf = max(2, -(-cold_bytes // (M * K * 2)))
        xs = [torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16) for _ in range(nbuf)]
        outs = [torch.empty(int(lib.convrot_fp6_bytes(M, K)) if fp6 else M * K, dtype=torch.uint8, device=dev)
                for _ in range(nbuf)]
        scs = [torch.empty((M,), dtype=torch.float32, device=dev) for _ in range(nbuf)]

        def launch(i):
            nat.check(lib.convrot_prepare(nat.ptr(xs[i % nbuf]), nat.DTYPE_BF16, M, K, G, mode,
                                          nat.ptr(outs[i % nbuf]), nat.ptr(scs[i % nbuf]), stream))

        for i in range(nbuf):
            launch(i)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for i in range(reps):
            launch(i)
        e1.record()
        torch.cuda.synchronize()
        out_us.append(e0.elapsed_time(e1) * 1e3 / reps)
        del xs, outs, scs
    return out_us


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}): every box of this build has one GPU "
              "and the sharded design is not built. Use --gpus 1.", file=sys.stderr)
        return 2
    import numpy as np
    import torch

    from convrot_mlx_amd import _native as nat
    from convrot_mlx_amd import core

    nat.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.calibrate_copy:
        src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    W = CONFIG3 if args.workload == "config3" else CONFIG2
    M, G, shapes = W["M"], W["G"], W["shapes"]
    fp6 = args.operands == "fp6"
    # configs[1]'s four linears total ~315 MB: three buffer sets keep a step out of the Infinity Cache
    sets = make_layers(torch, core, dev, M, G, shapes, seed=20260823,
                       sets=args.sets if args.workload == "config3" else max(args.sets, 3), fp6=True)
    torch.cuda.synchronize()
    runner = PathRunner(nat, dev, M, G, fp6=fp6)
    ms_per_step, prep_ms, gemm_ms, ms_events, ev_steps = measure_path(
        torch, np, runner, sets, shapes, M, args.steps, args.warmup)

    ops = np.array([2.0 * M * K * N for K, N in shapes])
    tops = ops.sum() / (ms_per_step * 1e-3) / 1e12
    gemm_tops = ops / (gemm_ms * 1e-3) / 1e12
    gemm_agg = ops.sum() / (gemm_ms.sum() * 1e-3) / 1e12
    out_bytes = 0.75 if fp6 else 1.0  # FP6 (6 bits) or int8 codes per feature
    prep_bytes = np.array([(2.0 + out_bytes) * M * K + 4 * M for K, _ in shapes])  # bf16 in, codes out, f32 scales
    prep_b2b_us = np.array(prep_back_to_back(torch, nat, dev, M, G, shapes, fp6))
    prep_gbps = prep_bytes / (prep_b2b_us * 1e-6) / 1e9
    prep_agg = prep_bytes.sum() / (prep_b2b_us.sum() * 1e-6) / 1e9
    peak = FP6_PEAK_TOPS if fp6 else INT8_PEAK_TOPS

    traffic, traffic_note = None, "no FETCH_SIZE/WRITE_SIZE profile for this workload"
    if TRAFFIC_FILE.exists() and args.workload == "config3" and fp6:
        try:
            tj = json.loads(TRAFFIC_FILE.read_text())
            traffic = tj.get("hbm_bytes_per_launch_avg")
            traffic_note = (f"not measured by this run: calibrated FETCH_SIZE + WRITE_SIZE per GEMM launch from "
                            f"{TRAFFIC_FILE.relative_to(ROOT)} ({tj.get('algorithmic_bytes_per_launch_avg')} "
                            "algorithmic bytes per launch)")
        except (OSError, ValueError):
            traffic = None

    result = {
        "metric": "W4A4 linear TOPS at FLUX shapes (% INT8 MFMA peak); prep kernel HBM GB/s",
        "value": round(float(tops), 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp6" if fp6 else "int8",
        "data": "synthetic (seeded N(0,1) activations with 0.5% x20 channels, N(0,0.02^2) weights with 1% x10 "
                "input channels, N(0,0.02^2) bias; random init)",
        "config": {
            "workload": ("benchmark configs[2]: FLUX W4A4 linears at M=4608 (4096 image + 512 text tokens), "
                         "group 256, bf16, with bias: 3072->9216, 3072->3072, 3072->12288, 12288->3072, "
                         "3072->21504, 15360->3072; complete path prep+GEMM+epilogue"
                         if args.workload == "config3" else
                         "benchmark configs[1]: FLUX double-block W4A4 linears at M=1536 (1024 image + 512 "
                         "text tokens), group 64, bf16, with bias: 3072->9216, 3072->3072, 3072->12288, "
                         "12288->3072; complete path prep+GEMM+epilogue"),
            "M": M, "group_size": G, "shapes_KxN": shapes, "buffer_sets": args.sets,
            "operands": ("FP6: the A4/W4 codes v as e2m3 values v/8, multiplied by the FP6 MFMA with block "
                         "scales 2^3 (exact integer products, float32 sums exact below 2^24): the INT8 path's "
                         "outputs bit for bit" if fp6 else "INT8: A4 codes as int8, W4 nibbles unpacked to int8"),
            "pct_int8_peak": round(100.0 * tops / INT8_PEAK_TOPS, 2),
        },
        "roofline": {
            "kernel": ("W4A4 GEMM on FP6 operands, compact weights (w4a4_gemm_fp6_kernel<..., CW=true>: "
                       "v_mfma_scale_f32_16x16x128_f8f6f4 + fused epilogue)" if fp6 else
                       "W4A4 GEMM (w4a4_gemm_agpr_kernel, 288x192 and 256x256 tiles: INT8 MFMA + fused epilogue)"),
            "bound": "mfma",
            "achieved": round(float(gemm_agg), 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(float(gemm_agg) / peak, 4),
            "frac_of_int8_peak": round(float(gemm_agg) / INT8_PEAK_TOPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_note,
            "per_shape_us": [round(t * 1e3, 2) for t in gemm_ms],
            "per_shape_tops": [round(float(t), 1) for t in gemm_tops],
            "per_shape_frac": [round(float(t) / peak, 4) for t in gemm_tops],
            "algorithmic": "2*M*N*K int ops per launch; achieved = sum of ops / sum of launch durations; peak = "
                           + ("the dense FP6 MFMA peak the kernel runs on" if fp6 else "the dense INT8 MFMA peak"),
            "timing": f"HIP events on the launch stream around each launch, over a pass of {ev_steps} steps run "
                      f"just before the timed region (that pass: {ms_events:.4f} ms per step with the markers)",
        },
        "prep_roofline": {
            "kernel": "prep_kernel (rotate + absmax + A4 quantize, " + ("FP6 codes out)" if fp6 else "int8 codes out)"),
            "bound": "hbm",
            "achieved": round(float(prep_agg), 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(float(prep_agg) / HBM_PEAK_GBPS, 4),
            "per_shape_us": [round(float(t), 2) for t in prep_b2b_us],
            "per_shape_GBps": [round(float(g), 1) for g in prep_gbps],
            "in_step_us": [round(t * 1e3, 2) for t in prep_ms],
            "algorithmic": ("2*M*K (bf16 in) + 0.75*M*K (FP6 out)" if fp6 else "2*M*K (bf16 in) + M*K (int8 out)")
                           + " + 4*M bytes per launch",
            "timing": "20 launches of each shape back to back between two HIP events, inputs and outputs "
                      "cycled through > 600 MB of distinct rows; in_step_us: HIP events around each launch in "
                      "the step pass (each marker adds a dispatch gap of a few microseconds)",
        },
        "per_shape": [{"K": K, "N": N, "path_us": round((p + g) * 1e3, 2),
                       "path_tops": round(float(o / ((p + g) * 1e-3) / 1e12), 1)}
                      for (K, N), p, g, o in zip(shapes, prep_ms, gemm_ms, ops)],
    }

    if not args.no_extras:
        other = PathRunner(nat, dev, M, G, fp6=not fp6)
        o_ms, o_prep, o_gemm, _, _ = measure_path(torch, np, other, sets, shapes, M, args.steps, 3)
        result["int8_operands" if fp6 else "fp6_operands"] = {
            "what": "the same step and buffers on " + ("INT8" if fp6 else "FP6") + " operands",
            "ms_per_step": round(o_ms, 4), "tops": round(float(ops.sum() / (o_ms * 1e-3) / 1e12), 1),
            "pct_int8_peak": round(100.0 * ops.sum() / (o_ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 2),
            "gemm_per_shape_us": [round(t * 1e3, 2) for t in o_gemm],
            "prep_per_shape_us": [round(t * 1e3, 2) for t in o_prep]}
        if fp6:
            full = PathRunner(nat, dev, M, G, fp6=True, full_weights=True)
            f_ms, f_prep, f_gemm, _, _ = measure_path(torch, np, full, sets, shapes, M, args.steps, 3)
            result["fp6_full_weights"] = {
                "what": "the same step on the 1536-byte FP6 weight blocks (0.75 byte a weight) for every shape, "
                        "instead of the forms ConvRotLinear caches (forms used: "
                        + ", ".join(L["form"] for L in sets[0]) + "; compact: 0.5 byte a weight, expanded "
                        "in registers)",
                "ms_per_step": round(f_ms, 4), "tops": round(float(ops.sum() / (f_ms * 1e-3) / 1e12), 1),
                "gemm_per_shape_us": [round(t * 1e3, 2) for t in f_gemm]}
    if not args.no_extras:
        dense = dense_control(torch, sets[0], M, shapes)
        dense["convrot_speedup"] = round(dense["ms_per_step"] / ms_per_step, 3)
        result["dense_bf16_control"] = dense
        result["config2_m1536"] = config2_figure(torch, np, core, nat, dev, fp6)
        result["flux_m4608_column_shard_8"] = shard_figure(torch, np, core, nat, dev, fp6)
        result["w4a16_config4"] = w4a16_figure(torch, core, nat, dev)
        result["video_transfer_shapes"] = video_figure(torch, np, core, nat, dev)
        if not args.no_config5:
            from examples.flux1_dev.dit import config5_figure

            torch.cuda.empty_cache()
            result["flux_dit_config5"] = config5_figure(steps=5)
            torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(np, sets[0], M, G, args.cpu_rows_per_thread, shapes)

    print(json.dumps(result), flush=True)
    return 0


def dense_control(torch, layers, M, shapes):
    """torch bf16 F.linear (hipBLASLt) on the same shapes and operands (dense bf16 weights);
    HIP events around each call, 20 steps after 3 warm-up steps."""
    import torch.nn.functional as F

    ws = [L["w"] for L in layers]
    bs = [L["bias"].to(torch.bfloat16) for L in layers]
    xs = [L["x"] for L in layers]
    for _ in range(3):
        for x, w, b in zip(xs, ws, bs):
            F.linear(x, w, b)
    torch.cuda.synchronize()
    n = 20
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(ws) + 1)] for _ in range(n)]
    t0 = time.perf_counter()
    for i in range(n):
        ev[i][0].record()
        for j, (x, w, b) in enumerate(zip(xs, ws, bs)):
            F.linear(x, w, b)
            ev[i][j + 1].record()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / n
    per = [sum(ev[i][j].elapsed_time(ev[i][j + 1]) for i in range(n)) / n for j in range(len(ws))]
    flops = sum(2 * M * K * N for K, N in shapes)
    return {"what": "torch.nn.functional.linear bf16 (hipBLASLt), the same six shapes and bf16 weights/activations",
            "ms_per_step": round(ms, 4), "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
            "pct_bf16_peak": round(100 * flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 2),
            "per_shape_us": [round(t * 1e3, 2) for t in per]}


def config2_figure(torch, np, core, nat, dev, fp6):
    """the four double-block linears at M=1536, G=64, complete path; three buffer
    sets (~630 MB) cycled so the Infinity Cache cannot hold a step's data."""
    M, G, shapes = CONFIG2["M"], CONFIG2["G"], CONFIG2["shapes"]
    sets = make_layers(torch, core, dev, M, G, shapes, seed=1536, sets=3, fp6=fp6)
    runner = PathRunner(nat, dev, M, G, fp6=fp6)
    ms, prep_ms, gemm_ms, _, _ = measure_path(torch, np, runner, sets, shapes, M, 50, 5)
    ops = np.array([2.0 * M * K * N for K, N in shapes])
    del sets
    torch.cuda.empty_cache()
    return {"shapes_KxN": shapes, "M": M, "group_size": G, "operands": "fp6" if fp6 else "int8",
            "ms_per_step": round(ms, 4),
            "tops": round(float(ops.sum() / (ms * 1e-3) / 1e12), 1),
            "gemm_tops": round(float(ops.sum() / (gemm_ms.sum() * 1e-3) / 1e12), 1),
            "gemm_per_shape_us": [round(t * 1e3, 2) for t in gemm_ms],
            "prep_per_shape_us": [round(t * 1e3, 2) for t in prep_ms]}


def video_figure(torch, np, core, nat, dev):
    """The complete W4A4 path (G=256, FP6 operands, as ConvRotLinear runs these sizes) and torch's
    dense bf16 linear on the reference's published video-transformer projections; two buffer sets
    cycled (each set is 0.2-0.8 GB).  The reference's figures are an M4 Pro's, listed as context."""
    G = 256
    rows = []
    for name, M, K, N, ref_s in VIDEO_SHAPES:
        sets = make_layers(torch, core, dev, M, G, [(K, N)], seed=M + K + N, sets=2, fp6=True)
        runner = PathRunner(nat, dev, M, G, fp6=True)
        ms, prep_ms, gemm_ms, _, _ = measure_path(torch, np, runner, sets, [(K, N)], M, 20, 3)
        dense = dense_control(torch, sets[0], M, [(K, N)])
        ops = 2.0 * M * K * N
        rows.append({"shape": f"{name}: M={M} K={K} N={N}", "path_us": round(ms * 1e3, 2),
                     "tops": round(ops / (ms * 1e-3) / 1e12, 1),
                     "pct_int8_peak": round(100 * ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 2),
                     "prep_us": round(float(prep_ms[0]) * 1e3, 2), "gemm_us": round(float(gemm_ms[0]) * 1e3, 2),
                     "dense_bf16_us": round(dense["ms_per_step"] * 1e3, 2),
                     "speedup_vs_dense_bf16": round(dense["ms_per_step"] / ms, 3),
                     "reference_m4pro_mpp_w4a4_us": round(ref_s * 1e6, 1)})
        del sets
        torch.cuda.empty_cache()
    return {"what": "complete W4A4 path (fused prep writing FP6 operands + FP6 GEMM + epilogue, G=256, bf16, "
                    "with bias) vs torch bf16 F.linear on the reference's published projection shapes; the "
                    "reference column is its M4 Pro MPP W4A4 median (docs/benchmarks/video-transfer.md:15-20), "
                    "other hardware, context only",
            "shapes": rows}


def shard_figure(torch, np, core, nat, dev, fp6):
    """4608x3072->1536, G=256: one GPU's share of an 8-way column split of the MLP-up linear
    (no collective runs; three buffer sets)."""
    M, G, shapes = CONFIG3["M"], CONFIG3["G"], [(3072, 12288 // 8)]
    sets = make_layers(torch, core, dev, M, G, shapes, seed=3, sets=3, fp6=fp6)
    runner = PathRunner(nat, dev, M, G, fp6=fp6)
    ms, prep_ms, gemm_ms, _, _ = measure_path(torch, np, runner, sets, shapes, M, 50, 5)
    ops = 2.0 * M * 3072 * 1536
    del sets
    torch.cuda.empty_cache()
    return {"shape": f"{M}x3072->1536 G={G}", "operands": "fp6" if fp6 else "int8",
            "us_per_linear": round(ms * 1e3, 2),
            "tops": round(ops / (ms * 1e-3) / 1e12, 1), "gemm_us": round(float(gemm_ms[0]) * 1e3, 2),
            "pct_int8_peak": round(100 * ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 2)}


def w4a16_figure(torch, core, nat, dev):
    """W4A16 (rotation prep -> int4-weight GEMM with the scale/bias epilogue), G=256,
    bf16, M in {1, 8, 32}.  A ~10 us launch is shorter than the host's launch interval, so the
    launches are captured in a HIP graph and replayed; every replay's output is checked against
    the eager one.  Weights cycle through > 512 MB so each launch streams its int4 weights from
    HBM.  The GEMM is convrot_w4a16_gemm_ws with a stream-K workspace, as ConvRotLinear calls it
    (12288->3072 at M=32 splits K over workgroups).  Headline bytes per GEMM launch: N*K/2 (int4
    weights)."""
    lib, stream_fn = nat.load(), nat.stream_of
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    work = torch.zeros(int(lib.convrot_w4a4_workspace_bytes()), dtype=torch.uint8, device=dev)
    G = CONFIG4["G"]
    figures = []
    for K, N in CONFIG4["shapes"]:
        wbytes = N * K // 2
        nsets = max(2, -(-600 * 2 ** 20 // wbytes))
        weights = [torch.randint(0, 256, core.cdna4_shape(N, K), dtype=torch.uint8, device=dev, generator=gen)
                   for _ in range(nsets)]
        ws = torch.rand(N, generator=gen, device=dev) * 0.01
        bias = torch.randn(N, generator=gen, device=dev) * 0.02
        for M in CONFIG4["Ms"]:
            x = torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16)
            rot = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
            y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

            def prep():
                nat.check(lib.convrot_prepare(nat.ptr(x), nat.DTYPE_BF16, M, K, G, nat.PREP_ROTATE, nat.ptr(rot),
                                              None, stream_fn(dev)))

            def gemm(i):
                nat.check(lib.convrot_w4a16_gemm_ws(nat.ptr(rot), nat.DTYPE_BF16, nat.ptr(weights[i]), nat.ptr(ws),
                                                    nat.ptr(bias), M, N, K, None, None, 0, 1, nat.ptr(work),
                                                    work.numel(), nat.ptr(y), nat.DTYPE_BF16, stream_fn(dev)))

            timings = {}
            for name, with_prep in (("gemm", False), ("path", True)):
                prep()
                gemm(nsets - 1)
                torch.cuda.synchronize()
                ref = y.clone()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    for i in range(nsets):
                        if with_prep:
                            prep()
                        gemm(i)
                for _ in range(2):
                    graph.replay()
                    torch.cuda.synchronize()
                    if not torch.equal(y, ref):
                        raise RuntimeError("W4A16 graph replay differs from the eager result")
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                reps = 4
                e0.record()
                for _ in range(reps):
                    graph.replay()
                e1.record()
                torch.cuda.synchronize()
                timings[name] = e0.elapsed_time(e1) * 1e3 / (reps * nsets)
                del graph
            gbps = wbytes / (timings["gemm"] * 1e-6) / 1e9
            figures.append({"M": M, "K": K, "N": N, "gemm_us": round(timings["gemm"], 2),
                            "path_us": round(timings["path"], 2), "int4_weight_GBps": round(gbps, 1),
                            "pct_hbm": round(100 * gbps / HBM_PEAK_GBPS, 1)})
        del weights
    return {"what": "W4A16 GEMM (int4 weights N*K/2 bytes per launch; convrot_w4a16_gemm_ws with a stream-K "
                    "workspace, as ConvRotLinear runs it) and complete path, G=256, bf16; HIP-graph replays, "
                    "weights cycled through > 512 MB",
            "shapes": figures}


def cpu_baseline(np, layers, M, G, rows_per_thread, shapes):
    """The CPU oracle (the C restatement of the reference's eager path: rotation + A4
    quantization + integer GEMM + epilogue) on every host thread this process may use, over a
    bounded sample -- the first rows_per_thread x threads rows of each linear -- median of 3
    repetitions.  Each thread runs whole rows; the C calls release the GIL.  Weight codes come
    from the GPU quantization (bit-identical to the oracle's, which the tests check)."""
    from concurrent.futures import ThreadPoolExecutor

    import torch

    from oracle import oracle as orc

    orc.build()
    threads = orc.cpu_threads()
    rows = min(M, rows_per_thread * threads)
    work = []
    for L in layers:
        x = L["x"][:rows].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        work.append((x, orc.unpack_signed_int4(L["qw"].cpu().numpy()), L["ws"].cpu().numpy(),
                     L["bias"].cpu().numpy()))
    chunks = [(r0, min(rows, r0 + rows_per_thread)) for r0 in range(0, rows, rows_per_thread)]

    def one(args):
        x, w_codes, ws, b, r0, r1 = args
        a_codes, xs = orc.prepare_codes(x[r0:r1], "bfloat16", G)
        orc.w4a4_matmul_codes(a_codes, w_codes, xs, ws, b, "bfloat16")

    reps = []
    with ThreadPoolExecutor(max_workers=threads) as pool:
        for _ in range(3):
            t0 = time.perf_counter()
            for x, w_codes, ws, b in work:
                list(pool.map(one, [(x, w_codes, ws, b, r0, r1) for r0, r1 in chunks]))
            reps.append(time.perf_counter() - t0)
    seconds = float(np.median(reps))
    ops = sum(2.0 * rows * K * N for K, N in shapes)
    cpu = platform.processor() or platform.machine()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(ops / seconds / 1e12, 6), "unit": "TOPS", "cores": threads, "kind": "port",
            "sample": f"the first {rows} of the {M} rows of each of the {len(shapes)} linears, complete path "
                      f"(prep + integer GEMM + epilogue), {threads} threads of {cpu} "
                      f"(os.cpu_count() = {os.cpu_count()}), median of 3 repetitions: "
                      f"{', '.join(f'{r:.2f}' for r in reps)} s"}


if __name__ == "__main__":
    sys.exit(main())
