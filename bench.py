#!/usr/bin/env python3
"""Benchmark of the complete ConvRot W4A4 linear path on one MI355X.

Workload: the four FLUX double-block linears at
M=1536 tokens, group 64, bf16, with bias -- QKV 3072->9216, attention out
3072->3072, MLP 3072->12288 and 12288->3072.  Weights ~N(0, 0.02^2) with 1%
of input channels x10, activations ~N(0, 1) with 0.5% of channels x20
(synthetic, seeded).  One step = the complete path (fused prep kernel ->
INT8-MFMA GEMM with fused scale/bias epilogue) over all four linears, with
inputs and weights already resident in HBM.  Three independent buffer sets
(~630 MB) are cycled so the 256 MB Infinity Cache cannot hold a step's data.

`value` comes from K steps launched back to back with no event markers in the
queue; per-kernel durations come from HIP events around every launch over a
pass of max(K, 50) steps run between the warm-up and the timed region.

Prints ONE JSON line (the driver's contract).  Extra keys:
  roofline       dominant kernel (the W4A4 GEMM) vs the INT8 MFMA peak
  prep_roofline  the prep kernel vs HBM peak
  cpu_baseline   the CPU oracle (C restatement, 1 thread) on a bounded row sample
  dense_bf16_control  torch bf16 linear (hipBLASLt) on the same shapes
  flux_m4608     config 3's 4608x3072->12288 G=256 complete-path figure
  flux_m4608_column_shard_8  the same linear at one GPU's share of an 8-way column
                 split (4608x3072->1536), the per-GPU work of the sharded design
  w4a16_config4  config 4 (W4A16, M in {1, 8, 32}): int4-weight GB/s of the GEMM and
                 the complete path (rotation + GEMM), replayed from a HIP graph
  flux_dit_config5  config 5: one step of a random-init FLUX.1-dev DiT (1536 tokens),
                 dense bf16 vs every Linear as W4A4 ConvRotLinear G=64 -- eager and
                 HIP-graph step latency, relative L2 / cosine deviation
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
BF16_PEAK_TFLOPS = 2500.0
HBM_PEAK_GBPS = 8000.0

CONFIG2 = {"M": 1536, "G": 64, "shapes": [(3072, 9216), (3072, 3072), (3072, 12288), (12288, 3072)]}
CONFIG3_MLP = {"M": 4608, "G": 256, "K": 3072, "N": 12288}
CONFIG4 = {"G": 256, "Ms": (1, 8, 32), "shapes": [(3072, 12288), (12288, 3072)]}
TRAFFIC_FILE = ROOT / "profiles" / "gemm_w4a4_flux_m1536_traffic.json"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--sets", type=int, default=3, help="buffer sets cycled to defeat the Infinity Cache")
    ap.add_argument("--cpu-rows", type=int, default=288, help="rows per linear in the CPU-baseline sample (~11 s)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the dense control and the config-3/4/5 figures")
    ap.add_argument("--no-config5", action="store_true", help="skip the FLUX DiT step (config 5)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run one 256 MiB device copy first (counter calibration for rocprofv3 --pmc)")
    return ap.parse_args()


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path. "
              "Use --gpus 1.", file=sys.stderr)
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

    M, G = CONFIG2["M"], CONFIG2["G"]
    shapes = CONFIG2["shapes"]

    def outliers(gen, shape, std, frac, factor):
        x = torch.randn(shape, generator=gen, device=dev, dtype=torch.float32) * std
        k = shape[-1]
        idx = torch.randperm(k, generator=gen, device=dev)[: max(1, round(frac * k))]
        x[:, idx] *= factor
        return x.to(torch.bfloat16)

    gen = torch.Generator(device=dev)
    gen.manual_seed(20260823)
    sets = []
    for _ in range(args.sets):
        layers = []
        for K, N in shapes:
            w = outliers(gen, (N, K), 0.02, 0.01, 10.0)
            qw, ws = core.quantize_convrot_weight(w, G)
            wq = core.repack_nk_weight_for_cdna4(qw)
            bias = (torch.randn(N, generator=gen, device=dev) * 0.02).float()
            x = outliers(gen, (M, K), 1.0, 0.005, 20.0)
            out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            qact = torch.empty((M, K), dtype=torch.int8, device=dev)
            xs = torch.empty((M,), dtype=torch.float32, device=dev)
            layers.append(dict(K=K, N=N, w=w, qw=qw, wq=wq, ws=ws, bias=bias, x=x, out=out, qact=qact, xs=xs))
        sets.append(layers)
    torch.cuda.synchronize()

    lib = nat.load()
    stream = nat.stream_of(dev)

    def prep(L):
        nat.check(lib.convrot_prepare(nat.ptr(L["x"]), nat.DTYPE_BF16, M, L["K"], G, nat.PREP_INT8,
                                      nat.ptr(L["qact"]), nat.ptr(L["xs"]), stream))

    def gemm(L):
        nat.check(lib.convrot_w4a4_gemm(nat.ptr(L["qact"]), nat.ACT_INT8, nat.ptr(L["xs"]), nat.ptr(L["wq"]),
                                        nat.ptr(L["ws"]), nat.ptr(L["bias"]), M, L["N"], L["K"],
                                        nat.ptr(L["out"]), nat.DTYPE_BF16, stream))

    def step(i, events=None):
        for j, L in enumerate(sets[i % len(sets)]):
            if events is None:
                prep(L)
                gemm(L)
            else:
                e = events[j]
                e[0].record()
                prep(L)
                e[1].record()
                gemm(L)
                e[2].record()

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # Per-kernel durations: max(K, 50) steps with HIP events around every prep
    # and GEMM launch, on the launch stream.  This pass runs before the timed
    # region, so that region also starts on a warm GPU when K and W are small.
    ev_steps = max(args.steps, 50)
    ev = [[[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in shapes] for _ in range(ev_steps)]
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    for i in range(ev_steps):
        step(i, ev[i])
    torch.cuda.synchronize()
    t3 = time.perf_counter()
    ms_per_step_events = (t3 - t2) * 1e3 / ev_steps

    # Timed region: K steps back to back.  HIP event markers are kept out of it:
    # each one is a separate queue packet that costs ~4 us of dispatch gap, and 12
    # per step would lengthen the step by ~17 %.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    ops_per_step = sum(2 * M * K * N for K, N in shapes)
    tops = ops_per_step / (ms_per_step * 1e-3) / 1e12

    prep_ms = np.zeros(len(shapes))
    gemm_ms = np.zeros(len(shapes))
    for i in range(ev_steps):
        for j in range(len(shapes)):
            prep_ms[j] += ev[i][j][0].elapsed_time(ev[i][j][1])
            gemm_ms[j] += ev[i][j][1].elapsed_time(ev[i][j][2])
    prep_ms /= ev_steps
    gemm_ms /= ev_steps
    gemm_ops = np.array([2 * M * K * N for K, N in shapes], dtype=np.float64)
    gemm_tops = gemm_ops.sum() / (gemm_ms.sum() * 1e-3) / 1e12
    prep_bytes = np.array([3 * M * K + 4 * M for K, _ in shapes], dtype=np.float64)  # bf16 in, int8 out, f32 scales
    prep_gbps = prep_bytes.sum() / (prep_ms.sum() * 1e-3) / 1e9

    traffic = None
    if TRAFFIC_FILE.exists():
        try:
            traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch_avg")
        except (OSError, ValueError):
            traffic = None

    result = {
        "metric": "W4A4 linear TOPS at FLUX shapes (% INT8 MFMA peak); prep kernel HBM GB/s",
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,1) activations with 0.5% x20 channels, N(0,0.02^2) weights with 1% x10 "
                "input channels; random init)",
        "config": {
            "workload": "benchmark configs[1]: FLUX double-block W4A4 linears, M=1536, group 64, bf16, with bias: "
                        "3072->9216, 3072->3072, 3072->12288, 12288->3072; complete path prep+GEMM+epilogue",
            "M": M, "group_size": G, "shapes_KxN": shapes, "buffer_sets": args.sets,
            "pct_int8_peak": round(100.0 * tops / INT8_PEAK_TOPS, 2),
        },
        "roofline": {
            "kernel": "w4a4_gemm_kernel (INT8 MFMA + fused epilogue)",
            "bound": "mfma",
            "achieved": round(gemm_tops, 2),
            "peak": INT8_PEAK_TOPS,
            "unit": "TFLOP/s",
            "frac": round(gemm_tops / INT8_PEAK_TOPS, 4),
            "traffic": traffic,
            "per_shape_us": [round(t * 1e3, 2) for t in gemm_ms],
            "algorithmic": "2*M*N*K int ops per launch",
            "timing": f"HIP events around each launch, over a pass of {ev_steps} steps run just before the "
                      f"timed region (that pass: {ms_per_step_events:.4f} ms per step with the event markers)",
        },
        "prep_roofline": {
            "kernel": "prep_kernel (rotate+absmax+A4 quantize, int8 out)",
            "bound": "hbm",
            "achieved": round(prep_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(prep_gbps / HBM_PEAK_GBPS, 4),
            "per_shape_us": [round(t * 1e3, 2) for t in prep_ms],
            "algorithmic": "2*M*K (bf16 in) + M*K (int8 out) + 4*M bytes per launch",
        },
    }

    if not args.no_extras:
        result["dense_bf16_control"] = dense_control(torch, sets[0], M, shapes)
        result["dense_bf16_control"]["convrot_speedup"] = round(
            result["dense_bf16_control"]["ms_per_step"] / ms_per_step, 3)
        result["flux_m4608"] = config3_figure(torch, core, nat, dev)
        # One GPU's share of an 8-way column split of the same linear (no collective runs).
        result["flux_m4608_column_shard_8"] = config3_figure(torch, core, nat, dev, N=CONFIG3_MLP["N"] // 8)
        result["w4a16_config4"] = w4a16_figure(torch, core, nat, dev)
        if not args.no_config5:
            from examples.flux1_dev.dit import config5_figure

            torch.cuda.empty_cache()
            result["flux_dit_config5"] = config5_figure(steps=5)
            torch.cuda.empty_cache()

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(np, sets[0], M, G, args.cpu_rows, shapes)

    print(json.dumps(result), flush=True)
    return 0


def dense_control(torch, layers, M, shapes):
    import torch.nn.functional as F

    ws = [L["w"] for L in layers]
    bs = [L["bias"].to(torch.bfloat16) for L in layers]
    xs = [L["x"] for L in layers]
    for _ in range(3):
        for x, w, b in zip(xs, ws, bs):
            F.linear(x, w, b)
    torch.cuda.synchronize()
    n = 20
    t0 = time.perf_counter()
    for _ in range(n):
        for x, w, b in zip(xs, ws, bs):
            F.linear(x, w, b)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / n
    flops = sum(2 * M * K * N for K, N in shapes)
    return {"what": "torch.nn.functional.linear bf16 (hipBLASLt), same four shapes, single buffer set",
            "ms_per_step": round(ms, 4), "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
            "pct_bf16_peak": round(100 * flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 2)}


def config3_figure(torch, core, nat, dev, N=None):
    """Config 3's MLP-up linear, 4608x3072->12288, G=256: complete path, 3 buffer sets.
    With N given, the same linear at that output width (one GPU's column shard)."""
    c = CONFIG3_MLP
    M, K, G = c["M"], c["K"], c["G"]
    N = c["N"] if N is None else N
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    lib, stream = nat.load(), nat.stream_of(dev)
    bufs = []
    for _ in range(3):
        w = (torch.randn((N, K), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
        qw, ws = core.quantize_convrot_weight(w, G)
        bufs.append(dict(wq=core.repack_nk_weight_for_cdna4(qw), ws=ws,
                         bias=(torch.randn(N, generator=gen, device=dev) * 0.02).float(),
                         x=torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16),
                         qact=torch.empty((M, K), dtype=torch.int8, device=dev),
                         xs=torch.empty((M,), dtype=torch.float32, device=dev),
                         out=torch.empty((M, N), dtype=torch.bfloat16, device=dev)))

    def run(B):
        nat.check(lib.convrot_prepare(nat.ptr(B["x"]), nat.DTYPE_BF16, M, K, G, nat.PREP_INT8, nat.ptr(B["qact"]),
                                      nat.ptr(B["xs"]), stream))
        nat.check(lib.convrot_w4a4_gemm(nat.ptr(B["qact"]), nat.ACT_INT8, nat.ptr(B["xs"]), nat.ptr(B["wq"]),
                                        nat.ptr(B["ws"]), nat.ptr(B["bias"]), M, N, K, nat.ptr(B["out"]),
                                        nat.DTYPE_BF16, stream))

    for i in range(6):
        run(bufs[i % 3])
    torch.cuda.synchronize()
    n = 30
    t0 = time.perf_counter()
    for i in range(n):
        run(bufs[i % 3])
    torch.cuda.synchronize()
    us = (time.perf_counter() - t0) * 1e6 / n
    tops = 2 * M * N * K / (us * 1e-6) / 1e12
    return {"shape": f"{M}x{K}->{N} G={G}", "us_per_linear": round(us, 2), "tops": round(tops, 2),
            "pct_int8_peak": round(100 * tops / INT8_PEAK_TOPS, 2)}


def w4a16_figure(torch, core, nat, dev):
    """Config 4: W4A16 (rotation prep -> int4-weight GEMM with the scale/bias epilogue), G=256,
    bf16, M in {1, 8, 32}.  A ~10 us launch is shorter than the host's launch interval, so the
    launches are captured in a HIP graph and replayed; every replay's output is checked against
    the eager one.  Weights cycle through > 512 MB so each launch streams its int4 weights from
    HBM.  Headline bytes per GEMM launch: N*K/2 (int4 weights)."""
    lib, stream_fn = nat.load(), nat.stream_of
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
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
                nat.check(lib.convrot_w4a16_gemm(nat.ptr(rot), nat.DTYPE_BF16, nat.ptr(weights[i]), nat.ptr(ws),
                                                 nat.ptr(bias), M, N, K, nat.ptr(y), nat.DTYPE_BF16, stream_fn(dev)))

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
    return {"what": "W4A16 GEMM (int4 weights N*K/2 bytes per launch) and complete path, G=256, bf16; "
                    "HIP-graph replays, weights cycled through > 512 MB",
            "shapes": figures}


def cpu_baseline(np, layers, M, G, rows, shapes):
    """The CPU oracle (C restatement, single thread) over a bounded sample: `rows` rows of every
    linear, complete path (rotation + A4 quantization + integer GEMM + epilogue).  Weight codes
    come from the GPU quantization (bit-identical to the oracle's, which the tests check)."""
    from oracle import oracle as orc

    orc.build()
    ops = 0
    seconds = 0.0
    for L in layers:
        K, N = L["K"], L["N"]
        x = L["x"][:rows].contiguous().view(__import__("torch").int16).cpu().numpy().view(np.uint16)
        w_codes = orc.unpack_signed_int4(L["qw"].cpu().numpy())
        ws = L["ws"].cpu().numpy()
        b = L["bias"].cpu().numpy()
        t0 = time.perf_counter()
        a_codes, xs = orc.prepare_codes(x, "bfloat16", G)
        orc.w4a4_matmul_codes(a_codes, w_codes, xs, ws, b, "bfloat16")
        seconds += time.perf_counter() - t0
        ops += 2 * rows * K * N
    tops = ops / seconds / 1e12
    cpu = platform.processor() or platform.machine()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(tops, 6), "unit": "TOPS", "cores": 1, "kind": "port",
            "sample": f"{rows} rows x each of the 4 config-2 linears (K,N)={shapes}, complete path, "
                      f"{seconds:.1f} s on 1 thread of {cpu} (host has {os.cpu_count()} logical CPUs)"}


if __name__ == "__main__":
    sys.exit(main())
