#!/usr/bin/env python3
"""Benchmark receipt for the MI355X ConvRot W4A4 and W4A16 paths at FLUX shapes.

Counterpart of the reference's TensorOps benchmark (/root/reference/benchmarks/tensorops.py):
the same receipt sections -- a correctness gate, then per shape a dense-bf16 control,
activation-preparation costs, kernel-only costs and complete linear-path costs, each
with wall-clock seconds per iteration (synchronized), best / median, total and
incremental peak device memory, and speedups against the dense control.

Kernel names map as follows (reference -> here):
  mppW4A4 (int8 A4 codes)               -> hipW4A4      (convrot_w4a4_gemm, int8 activations)
  legacyPackedMetalM32N32K64 (packed A4) -> hipW4A4Packed (convrot_w4a4_gemm, packed activations)
  mppW4A16                              -> hipW4A16     (convrot_w4a16_gemm)
  (none)                                -> hipW4A4Fp6   (convrot_w4a4_gemm_fp6: the A4 / W4 codes as FP6
                                           operands, same outputs; K % 128 == 0 shapes only)
The correctness gate checks the kernels against a float64 CPU evaluation of the eager
contract written here in torch (exact integer dot, then the float32 epilogue in the
reference's order), at the reference's gate sizes (37 x 256 -> 46).

    python benchmarks/tensorops.py [--shape MxKxN ...] [--iterations 3] [--output receipt.json]
"""

from __future__ import annotations

import argparse
import json
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT / "convrot-mlx_amd") not in sys.path:
    sys.path.insert(0, str(ROOT / "convrot-mlx_amd"))

import torch  # noqa: E402
import torch.nn.functional as F  # noqa: E402

import convrot_mlx_amd as api  # noqa: E402

GIB = 1024**3
MIB = 1024**2
GROUP = 256  # the reference's default ConvRot group size


def _dev() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("the ConvRot HIP kernels need a ROCm device")
    return torch.device("cuda:0")


def random_packed(rows: int, columns: int, gen: torch.Generator, dev) -> torch.Tensor:
    values = torch.randint(-7, 8, (rows, columns), dtype=torch.int8, device=dev, generator=gen)
    return api.pack_signed_int4(values)


def timed(function, *, iterations: int) -> dict[str, object]:
    """benchmarks/tensorops.py:52-81: a warm-up call, then per iteration the synchronized
    wall time and the device-memory peak (total, and above what was live before)."""
    warm = function()
    torch.cuda.synchronize()
    del warm
    seconds, total_peaks, incremental_peaks = [], [], []
    for _ in range(iterations):
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        started = time.perf_counter()
        output = function()
        torch.cuda.synchronize()
        seconds.append(time.perf_counter() - started)
        peak = torch.cuda.max_memory_allocated()
        total_peaks.append(peak / GIB)
        incremental_peaks.append(max(0, peak - before) / MIB)
        del output
    return {
        "seconds": [round(v, 6) for v in seconds],
        "bestSeconds": round(min(seconds), 6),
        "medianSeconds": round(statistics.median(seconds), 6),
        "totalPeakGiB": round(max(total_peaks), 6),
        "incrementalPeakMiB": round(max(incremental_peaks), 3),
    }


def _unpack_cpu(packed: torch.Tensor) -> torch.Tensor:
    """Two's-complement nibbles, low nibble = even column (core.py:108-120), on the CPU."""
    p = packed.cpu().to(torch.int16)
    lo, hi = p & 0xF, (p >> 4) & 0xF
    lo = torch.where(lo >= 8, lo - 16, lo)
    hi = torch.where(hi >= 8, hi - 16, hi)
    return torch.stack([lo, hi], dim=-1).reshape(packed.shape[0], -1).to(torch.int64)


def correctness_gate(gen: torch.Generator, dev) -> dict[str, object]:
    """benchmarks/tensorops.py:84-164, with the expected values computed on the CPU."""
    m, k, n = 37, 256, 46
    qact = random_packed(m, k, gen, dev)
    qweight_nk = random_packed(n, k, gen, dev)
    qweight = api.repack_nk_weight_for_cdna4(qweight_nk)
    xs = (torch.rand((m,), generator=gen, device=dev) * 0.19 + 0.01).float()
    ws = (torch.rand((n,), generator=gen, device=dev) * 0.19 + 0.01).float()
    bias = (torch.rand((n,), generator=gen, device=dev) * 2 - 1).float()

    a_codes, w_codes = _unpack_cpu(qact), _unpack_cpu(qweight_nk)
    dots = a_codes @ w_codes.T  # exact
    expected_a4 = ((dots.to(torch.float32) * xs.cpu()[:, None]) * ws.cpu()[None, :]) + bias.cpu()[None, :]
    actual_a4 = api.hip_w4a4_matmul(qact, qweight, xs, ws, bias, output_dtype=torch.float32, out_features=n)
    ones_m, ones_n = torch.ones((m,), device=dev), torch.ones((n,), device=dev)
    zero_n = torch.zeros((n,), device=dev)
    actual_int = api.hip_w4a4_matmul(qact, qweight, ones_m, ones_n, zero_n, output_dtype=torch.float32,
                                     out_features=n)
    activation = torch.randn((m, k), generator=gen, device=dev).to(torch.bfloat16)
    expected_a16 = ((activation.cpu().double() @ w_codes.double().T) * ws.cpu().double()[None, :]
                    + bias.cpu().double()[None, :])
    actual_a16 = api.hip_w4a16_matmul(activation, qweight, ws, bias, output_dtype=torch.float32, out_features=n)
    # FP6 operands: the same codes (the activation rows converted like weight columns)
    a6 = api.fp6_weight(api.repack_nk_weight_for_cdna4(qact), m, k)
    w6 = api.fp6_weight(qweight, n, k)
    actual_int6 = api.hip_w4a4_fp6_matmul(a6, w6, ones_m, ones_n, zero_n, output_dtype=torch.float32, rows=m,
                                          out_features=n, in_features=k)
    actual_a6 = api.hip_w4a4_fp6_matmul(a6, w6, xs, ws, bias, output_dtype=torch.float32, rows=m, out_features=n,
                                        in_features=k)
    torch.cuda.synchronize()

    integer_exact = bool(torch.equal(actual_int.cpu(), dots.to(torch.float32)))
    fp6_exact = bool(torch.equal(actual_int6.cpu(), dots.to(torch.float32))) and bool(
        torch.equal(actual_a6.cpu(), actual_a4.cpu()))
    a4_max = float((actual_a4.cpu() - expected_a4).abs().max())
    a16_max = float((actual_a16.cpu().double() - expected_a16).abs().max())
    # float32 accumulation bound for the W4A16 dot: K * 2^-24 * sum|a*w| * ws, plus one output ulp
    mag = (activation.cpu().double().abs() @ w_codes.double().abs().T)
    a16_tol = float((k * 2.0**-24 * mag * ws.cpu().double()[None, :]).max() + 2.0**-23 * expected_a16.abs().max())
    if not integer_exact:
        raise RuntimeError("W4A4 failed the exact integer-dot gate")
    if not fp6_exact:
        raise RuntimeError("W4A4 on FP6 operands failed the exact integer-dot / same-output gate")
    if a4_max > 1e-5:
        raise RuntimeError(f"W4A4 failed the FP32 epilogue gate: maximum error {a4_max}")
    if a16_max > a16_tol:
        raise RuntimeError(f"W4A16 failed the FP32 gate: maximum error {a16_max} > {a16_tol}")
    return {
        "hipW4A4ExactIntegerDot": integer_exact,
        "hipW4A4Fp6ExactIntegerDotAndSameOutput": fp6_exact,
        "hipW4A4Float32EpilogueMaximumAbsoluteError": a4_max,
        "hipW4A4Float32EpilogueTolerance": 1e-5,
        "hipW4A16MaximumAbsoluteError": a16_max,
        "hipW4A16Tolerance": a16_tol,
    }


def benchmark_shape(m: int, k: int, n: int, *, iterations: int, gen: torch.Generator, dev) -> dict[str, object]:
    """benchmarks/tensorops.py:167-295."""
    activation = torch.randn((m, k), generator=gen, device=dev).to(torch.bfloat16)
    dense_weight = torch.randn((n, k), generator=gen, device=dev).to(torch.bfloat16)
    qweight = api.repack_nk_weight_for_cdna4(random_packed(n, k, gen, dev))
    wscales = torch.full((n,), 0.125, dtype=torch.float32, device=dev)
    bias = torch.zeros((n,), dtype=torch.float32, device=dev)
    dense_bias = bias.to(torch.bfloat16)

    qact, xscales = api.hip_fused_prepare_convrot_activation(activation, GROUP)
    qact_i8, xscales_i8 = api.hip_fused_prepare_convrot_activation_i8(activation, GROUP)
    rotated = api.hip_fused_rotate_convrot_activation(activation, GROUP)
    fp6 = k % 128 == 0  # FP6 operands: the same codes as e2m3 values v/8 (this build's own path)
    if fp6:
        qact6, xscales6 = api.hip_fused_prepare_convrot_activation_fp6(activation, GROUP)
        w6 = api.fp6_weight(qweight, n, k)
    torch.cuda.synchronize()
    bf16 = torch.bfloat16

    dense = timed(lambda: F.linear(activation, dense_weight, dense_bias), iterations=iterations)
    packed_kernel = timed(lambda: api.hip_w4a4_matmul(qact, qweight, xscales, wscales, bias, output_dtype=bf16,
                                                      out_features=n), iterations=iterations)
    a4_kernel = timed(lambda: api.hip_w4a4_int8_matmul(qact_i8, qweight, xscales_i8, wscales, bias,
                                                       output_dtype=bf16, out_features=n), iterations=iterations)
    a16_kernel = timed(lambda: api.hip_w4a16_matmul(rotated, qweight, wscales, bias, output_dtype=bf16,
                                                    out_features=n), iterations=iterations)
    a4_preparation = timed(lambda: api.hip_fused_prepare_convrot_activation(activation, GROUP),
                           iterations=iterations)
    rotation = timed(lambda: api.compiled_regular_hadamard(activation, GROUP), iterations=iterations)
    fused_rotation = timed(lambda: api.hip_fused_rotate_convrot_activation(activation, GROUP),
                           iterations=iterations)
    a4_i8_preparation = timed(lambda: api.hip_fused_prepare_convrot_activation_i8(activation, GROUP),
                              iterations=iterations)

    def packed_path():
        prepared, scales = api.hip_fused_prepare_convrot_activation(activation, GROUP)
        return api.hip_w4a4_matmul(prepared, qweight, scales, wscales, bias, output_dtype=bf16, out_features=n)

    def a4_path():
        prepared, scales = api.hip_fused_prepare_convrot_activation_i8(activation, GROUP)
        return api.hip_w4a4_int8_matmul(prepared, qweight, scales, wscales, bias, output_dtype=bf16,
                                        out_features=n)

    def a16_path():
        prepared = api.hip_fused_rotate_convrot_activation(activation, GROUP)
        return api.hip_w4a16_matmul(prepared, qweight, wscales, bias, output_dtype=bf16, out_features=n)

    packed_path_result = timed(packed_path, iterations=iterations)
    a4_path_result = timed(a4_path, iterations=iterations)
    a16_path_result = timed(a16_path, iterations=iterations)
    extra = []
    if fp6:
        fp6_kernel = timed(lambda: api.hip_w4a4_fp6_matmul(qact6, w6, xscales6, wscales, bias, output_dtype=bf16,
                                                           rows=m, out_features=n, in_features=k),
                           iterations=iterations)
        fp6_preparation = timed(lambda: api.hip_fused_prepare_convrot_activation_fp6(activation, GROUP),
                                iterations=iterations)

        def fp6_path():
            prepared, scales = api.hip_fused_prepare_convrot_activation_fp6(activation, GROUP)
            return api.hip_w4a4_fp6_matmul(prepared, w6, scales, wscales, bias, output_dtype=bf16, rows=m,
                                           out_features=n, in_features=k)

        fp6_path_result = timed(fp6_path, iterations=iterations)
        extra = [fp6_kernel, fp6_path_result]
    for result in (packed_kernel, a4_kernel, a16_kernel, packed_path_result, a4_path_result, a16_path_result,
                   *extra):
        result["speedupVsDenseBf16"] = round(dense["medianSeconds"] / result["medianSeconds"], 3)
    a4_kernel["speedupVsPackedKernel"] = round(packed_kernel["medianSeconds"] / a4_kernel["medianSeconds"], 3)
    a16_kernel["speedupVsPackedKernel"] = round(packed_kernel["medianSeconds"] / a16_kernel["medianSeconds"], 3)
    a4_path_result["speedupVsPackedPath"] = round(
        packed_path_result["medianSeconds"] / a4_path_result["medianSeconds"], 3)
    a16_path_result["speedupVsPackedPath"] = round(
        packed_path_result["medianSeconds"] / a16_path_result["medianSeconds"], 3)
    receipt = {
        "shape": {"m": m, "k": k, "n": n},
        "denseBf16": dense,
        "activationPreparation": {
            "fusedHadamardAndA4Pack": a4_preparation,
            "fusedHadamardAndA4Int8": a4_i8_preparation,
            "compiledHadamardOnlyControl": rotation,
            "fusedHadamardOnly": fused_rotation,
        },
        "kernelOnly": {"hipW4A4Packed": packed_kernel, "hipW4A4": a4_kernel, "hipW4A16": a16_kernel},
        "completeLinearPath": {"hipW4A4Packed": packed_path_result, "hipW4A4": a4_path_result,
                               "hipW4A16": a16_path_result},
    }
    if fp6:
        fp6_kernel["speedupVsInt8Kernel"] = round(a4_kernel["medianSeconds"] / fp6_kernel["medianSeconds"], 3)
        fp6_path_result["speedupVsInt8Path"] = round(
            a4_path_result["medianSeconds"] / fp6_path_result["medianSeconds"], 3)
        receipt["activationPreparation"]["fusedHadamardAndA4Fp6"] = fp6_preparation
        receipt["kernelOnly"]["hipW4A4Fp6"] = fp6_kernel
        receipt["completeLinearPath"]["hipW4A4Fp6"] = fp6_path_result
    return receipt


def parse_shape(value: str) -> tuple[int, int, int]:
    """benchmarks/tensorops.py:298-308."""
    try:
        m, k, n = (int(part) for part in value.lower().split("x"))
    except (TypeError, ValueError) as error:
        raise argparse.ArgumentTypeError("shape must be MxKxN") from error
    if min(m, k, n) < 1 or k % 256 or n % 2:
        raise argparse.ArgumentTypeError("dimensions must be positive, K divisible by 256, and N even")
    return m, k, n


def main(argv: list[str] | None = None) -> dict:
    parser = argparse.ArgumentParser()
    parser.add_argument("--shape", action="append", type=parse_shape)
    parser.add_argument("--iterations", type=int, default=3)
    parser.add_argument("--output", type=Path)
    args = parser.parse_args(argv)
    if args.iterations < 1:
        raise ValueError("iterations must be positive")
    if args.output and (args.output.exists() or args.output.is_symlink()):
        raise FileExistsError(f"Refusing to overwrite benchmark receipt: {args.output}")
    shapes = args.shape or [(1536, 3072, 3072), (1536, 3072, 21504), (1536, 21504, 3072)]
    dev = _dev()
    gen = torch.Generator(device=dev)
    gen.manual_seed(20260823)
    receipt = {
        "schema": "convrot-mlx-amd.hip-tensorops-benchmark.v1",
        "platform": platform.platform(),
        "torchVersion": torch.__version__,
        "device": torch.cuda.get_device_name(dev),
        "convrotGroupSize": GROUP,
        "iterations": args.iterations,
        "correctness": correctness_gate(gen, dev),
        "benchmarks": [benchmark_shape(*shape, iterations=args.iterations, gen=gen, dev=dev) for shape in shapes],
    }
    rendered = json.dumps(receipt, indent=2, sort_keys=True) + "\n"
    if args.output:
        args.output.parent.mkdir(parents=True, exist_ok=True)
        args.output.write_text(rendered)
    print(rendered, end="")
    return receipt


if __name__ == "__main__":
    main()
