"""Benchmark receipts for the ConvRot HIP kernels."""
