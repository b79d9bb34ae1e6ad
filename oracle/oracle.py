"""CPU oracle for the ConvRot W4A4 / W4A16 path -- TEST INFRASTRUCTURE ONLY.

This module is the checker the HIP kernels are compared against.  It is never
imported by the product package (`convrot_mlx_amd`); only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` use it.

Two halves:

* arithmetic (rotation, quantization, both matmul epilogues) is the C
  restatement in `convrot_oracle.c`, loaded here through ctypes;
* the integer/byte layout functions are restated in numpy below.

Every function cites the reference function it restates
(`/root/reference/src/convrot_mlx/core.py`).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
DTYPE_CODES = {"float32": DTYPE_F32, "float16": DTYPE_F16, "bfloat16": DTYPE_BF16}

INT4_MAX = 7  # core.py:34


def build(force: bool = False) -> Path:
    """Compile the C restatement with the committed Makefile."""
    src = HERE / "convrot_oracle.c"
    if force or not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < src.stat().st_mtime:
        subprocess.run(["make", "-s", "-B", "-C", str(HERE), "liboracle.so"], check=True)
    return LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.cr_oracle_regular_hadamard.argtypes = [vp, i32, i64, i64, i32, vp, vp]
        L.cr_oracle_quantize_rowwise.argtypes = [vp, i32, i64, i64, vp, vp, vp]
        L.cr_oracle_prepare.argtypes = [vp, i32, i64, i64, i32, vp, vp, vp]
        L.cr_oracle_w4a4_matmul.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i32, vp, vp]
        L.cr_oracle_w4a4_epilogue.argtypes = [vp, vp, vp, vp, i64, i64, i32, vp]
        L.cr_oracle_w4a16_matmul.argtypes = [vp, i32, vp, vp, vp, i64, i64, i64, i32, vp, vp, vp]
        L.cr_oracle_f32_to_dtype.argtypes = [vp, i64, i32, vp]
        L.cr_oracle_modulate.argtypes = [vp, i32, i64, i64, vp, vp, i64, ctypes.c_float, vp]
        L.cr_oracle_gelu.argtypes = [vp, i32, i64, vp]
        L.cr_oracle_dtype_to_f32.argtypes = [vp, i64, i32, vp]
        L.cr_f32_to_bf16.argtypes = [ctypes.c_float]
        L.cr_f32_to_bf16.restype = ctypes.c_uint16
        L.cr_f32_to_f16.argtypes = [ctypes.c_float]
        L.cr_f32_to_f16.restype = ctypes.c_uint16
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


# ----------------------------------------------------------------- dtypes
# Activations travel as uint16 bit patterns (bf16 / f16) or float32.


def from_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to `dtype` (RNE).  Returns uint16 bits or float32.

    Mirrors `mx.array(float32).astype(mx.bfloat16)` used to build every test
    input in /root/reference/tests/test_core.py (e.g. :56-58).
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dtype == "float32":
        return x.copy()
    out = np.empty(x.shape, dtype=np.uint16)
    lib().cr_oracle_f32_to_dtype(_ptr(x), x.size, DTYPE_CODES[dtype], _ptr(out))
    return out


def to_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "float32":
        return np.ascontiguousarray(x, dtype=np.float32).copy()
    x = np.ascontiguousarray(x, dtype=np.uint16)
    out = np.empty(x.shape, dtype=np.float32)
    lib().cr_oracle_dtype_to_f32(_ptr(x), x.size, DTYPE_CODES[dtype], _ptr(out))
    return out


# ----------------------------------------------------------------- arithmetic


def _validate_group_size(group_size: int) -> None:
    """core.py:50-61."""
    if group_size < 4:
        raise ValueError(f"Regular Hadamard size must be a power of 4, got {group_size}")
    value = group_size
    while value > 1 and value % 4 == 0:
        value //= 4
    if value != 1:
        raise ValueError(f"Regular Hadamard size must be a power of 4, got {group_size}")


def regular_hadamard(x: np.ndarray, dtype: str, group_size: int = 256) -> np.ndarray:
    """core.py:64-94 with per-op dtype rounding (C restatement)."""
    _validate_group_size(group_size)
    x = np.ascontiguousarray(x)
    rows = int(np.prod(x.shape[:-1])) if x.ndim > 1 else 1
    K = x.shape[-1]
    if K % group_size:
        raise ValueError(f"features {K} not divisible by ConvRot group size {group_size}")
    out = np.empty_like(x)
    work = np.empty(K, dtype=np.float32)
    rc = lib().cr_oracle_regular_hadamard(_ptr(x), DTYPE_CODES[dtype], rows, K, group_size, _ptr(out), _ptr(work))
    assert rc == 0
    return out


def quantize_rowwise_codes(x: np.ndarray, dtype: str) -> tuple[np.ndarray, np.ndarray]:
    """quantize_signed_int4_rowwise (core.py:149-158) before packing: int8 codes, f32 scales."""
    x = np.ascontiguousarray(x)
    if x.ndim != 2:
        raise ValueError(f"rowwise int4 quantization expects 2D input, got {x.shape}")
    rows, K = x.shape
    codes = np.empty((rows, K), dtype=np.int8)
    scales = np.empty(rows, dtype=np.float32)
    work = np.empty(K, dtype=np.float32)
    lib().cr_oracle_quantize_rowwise(_ptr(x), DTYPE_CODES[dtype], rows, K, _ptr(codes), _ptr(scales), _ptr(work))
    return codes, scales


def quantize_signed_int4_rowwise(x: np.ndarray, dtype: str) -> tuple[np.ndarray, np.ndarray]:
    """core.py:149-158: packed codes and float32 scales."""
    codes, scales = quantize_rowwise_codes(x, dtype)
    return pack_signed_int4(codes), scales


def prepare_codes(x: np.ndarray, dtype: str, group_size: int = 256) -> tuple[np.ndarray, np.ndarray]:
    """prepare_convrot_activation (core.py:161-167) before packing."""
    _validate_group_size(group_size)
    x = np.ascontiguousarray(x)
    rows, K = x.shape
    if K % group_size:
        raise ValueError(f"features {K} not divisible by ConvRot group size {group_size}")
    codes = np.empty((rows, K), dtype=np.int8)
    scales = np.empty(rows, dtype=np.float32)
    work = np.empty(K, dtype=np.float32)
    rc = lib().cr_oracle_prepare(_ptr(x), DTYPE_CODES[dtype], rows, K, group_size, _ptr(codes), _ptr(scales), _ptr(work))
    assert rc == 0
    return codes, scales


def prepare_convrot_activation(x: np.ndarray, dtype: str, group_size: int = 256) -> tuple[np.ndarray, np.ndarray]:
    """core.py:161-167: packed A4 codes and float32 row scales."""
    codes, scales = prepare_codes(x, dtype, group_size)
    return pack_signed_int4(codes), scales


def quantize_convrot_weight(weight: np.ndarray, dtype: str, group_size: int = 256) -> tuple[np.ndarray, np.ndarray]:
    """core.py:514-527: identical math to the activation path, NK packed output."""
    if weight.ndim != 2:
        raise ValueError(f"ConvRot weight must be 2D, got {weight.shape}")
    if weight.shape[-1] % group_size:
        raise ValueError(
            f"in_features {weight.shape[-1]} not divisible by ConvRot group size {group_size}"
        )
    return prepare_convrot_activation(weight, dtype, group_size)


def modulate(x: np.ndarray, dtype: str, shift: np.ndarray, scale: np.ndarray, rows_per_vector: int,
             eps: float = 1e-6) -> np.ndarray:
    """Input transform of the fused modulated producer (no reference counterpart; the
    adaLN pattern `(1 + scale) * layer_norm(x) + shift`), C restatement:
    LayerNorm moments as float64 sums in the order fixed in convrot_oracle.c, then
    per-op dtype rounding."""
    x = np.ascontiguousarray(x)
    shift = np.ascontiguousarray(shift)
    scale = np.ascontiguousarray(scale)
    rows, K = x.shape
    out = np.empty_like(x)
    rc = lib().cr_oracle_modulate(_ptr(x), DTYPE_CODES[dtype], rows, K, _ptr(shift), _ptr(scale),
                                  rows_per_vector, eps, _ptr(out))
    assert rc == 0
    return out


def gelu_tanh(x: np.ndarray, dtype: str) -> np.ndarray:
    """Input transform of the fused GELU producer (no reference counterpart: the FLUX MLP
    activation nn.GELU(approximate="tanh")), C restatement: the fixed float32 sequence of
    convrot_oracle.c (exp by Cody-Waite reduction and a degree-7 polynomial, fma, one IEEE
    division), rounded once to the dtype."""
    x = np.ascontiguousarray(x)
    out = np.empty_like(x)
    rc = lib().cr_oracle_gelu(_ptr(x), DTYPE_CODES[dtype], x.size, _ptr(out))
    assert rc == 0
    return out


def gelu_producer_rows(head: np.ndarray | None, x: np.ndarray, dtype: str) -> np.ndarray:
    """The rows the fused GELU producer prepares: [head | gelu_tanh(x)] along features."""
    g = gelu_tanh(x, dtype)
    return g if head is None or head.shape[-1] == 0 else np.ascontiguousarray(np.concatenate([head, g], axis=-1))


def gated_residual(lin: np.ndarray, residual: np.ndarray, gate: np.ndarray | None, rows_per_gate: int,
                   dtype: str) -> np.ndarray:
    """Consumer of the gated-residual GEMM epilogue (no reference counterpart: a DiT
    block's `x + gate * linear(...)`, two eager elementwise ops):
        out[m] = dt(residual[m] + dt(gate[m // rows_per_gate] * lin[m]))
    on [M, N] arrays of dtype bits (float32 values for "float32"), each op one float32
    IEEE operation rounded once to dtype (numpy float32 arithmetic, then from_f32).
    gate: [G, N] rows, or None for dt(residual + lin)."""
    lin32 = to_f32(lin, dtype)
    res32 = to_f32(residual, dtype)
    if gate is None:
        return from_f32(res32 + lin32, dtype)
    rows = np.arange(lin.shape[0]) // rows_per_gate
    g32 = to_f32(np.ascontiguousarray(gate), dtype)[rows]
    prod = to_f32(from_f32(g32 * lin32, dtype), dtype)
    return from_f32(res32 + prod, dtype)


def w4a4_matmul_codes(a_codes, w_codes, xscales, wscales, bias, out_dtype: str, want_dots: bool = False):
    """reference_w4a4_matmul (core.py:1155-1171) on unpacked codes (w in NK orientation)."""
    a_codes = np.ascontiguousarray(a_codes, dtype=np.int8)
    w_codes = np.ascontiguousarray(w_codes, dtype=np.int8)
    M, K = a_codes.shape
    N = w_codes.shape[0]
    assert w_codes.shape[1] == K
    xs = np.ascontiguousarray(xscales, dtype=np.float32)
    ws = np.ascontiguousarray(wscales, dtype=np.float32)
    b = np.ascontiguousarray(bias, dtype=np.float32)
    out = np.empty((M, N), dtype=np.float32 if out_dtype == "float32" else np.uint16)
    dots = np.empty((M, N), dtype=np.int32) if want_dots else None
    lib().cr_oracle_w4a4_matmul(
        _ptr(a_codes), _ptr(w_codes), _ptr(xs), _ptr(ws), _ptr(b), M, N, K,
        DTYPE_CODES[out_dtype], _ptr(out), _ptr(dots) if want_dots else None,
    )
    return (out, dots) if want_dots else out


def w4a4_dots_exact(a_codes, w_codes) -> np.ndarray:
    """Exact int32 dots a_codes [M, K] . w_codes [N, K]^T through a float32 matmul, the way
    reference_w4a4_matmul (core.py:1166-1167) forms them: every product of two codes in
    [-8, 7] is an integer of magnitude <= 64 and every partial sum an integer of magnitude
    <= 64 K < 2^24, so each float32 add (or fma) is exact in any order and the BLAS result
    equals the int64 dot.  Rows go through in slabs to bound the float32 copies."""
    a_codes = np.ascontiguousarray(a_codes, dtype=np.int8)
    w_codes = np.ascontiguousarray(w_codes, dtype=np.int8)
    M, K = a_codes.shape
    assert w_codes.shape[1] == K and 64 * K < 2 ** 24, "float32 dots are exact only while 64 K < 2^24"
    wf = w_codes.astype(np.float32).T.copy()
    out = np.empty((M, w_codes.shape[0]), dtype=np.int32)
    slab = max(1, (1 << 26) // max(1, K + w_codes.shape[0]))
    for m0 in range(0, M, slab):
        out[m0:m0 + slab] = np.matmul(a_codes[m0:m0 + slab].astype(np.float32), wf)
    return out


def w4a4_epilogue(dots, xscales, wscales, bias, out_dtype: str) -> np.ndarray:
    """The float32 epilogue of reference_w4a4_matmul (core.py:1168-1171) on given int32 dots."""
    dots = np.ascontiguousarray(dots, dtype=np.int32)
    M, N = dots.shape
    xs = np.ascontiguousarray(xscales, dtype=np.float32)
    ws = np.ascontiguousarray(wscales, dtype=np.float32)
    b = np.ascontiguousarray(bias, dtype=np.float32)
    assert xs.shape == (M,) and ws.shape == (N,) and b.shape == (N,)
    out = np.empty((M, N), dtype=np.float32 if out_dtype == "float32" else np.uint16)
    lib().cr_oracle_w4a4_epilogue(_ptr(dots), _ptr(xs), _ptr(ws), _ptr(b), M, N, DTYPE_CODES[out_dtype], _ptr(out))
    return out


def w4a4_matmul_codes_large(a_codes, w_codes, xscales, wscales, bias, out_dtype: str) -> np.ndarray:
    """w4a4_matmul_codes for full-size products: exact dots by w4a4_dots_exact, then the C
    epilogue (the same float32 sequence as cr_oracle_w4a4_matmul)."""
    return w4a4_epilogue(w4a4_dots_exact(a_codes, w_codes), xscales, wscales, bias, out_dtype)


def reference_w4a4_matmul(qact, qweight_nk, xscales, wscales, bias, out_dtype: str):
    """core.py:1155-1171 on packed operands."""
    return w4a4_matmul_codes(unpack_signed_int4(qact), unpack_signed_int4(qweight_nk), xscales, wscales, bias, out_dtype)


def w4a16_matmul_codes(act, act_dtype: str, w_codes, wscales, bias, out_dtype: str):
    """mpp_w4a16_matmul (core.py:1123-1152) numerics on NK codes.

    Returns (out, dots_f32, abs_sum_f32) -- the last is sum_k |a_k * w_k| per
    output, which sizes the summation-order tolerance of the comparison.
    """
    act = np.ascontiguousarray(act)
    w_codes = np.ascontiguousarray(w_codes, dtype=np.int8)
    M, K = act.shape
    N = w_codes.shape[0]
    ws = np.ascontiguousarray(wscales, dtype=np.float32)
    b = np.ascontiguousarray(bias, dtype=np.float32)
    out = np.empty((M, N), dtype=np.float32 if out_dtype == "float32" else np.uint16)
    dots = np.empty((M, N), dtype=np.float32)
    mag = np.empty((M, N), dtype=np.float32)
    lib().cr_oracle_w4a16_matmul(
        _ptr(act), DTYPE_CODES[act_dtype], _ptr(w_codes), _ptr(ws), _ptr(b), M, N, K,
        DTYPE_CODES[out_dtype], _ptr(out), _ptr(dots), _ptr(mag),
    )
    return out, dots, mag


# ----------------------------------------------------------------- layouts


def pack_signed_int4(values: np.ndarray) -> np.ndarray:
    """core.py:97-105: two's-complement nibbles, even column in the low nibble."""
    values = np.asarray(values)
    if values.shape[-1] % 2:
        raise ValueError(f"last dimension must be even, got {values.shape[-1]}")
    v = values.astype(np.int32)
    lo = v[..., 0::2] & 0x0F
    hi = v[..., 1::2] & 0x0F
    return (lo | (hi << 4)).astype(np.uint8)


def unpack_signed_int4(packed: np.ndarray) -> np.ndarray:
    """core.py:108-120: nibbles to int8 in [-8, 7], low nibble first."""
    d = np.asarray(packed).astype(np.int32)
    lo = d & 0x0F
    hi = (d >> 4) & 0x0F
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    out = np.stack([lo, hi], axis=-1).reshape(*d.shape[:-1], d.shape[-1] * 2)
    return out.astype(np.int8)


def repack_nk_weight_for_mpp(qweight: np.ndarray) -> np.ndarray:
    """core.py:123-133: N x packed-K -> K x packed-N (requires even N)."""
    if qweight.ndim != 2:
        raise ValueError(f"MPP weight repack expects a 2D tensor, got {qweight.shape}")
    unpacked = unpack_signed_int4(qweight)
    if unpacked.shape[0] % 2:
        raise ValueError(f"MPP int4 packing requires even out_features, got {unpacked.shape[0]}")
    return pack_signed_int4(unpacked.T)


def repack_mpp_weight_to_nk(qweight: np.ndarray) -> np.ndarray:
    """core.py:136-146: K x packed-N -> N x packed-K (requires even K)."""
    if qweight.ndim != 2:
        raise ValueError(f"MPP weight repack expects a 2D tensor, got {qweight.shape}")
    unpacked = unpack_signed_int4(qweight)
    if unpacked.shape[0] % 2:
        raise ValueError(f"row-major int4 packing requires even in_features, got {unpacked.shape[0]}")
    return pack_signed_int4(unpacked.T)


# CDNA4 tile layout (no reference counterpart; defined by this build).
# Blocks of 16 output rows x 128 features, 1024 bytes each, ordered
# [K_pad/128][N_pad/16].  Inside a block, byte  16*L + 4*c + j  (lane
# L = 16*q + r, dword c, byte j) holds row r's codes for features
#   k = 32*q + 8*c + j      (low nibble)
#   k = 32*q + 8*c + j + 4  (high nibble)
# N is zero-padded to a multiple of 16 and K to a multiple of 128.
CDNA4_BLOCK_N, CDNA4_BLOCK_K = 16, 128


def cdna4_shape(n: int, k: int) -> tuple[int, int, int]:
    npad = -(-n // CDNA4_BLOCK_N) * CDNA4_BLOCK_N
    kpad = -(-k // CDNA4_BLOCK_K) * CDNA4_BLOCK_K
    return kpad // CDNA4_BLOCK_K, npad // CDNA4_BLOCK_N, 1024


def codes_to_cdna4(w_codes: np.ndarray) -> np.ndarray:
    """NK int8 codes [N, K] -> CDNA4 packed blocks (see the layout comment)."""
    N, K = w_codes.shape
    kb, nb, _ = cdna4_shape(N, K)
    full = np.zeros((nb * 16, kb * 128), dtype=np.int32)
    full[:N, :K] = w_codes
    # full[n, k] with n = 16*nblk + r, k = 128*kblk + 32*q + 8*c + j + 4*h
    t = full.reshape(nb, 16, kb, 4, 4, 2, 4)  # nblk, r, kblk, q, c, h, j
    lo = t[..., 0, :] & 0xF
    hi = t[..., 1, :] & 0xF
    byte = (lo | (hi << 4)).astype(np.uint8)  # nblk, r, kblk, q, c, j
    # -> kblk, nblk, q, r, c, j
    return np.ascontiguousarray(byte.transpose(2, 0, 3, 1, 4, 5)).reshape(kb, nb, 1024)


def cdna4_to_codes(blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    """Exact inverse of codes_to_cdna4, dropping the padding."""
    kb, nb, _ = blocks.shape
    b = blocks.reshape(kb, nb, 4, 16, 4, 4).astype(np.int32)  # kblk, nblk, q, r, c, j
    lo = b & 0xF
    hi = (b >> 4) & 0xF
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    t = np.stack([lo, hi], axis=-2)  # kblk, nblk, q, r, c, h, j
    full = t.transpose(1, 3, 0, 2, 4, 5, 6).reshape(nb * 16, kb * 128)
    return full[:n, :k].astype(np.int8)


def nk_to_cdna4(qweight_nk: np.ndarray) -> np.ndarray:
    n = qweight_nk.shape[0]
    return codes_to_cdna4(unpack_signed_int4(qweight_nk)) if n else np.zeros((0, 0, 1024), np.uint8)


def cdna4_to_nk(blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    return pack_signed_int4(cdna4_to_codes(blocks, n, k))


# FP6 operand layout (no reference counterpart; defined by this build), for
# activations (rows) and weights (columns) alike.  A code v in [-8, 7] is
# stored as the OCP MX e2m3 encoding (sign bit 5, exponent bits 4..3 with bias
# 1, mantissa bits 2..0) of v/8: for |v| <= 7 the subnormal with mantissa |v|,
# for -8 the normal -1.0; zero is +0.  The GEMM multiplies both operands by
# 2^3 (the MFMA's block scales), so products are v*w exactly.  Blocks of 16
# rows x 128 features, 1536 bytes each, ordered [K/128][R_pad/16]; lane
# L = 16*q + r of a block holds row r's features 32*q + i (i = 0..31), feature
# i at bits 6i..6i+5 of a 192-bit little-endian stream whose bytes 0..15 sit
# at 16*L and bytes 16..23 at 1024 + 8*L.  Rows are zero-padded to a multiple
# of 16; K must be a multiple of 128.
FP6_BLOCK_BYTES = 1536


def e2m3_value(code) -> np.ndarray:
    """Value of an e2m3 code by the format's definition: (-1)^s * 2^(e-1) * (1 + m/8)
    for e > 0, (-1)^s * m/8 for e = 0."""
    c = np.asarray(code, dtype=np.int64)
    s, e, m = (c >> 5) & 1, (c >> 3) & 3, c & 7
    mag = np.where(e > 0, np.ldexp(1.0 + m / 8.0, (e - 1).astype(np.int32)), m / 8.0)
    return np.where(s == 1, -mag, mag)


def fp6_code(v) -> np.ndarray:
    """FP6 field of integer codes in [-8, 7]: the e2m3 encoding of v/8 (zero as +0)."""
    v = np.asarray(v, dtype=np.int64)
    if v.size and (v.min() < -8 or v.max() > 7):
        raise ValueError("FP6 codes hold the integers -8 .. 7 only")
    mag = np.where(v == -8, 8, np.abs(v)).astype(np.uint64)  # -8/8 = -1.0 is e=1, m=0: bits 0b001000
    return mag | np.where(v < 0, 32, 0).astype(np.uint64)


def fp6_value(code) -> np.ndarray:
    """Integer code of an FP6 field (8 times its e2m3 value)."""
    return e2m3_value(code) * 8.0


def codes_to_fp6(codes: np.ndarray) -> np.ndarray:
    """Row-major int8 codes [R, K] (K % 128 == 0) -> FP6 blocks [K/128, R_pad/16, 1536]."""
    R, K = codes.shape
    if K % 128:
        raise ValueError(f"FP6 layout requires K divisible by 128, got {K}")
    rb, kb = -(-R // 16), K // 128
    full = np.zeros((rb * 16, K), np.int8)
    full[:R] = codes
    c = fp6_code(full).reshape(rb, 16, kb, 4, 4, 8)  # rblk, r, kblk, q, chunk of 8 fields, field
    words = (c << (6 * np.arange(8, dtype=np.uint64))).sum(-1)  # 48-bit chunks (disjoint bit fields)
    stream = ((words[..., None] >> (8 * np.arange(6, dtype=np.uint64))) & 0xFF).astype(np.uint8)
    stream = stream.reshape(rb, 16, kb, 4, 24).transpose(2, 0, 3, 1, 4)  # kblk, rblk, q, r, 24
    head = stream[..., :16].reshape(kb, rb, 1024)
    tail = stream[..., 16:].reshape(kb, rb, 512)
    return np.ascontiguousarray(np.concatenate([head, tail], axis=-1))


def fp6_to_codes(blocks: np.ndarray, rows: int, k: int) -> np.ndarray:
    """Exact inverse of codes_to_fp6, dropping the padding (every code must be an integer)."""
    kb, rb, _ = blocks.shape
    head = blocks[..., :1024].reshape(kb, rb, 4, 16, 16)
    tail = blocks[..., 1024:].reshape(kb, rb, 4, 16, 8)
    stream = np.concatenate([head, tail], axis=-1).astype(np.uint64)  # kblk, rblk, q, r, 24
    bits = np.zeros(stream.shape[:-1], dtype=object)
    for j in range(24):
        bits = bits + (stream[..., j].astype(object) << (8 * j))
    fields = np.stack([(bits >> (6 * i)) & 63 for i in range(32)], axis=-1).astype(np.int64)
    vals = fp6_value(fields)
    if not np.array_equal(vals, np.round(vals)):
        raise ValueError("FP6 blocks hold a code that is not an integer")
    full = vals.astype(np.int64).transpose(1, 3, 0, 2, 4).reshape(rb * 16, kb * 128)
    return full[:rows, :k].astype(np.int8)


# Compact FP6 weight layout (no reference counterpart).  A weight whose codes lie in [-7, 7]
# (every weight quantize_convrot_weight produces: core.py:154-158 clips to +-7) has FP6 fields
# whose two exponent bits are zero, so each field carries 4 bits of information.  The compact
# layout keeps the FP6 operand layout's blocks of 16 rows x 128 features and lane order, at
# 1024 bytes a block ([K/128][R_pad/16][1024]): lane L's four dwords I0..I3 at byte 16*L
# hold the FP6 stream dwords D0..D5 of that lane (feature i at stream bits 6i..6i+5) as
#     I0 = (D0 & ~Z0) | (D2 & Z0)    I1 = (D1 & ~Z1) | (D2 & Z1)
#     I2 = (D3 & ~Z0) | (D5 & Z0)    I3 = (D4 & ~Z1) | (D5 & Z1)
# where Z0 / Z1 are the exponent-bit positions of D0 / D1 (D3 / D4): the exponent bits of
# D0 and D1 hold D2's information bits, and D2's own exponent bits are exactly the positions
# in neither mask.  Expansion back to the operand: D0 = I0 & ~Z0, D1 = I1 & ~Z1,
# D2 = (I0 & Z0) | (I1 & Z1), four bit operations per 16 fields.
FP6C_Z0 = 0x18618618
FP6C_Z1 = 0x86186186
FP6C_BLOCK_BYTES = 1024


def _fp6_lane_dwords(blocks: np.ndarray) -> np.ndarray:
    """FP6 blocks [kb, rb, 1536] -> the stream dwords D0..D5 of each lane, [kb, rb, 64, 6] uint32."""
    kb, rb, _ = blocks.shape
    head = np.ascontiguousarray(blocks[..., :1024]).view("<u4").reshape(kb, rb, 64, 4)
    tail = np.ascontiguousarray(blocks[..., 1024:]).view("<u4").reshape(kb, rb, 64, 2)
    return np.concatenate([head, tail], axis=-1)


def codes_to_fp6c(codes: np.ndarray) -> np.ndarray:
    """Row-major int8 codes [R, K] in [-7, 7] (K % 128 == 0) -> compact FP6 blocks
    [K/128, R_pad/16, 1024]."""
    codes = np.asarray(codes)
    if codes.size and (codes.min() < -7 or codes.max() > 7):
        raise ValueError("the compact FP6 layout holds the codes -7 .. 7 only")
    d = _fp6_lane_dwords(codes_to_fp6(codes))
    z0, z1 = np.uint32(FP6C_Z0), np.uint32(FP6C_Z1)
    i0 = (d[..., 0] & ~z0) | (d[..., 2] & z0)
    i1 = (d[..., 1] & ~z1) | (d[..., 2] & z1)
    i2 = (d[..., 3] & ~z0) | (d[..., 5] & z0)
    i3 = (d[..., 4] & ~z1) | (d[..., 5] & z1)
    lanes = np.stack([i0, i1, i2, i3], axis=-1).astype("<u4")
    kb, rb = lanes.shape[:2]
    return np.ascontiguousarray(lanes.view(np.uint8).reshape(kb, rb, 1024))


def fp6c_expand(blocks: np.ndarray) -> np.ndarray:
    """Compact FP6 blocks [kb, rb, 1024] -> the FP6 operand blocks [kb, rb, 1536] the GEMM's
    matrix instruction reads (the kernel's in-register expansion)."""
    kb, rb, _ = blocks.shape
    i = np.ascontiguousarray(blocks).view("<u4").reshape(kb, rb, 64, 4)
    z0, z1 = np.uint32(FP6C_Z0), np.uint32(FP6C_Z1)
    d = np.stack([i[..., 0] & ~z0, i[..., 1] & ~z1, (i[..., 0] & z0) | (i[..., 1] & z1),
                  i[..., 2] & ~z0, i[..., 3] & ~z1, (i[..., 2] & z0) | (i[..., 3] & z1)], axis=-1).astype("<u4")
    head = d[..., :4].view(np.uint8).reshape(kb, rb, 1024)
    tail = np.ascontiguousarray(d[..., 4:]).view(np.uint8).reshape(kb, rb, 512)
    return np.ascontiguousarray(np.concatenate([head, tail], axis=-1))


def fp6c_to_codes(blocks: np.ndarray, rows: int, k: int) -> np.ndarray:
    """Exact inverse of codes_to_fp6c, dropping the padding."""
    return fp6_to_codes(fp6c_expand(blocks), rows, k)


def cpu_threads() -> int:
    return len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
