"""ConvRot W4A4 / W4A16 primitives on MI355X (gfx950), PyTorch-ROCm host side.

Mirrors the public API of the reference package `convrot_mlx`
(/root/reference/src/convrot_mlx/core.py, re-exported by its __init__.py).
Every compute function runs one of the hand-written HIP kernels behind the C
ABI in include/convrot_amd.h; argument validation happens here first, with
the reference's messages, so a bad call raises ValueError before any launch.

Quantization contract (the reference's, core.py:4-21): each group of 64 or
256 features is rotated by a normalized regular Hadamard matrix, each row is
quantized symmetrically as absmax/7 into signed [-7, 7], two's-complement
nibbles are packed low nibble first, the integer GEMM is exact and the
epilogue is ((dot * xscale) * wscale) + bias in float32.

Weight layouts
  NK    uint8 [N, K/2], low nibble = even input feature   (core.py:1252-1253)
  KN    uint8 [K, N/2], low nibble = even output feature  (core.py:1249-1250)
  CDNA4 uint8 [ceil(K/128), ceil(N/16), 1024] tile blocks read directly by
        the gfx950 GEMMs (16 output rows x 128 features per 1 KB block).
"""

from __future__ import annotations

import math
import os

import torch
from torch import nn

from . import _native as nat

CONVROT_GROUP_SIZE = 256  # core.py:32
INT4_MAX = 7  # core.py:34
# The reference fuses groups 64 and 256 (core.py:33); the gfx950 kernel also
# covers the other powers of four its eager path accepts, up to 1024.
SUPPORTED_FUSED_GROUP_SIZES = frozenset({4, 16, 64, 256, 1024})
# "hip-*" store the CDNA4 tile layout; "mpp-*" keep the reference's KN layout
# contract for qweight (core.py:1244-1250) and repack it once on device.
SUPPORTED_BACKENDS = frozenset({"hip-w4a4", "hip-w4a16", "mpp-w4a4", "mpp-w4a16"})
# One fused HIP preprocessor; the reference's names are accepted as aliases.
SUPPORTED_PREPROCESSORS = frozenset({"hip-fused", "metal-fused", "mlx-compiled"})

WEIGHT_LAYOUT_NK = "packed-nk-low-nibble-even-feature"
WEIGHT_LAYOUT_KN = "packed-kn-low-nibble-even-output"
WEIGHT_LAYOUT_CDNA4 = "packed-cdna4-n16-k128-split-nibble"


# ------------------------------------------------------------------ validation


def _validate_group_size(group_size: int) -> None:
    """core.py:50-61."""
    if group_size < 4:
        raise ValueError(f"Regular Hadamard size must be a power of 4, got {group_size}")
    value = group_size
    while value > 1 and value % 4 == 0:
        value //= 4
    if value != 1:
        raise ValueError(f"Regular Hadamard size must be a power of 4, got {group_size}")


def _validate_fused(x: torch.Tensor, group_size: int, what: str) -> None:
    """core.py:431-442 (and :462-473, :493-502)."""
    if x.ndim != 2:
        raise ValueError(f"fused ConvRot {what} expects 2D input, got {tuple(x.shape)}")
    _validate_group_size(group_size)
    if group_size not in SUPPORTED_FUSED_GROUP_SIZES:
        raise ValueError(
            f"fused ConvRot {what} supports groups {sorted(SUPPORTED_FUSED_GROUP_SIZES)}, got {group_size}"
        )
    if x.shape[1] % group_size:
        raise ValueError(f"features {x.shape[1]} not divisible by ConvRot group size {group_size}")


def _log4(group_size: int) -> int:
    s = 0
    while group_size > 1:
        group_size //= 4
        s += 1
    return s


def cdna4_shape(out_features: int, in_features: int) -> tuple[int, int, int]:
    """Shape of a CDNA4-layout weight for an (out_features, in_features) linear."""
    return (-(-in_features // 128), -(-out_features // 16), 1024)


# ------------------------------------------------------------------ preparation


def fp6_shape(rows: int, features: int) -> tuple[int, int, int]:
    """Shape of the FP6 operand blocks of a [rows, features] operand (features % 128 == 0):
    [features/128, ceil(rows/16), 1536] bytes (layout in include/convrot_amd.h)."""
    return (features // 128, -(-rows // 16), 1536)


def _prep_out(kind: int, rows: int, features: int, like: torch.Tensor) -> torch.Tensor:
    """Output buffer of a preparation mode (FP6 blocks of a ragged last row block are
    only partly written; their padding rows only reach GEMM rows that are never stored)."""
    if kind == nat.PREP_PACKED:
        return torch.empty((rows, features // 2), dtype=torch.uint8, device=like.device)
    if kind == nat.PREP_INT8:
        return torch.empty((rows, features), dtype=torch.int8, device=like.device)
    if kind == nat.PREP_FP6:
        return torch.empty(fp6_shape(rows, features), dtype=torch.uint8, device=like.device)
    return torch.empty((rows, features), dtype=like.dtype, device=like.device)


def _prepare(x: torch.Tensor, group_size: int, mode: int) -> tuple[torch.Tensor, torch.Tensor | None]:
    nat.require_device(x)
    x = x.contiguous()
    rows, features = x.shape
    kind = mode & ~nat.PREP_NO_ROTATE
    out = _prep_out(kind, rows, features, x)
    scales = None if kind == nat.PREP_ROTATE else torch.empty((rows,), dtype=torch.float32, device=x.device)
    lib = nat.load()
    nat.check(
        lib.convrot_prepare(
            nat.ptr(x), nat.dtype_code(x.dtype), rows, features, group_size, mode,
            nat.ptr(out), nat.ptr(scales), nat.stream_of(x.device),
        )
    )
    return out, scales


def _modulation_rows(rows: int, features: int, shift: torch.Tensor, scale: torch.Tensor):
    """shift / scale as [V, K] rows of the activation dtype, and the rows of x per vector."""
    if shift.shape[-1] != features or scale.shape[-1] != features:
        raise ValueError(f"shift and scale must end in {features} features, got {tuple(shift.shape)} and "
                         f"{tuple(scale.shape)}")
    sh, sc = shift.reshape(-1, features), scale.reshape(-1, features)
    if sh.shape[0] != sc.shape[0]:
        raise ValueError(f"shift has {sh.shape[0]} rows but scale has {sc.shape[0]}")
    vectors = sh.shape[0]
    if vectors == 0 or rows % vectors:
        raise ValueError(f"{rows} activation rows do not split evenly over {vectors} modulation vectors")
    return sh, sc, rows // vectors


def _prepare_modulated(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, group_size: int, mode: int,
                       eps: float) -> tuple[torch.Tensor, torch.Tensor | None]:
    nat.require_device(x, shift, scale)
    x = x.contiguous()
    rows, features = x.shape
    sh, sc, per_vector = _modulation_rows(rows, features, shift, scale)
    sh = sh.to(x.dtype).contiguous()
    sc = sc.to(x.dtype).contiguous()
    out = _prep_out(mode, rows, features, x)
    scales = None if mode == nat.PREP_ROTATE else torch.empty((rows,), dtype=torch.float32, device=x.device)
    nat.check(
        nat.load().convrot_prepare_modulated(
            nat.ptr(x), nat.dtype_code(x.dtype), rows, features, group_size, mode, nat.ptr(sh), nat.ptr(sc),
            per_vector, float(eps), nat.ptr(out), nat.ptr(scales), nat.stream_of(x.device),
        )
    )
    return out, scales


def hip_fused_modulated_prepare(
    x: torch.Tensor,
    shift: torch.Tensor,
    scale: torch.Tensor,
    group_size: int = CONVROT_GROUP_SIZE,
    *,
    eps: float = 1e-6,
    output: str = "int8",
):
    """Fused producer: ConvRot preparation of `(1 + scale) * layer_norm(x) + shift`.

    One kernel computes a LayerNorm without affine parameters (moments from
    float64 sums), the adaLN modulation with a dtype rounding after every op,
    the regular-Hadamard rotation and the A4 quantization.  No counterpart in
    the reference, which runs the normalization and modulation as separate ops
    before ConvRotLinear (examples/flux1_dev/adapter.py:45-70).

    x: [rows, K] (or [..., K]); shift, scale: [V, K] (or [V, 1, K]) with rows
    divisible by V -- rows r*rows/V .. use vector r, as x [B, L, K] with
    shift [B, 1, K] does.  output: "int8" (int8 codes + f32 scales), "packed"
    (uint8 [rows, K/2] + scales) or "rotate" (rotated activation of x's dtype).
    """
    modes = {"int8": nat.PREP_INT8, "packed": nat.PREP_PACKED, "rotate": nat.PREP_ROTATE}
    if output not in modes:
        raise ValueError(f"output must be one of {sorted(modes)}, got {output!r}")
    _validate_fused(x.reshape(-1, x.shape[-1]), group_size, "modulated activation preparation")
    out, scales = _prepare_modulated(x.reshape(-1, x.shape[-1]), shift, scale, group_size, modes[output], eps)
    return out if output == "rotate" else (out, scales)


def _gelu_operand(t: torch.Tensor) -> torch.Tensor:
    """A producer operand as rows the kernel can read in place: unit feature stride, a row
    stride that covers the row, 16-byte aligned rows (else a contiguous copy on the device)."""
    esize = t.element_size()
    if (t.stride(-1) != 1 or t.stride(0) < t.shape[1] or t.data_ptr() % 16 or (t.stride(0) * esize) % 16):
        t = t.contiguous()
    return t


def _prepare_gelu(x: torch.Tensor, head: torch.Tensor | None, group_size: int,
                  mode: int) -> tuple[torch.Tensor, torch.Tensor | None]:
    if head is not None and head.shape[-1] == 0:
        head = None
    nat.require_device(x, *([head] if head is not None else []))
    x = _gelu_operand(x)
    rows, x_features = x.shape
    head_features = 0
    if head is not None:
        if head.shape[0] != rows:
            raise ValueError(f"GELU producer head has {head.shape[0]} rows, x has {rows}")
        if head.dtype != x.dtype:
            raise ValueError(f"GELU producer head dtype {head.dtype} differs from x dtype {x.dtype}")
        head = _gelu_operand(head)
        head_features = head.shape[1]
    features = head_features + x_features
    out = _prep_out(mode, rows, features, x)
    scales = None if mode == nat.PREP_ROTATE else torch.empty((rows,), dtype=torch.float32, device=x.device)
    nat.check(
        nat.load().convrot_prepare_gelu(
            nat.ptr(head), head_features, head.stride(0) if head is not None else 0, nat.ptr(x), x_features,
            x.stride(0), nat.dtype_code(x.dtype), rows, group_size, mode, nat.ptr(out), nat.ptr(scales),
            nat.stream_of(x.device),
        )
    )
    return out, scales


def hip_fused_gelu_prepare(
    x: torch.Tensor,
    group_size: int = CONVROT_GROUP_SIZE,
    *,
    head: torch.Tensor | None = None,
    output: str = "int8",
):
    """Fused producer: ConvRot preparation of `cat([head, gelu(x)], -1)`.

    gelu is the tanh GELU (nn.GELU(approximate="tanh")) as a fixed float32 sequence,
    rounded once to x's dtype; one kernel applies it, concatenates, rotates and
    quantizes, reading x and head in place (row-strided views such as a slice of a
    fused projection's output need no copy).  No counterpart in the reference, which
    runs the activation and the concatenation as separate ops before ConvRotLinear.

    x: [..., Kx]; head: None or [..., Kh] with the same leading shape and dtype;
    Kx and Kh divisible by 16, Kh + Kx by group_size.  output as in
    hip_fused_modulated_prepare.
    """
    modes = {"int8": nat.PREP_INT8, "packed": nat.PREP_PACKED, "rotate": nat.PREP_ROTATE}
    if output not in modes:
        raise ValueError(f"output must be one of {sorted(modes)}, got {output!r}")
    x2d = x.reshape(-1, x.shape[-1])
    h2d = None if head is None else head.reshape(-1, head.shape[-1])
    features = x2d.shape[1] + (0 if h2d is None else h2d.shape[1])
    _validate_fused(torch.empty((0, features), device="meta"), group_size, "GELU activation preparation")
    out, scales = _prepare_gelu(x2d, h2d, group_size, modes[output])
    return out if output == "rotate" else (out, scales)


def hip_fused_prepare_convrot_activation(x: torch.Tensor, group_size: int = CONVROT_GROUP_SIZE):
    """Rotation + absmax + A4 quantize + pack in one pass.

    Returns (uint8 [M, K/2] packed codes, float32 [M] scales); bit-identical
    to prepare_convrot_activation (core.py:161-167) and to the reference's
    fused kernel metal_fused_prepare_convrot_activation (core.py:425-453).
    """
    _validate_fused(x, group_size, "activation preparation")
    return _prepare(x, group_size, nat.PREP_PACKED)


def hip_fused_prepare_convrot_activation_i8(x: torch.Tensor, group_size: int = CONVROT_GROUP_SIZE):
    """As above, writing each signed A4 code as one int8 (core.py:456-484)."""
    _validate_fused(x, group_size, "activation preparation")
    return _prepare(x, group_size, nat.PREP_INT8)


def hip_fused_rotate_convrot_activation(x: torch.Tensor, group_size: int = CONVROT_GROUP_SIZE) -> torch.Tensor:
    """Rotation only, in the input dtype (core.py:487-511)."""
    _validate_fused(x, group_size, "rotation")
    return _prepare(x, group_size, nat.PREP_ROTATE)[0]


def regular_hadamard(x: torch.Tensor, group_size: int = CONVROT_GROUP_SIZE) -> torch.Tensor:
    """Right-multiply each feature group by the normalized regular Hadamard (core.py:64-94).

    Any leading shape; per-op rounding in the input dtype, exactly as the
    reference's eager radix-4 butterfly.
    """
    _validate_group_size(group_size)
    features = x.shape[-1]
    if features % group_size:
        raise ValueError(f"features {features} not divisible by ConvRot group size {group_size}")
    if group_size not in SUPPORTED_FUSED_GROUP_SIZES:
        raise ValueError(
            f"fused ConvRot rotation supports groups {sorted(SUPPORTED_FUSED_GROUP_SIZES)}, got {group_size}"
        )
    x2d = x.reshape(-1, features)
    return _prepare(x2d, group_size, nat.PREP_ROTATE)[0].reshape(x.shape)


def quantize_signed_int4_rowwise(x: torch.Tensor):
    """Symmetric absmax/7 row quantization without rotation (core.py:149-158), for any even
    number of features like the reference.  The kernel reads rows in 16-feature chunks, so a
    row whose length is not a multiple of 16 is zero-padded on the device first: zeros change
    neither the row absmax nor any code, and the padded codes fall in whole bytes past K/2."""
    if x.ndim != 2:
        raise ValueError(f"rowwise int4 quantization expects 2D input, got {tuple(x.shape)}")
    features = x.shape[-1]
    if features % 2:
        raise ValueError(f"last dimension must be even, got {features}")
    if features % 16 == 0 or x.shape[0] == 0:
        return _prepare(x, 1, nat.PREP_PACKED | nat.PREP_NO_ROTATE)
    nat.require_device(x)
    padded = torch.nn.functional.pad(x, (0, -features % 16))
    q, scales = _prepare(padded, 1, nat.PREP_PACKED | nat.PREP_NO_ROTATE)
    return q[:, : features // 2].contiguous(), scales


def prepare_convrot_activation(x: torch.Tensor, group_size: int = CONVROT_GROUP_SIZE):
    """Rotate and row-quantize an activation (core.py:161-167)."""
    _validate_group_size(group_size)
    if x.ndim != 2:
        raise ValueError(f"rowwise int4 quantization expects 2D input, got {tuple(x.shape)}")
    if x.shape[-1] % group_size:
        raise ValueError(f"features {x.shape[-1]} not divisible by ConvRot group size {group_size}")
    return _prepare(x, group_size, nat.PREP_PACKED)


def quantize_convrot_weight(weight: torch.Tensor, group_size: int = CONVROT_GROUP_SIZE):
    """Rotate a dense (out, in) weight and store it as packed signed W4, NK layout (core.py:514-527)."""
    if weight.ndim != 2:
        raise ValueError(f"ConvRot weight must be 2D, got {tuple(weight.shape)}")
    if weight.shape[-1] % group_size:
        raise ValueError(f"in_features {weight.shape[-1]} not divisible by ConvRot group size {group_size}")
    _validate_group_size(group_size)
    return _prepare(weight, group_size, nat.PREP_PACKED)


# ------------------------------------------------------------------ layouts


def pack_signed_int4(values: torch.Tensor) -> torch.Tensor:
    """Pack signed nibbles low-column first (core.py:97-105)."""
    if values.shape[-1] % 2:
        raise ValueError(f"last dimension must be even, got {values.shape[-1]}")
    nat.require_device(values)
    v = values.to(torch.int8).contiguous()
    cols = v.shape[-1] // 2
    rows = v.numel() // max(v.shape[-1], 1)
    out = torch.empty((*v.shape[:-1], cols), dtype=torch.uint8, device=v.device)
    nat.check(nat.load().convrot_pack_int4(nat.ptr(v), rows, cols, nat.ptr(out), nat.stream_of(v.device)))
    return out


def unpack_signed_int4(packed: torch.Tensor) -> torch.Tensor:
    """Unpack two's-complement nibbles to int8 in [-8, 7] (core.py:108-120, kernel :915-922)."""
    nat.require_device(packed)
    p = packed.contiguous()
    if p.dtype != torch.uint8:
        p = p.to(torch.uint8)
    cols = p.shape[-1]
    rows = p.numel() // max(cols, 1)
    out = torch.empty((*p.shape[:-1], cols * 2), dtype=torch.int8, device=p.device)
    nat.check(nat.load().convrot_unpack_int4(nat.ptr(p), rows, cols, nat.ptr(out), nat.stream_of(p.device)))
    return out


def _repack(q: torch.Tensor, in_layout: int, out_layout: int, n: int, k: int, out_shape) -> torch.Tensor:
    nat.require_device(q)
    q = q.contiguous()
    out = torch.empty(out_shape, dtype=torch.uint8, device=q.device)
    nat.check(
        nat.load().convrot_repack_weight(
            nat.ptr(q), in_layout, nat.ptr(out), out_layout, n, k, nat.stream_of(q.device)
        )
    )
    return out


def repack_nk_weight_for_mpp(qweight: torch.Tensor) -> torch.Tensor:
    """Bit-exact N x packed-K to K x packed-N conversion (core.py:123-133)."""
    if qweight.ndim != 2:
        raise ValueError(f"MPP weight repack expects a 2D tensor, got {tuple(qweight.shape)}")
    n, k = qweight.shape[0], qweight.shape[1] * 2
    if n % 2:
        raise ValueError(f"MPP int4 packing requires even out_features, got {n}")
    return _repack(qweight, nat.LAYOUT_NK, nat.LAYOUT_KN, n, k, (k, n // 2))


def repack_mpp_weight_to_nk(qweight: torch.Tensor) -> torch.Tensor:
    """Reverse the K x packed-N layout back to N x packed-K (core.py:136-146)."""
    if qweight.ndim != 2:
        raise ValueError(f"MPP weight repack expects a 2D tensor, got {tuple(qweight.shape)}")
    k, n = qweight.shape[0], qweight.shape[1] * 2
    if k % 2:
        raise ValueError(f"row-major int4 packing requires even in_features, got {k}")
    return _repack(qweight, nat.LAYOUT_KN, nat.LAYOUT_NK, n, k, (n, k // 2))


def repack_nk_weight_for_cdna4(qweight: torch.Tensor) -> torch.Tensor:
    """N x packed-K -> CDNA4 tile blocks (lossless; zero padding to 16 x 128)."""
    if qweight.ndim != 2:
        raise ValueError(f"CDNA4 weight repack expects a 2D tensor, got {tuple(qweight.shape)}")
    n, k = qweight.shape[0], qweight.shape[1] * 2
    return _repack(qweight, nat.LAYOUT_NK, nat.LAYOUT_CDNA4, n, k, cdna4_shape(n, k))


def repack_cdna4_weight_to_nk(qweight: torch.Tensor, out_features: int, in_features: int) -> torch.Tensor:
    """Exact inverse of repack_nk_weight_for_cdna4 (drops the padding)."""
    _check_cdna4(qweight, out_features, in_features)
    if in_features % 2:
        raise ValueError(f"row-major int4 packing requires even in_features, got {in_features}")
    return _repack(qweight, nat.LAYOUT_CDNA4, nat.LAYOUT_NK, out_features, in_features,
                   (out_features, in_features // 2))


def repack_mpp_weight_for_cdna4(qweight: torch.Tensor) -> torch.Tensor:
    """K x packed-N (the reference's MPP layout) -> CDNA4 tile blocks."""
    if qweight.ndim != 2:
        raise ValueError(f"MPP W4 weight must be 2D, got {tuple(qweight.shape)}")
    k, n = qweight.shape[0], qweight.shape[1] * 2
    return _repack(qweight, nat.LAYOUT_KN, nat.LAYOUT_CDNA4, n, k, cdna4_shape(n, k))


def repack_cdna4_weight_to_mpp(qweight: torch.Tensor, out_features: int, in_features: int) -> torch.Tensor:
    """CDNA4 tile blocks -> K x packed-N."""
    _check_cdna4(qweight, out_features, in_features)
    if out_features % 2:
        raise ValueError(f"MPP int4 packing requires even out_features, got {out_features}")
    return _repack(qweight, nat.LAYOUT_CDNA4, nat.LAYOUT_KN, out_features, in_features,
                   (in_features, out_features // 2))


def _check_cdna4(qweight: torch.Tensor, n: int, k: int) -> None:
    want = cdna4_shape(n, k)
    if tuple(qweight.shape) != want or qweight.dtype != torch.uint8:
        raise ValueError(f"CDNA4 weight for ({n}, {k}) must be uint8 {want}, got {qweight.dtype} {tuple(qweight.shape)}")


# ------------------------------------------------------------------ GEMMs


def _weight_n(qweight: torch.Tensor, k: int) -> int:
    """Output features of a W4 weight given as CDNA4 blocks (3-D) or the reference's
    K x packed-N layout (2-D, validated as in core.py:1030-1039)."""
    if qweight.ndim == 3:
        kb, nb, blk = qweight.shape
        if blk != 1024 or kb != -(-k // 128):
            raise ValueError(f"CDNA4 W4 weight {tuple(qweight.shape)} does not match activation K={k}")
        return nb * 16
    return _validate_mpp_weight_layout(qweight, k)


def _as_cdna4(qweight: torch.Tensor, n: int, k: int) -> torch.Tensor:
    """CDNA4 blocks for the GEMMs; a K x packed-N weight is repacked on device per call
    (ConvRotLinear caches the repacked tensor instead)."""
    if qweight.ndim == 3:
        _check_cdna4(qweight, n, k)
        return qweight.contiguous()
    if qweight.shape[1] * 2 != n:
        raise ValueError(f"MPP W4 weight {tuple(qweight.shape)} does not hold {n} output features")
    return repack_mpp_weight_for_cdna4(qweight)


def _validate_mpp_weight_layout(qweight: torch.Tensor, k: int) -> int:
    """core.py:1030-1039."""
    if qweight.ndim != 2:
        raise ValueError(f"MPP W4 weight must be 2D, got {tuple(qweight.shape)}")
    if qweight.shape[0] != k:
        raise ValueError(
            f"MPP W4 weight must use K x packed-N layout; activation K={k}, weight={tuple(qweight.shape)}"
        )
    if k % 32:
        raise ValueError(f"MPP W4 TensorOp requires K divisible by 32, got {k}")
    return qweight.shape[1] * 2


def _validate_mpp_epilogue(m: int, n: int, xscales, wscales, bias) -> None:
    """core.py:1042-1058."""
    if xscales is not None and tuple(xscales.shape) != (m,):
        raise ValueError(f"MPP activation scales must have shape {(m,)}, got {tuple(xscales.shape)}")
    if tuple(wscales.shape) != (n,):
        raise ValueError(f"MPP weight scales must have shape {(n,)}, got {tuple(wscales.shape)}")
    if bias is not None and tuple(bias.shape) != (n,):
        raise ValueError(f"MPP bias must have shape {(n,)}, got {tuple(bias.shape)}")


def _f32(t: torch.Tensor | None) -> torch.Tensor | None:
    return None if t is None else t.to(torch.float32).contiguous()


class GatedResidual:
    """The gated residual a W4A4 GEMM applies in its epilogue:
    out = residual + gate * linear, each op rounded to the output dtype.

    residual: [M, N] contiguous, the output dtype.  gate: None (plain residual
    add) or a tensor whose row m // rows_per_gate, `stride` elements per row,
    gates output row m.  `inplace` writes the result into `residual`."""

    __slots__ = ("residual", "gate", "stride", "rows_per_gate", "inplace")

    def __init__(self, residual, gate=None, stride=0, rows_per_gate=1, inplace=False):
        self.residual, self.gate, self.stride = residual, gate, stride
        self.rows_per_gate, self.inplace = rows_per_gate, inplace


def _gate_rows(gate: torch.Tensor, out_shape: tuple) -> tuple[torch.Tensor, int, int]:
    """A gate broadcastable to out_shape ([*lead, N]) as (tensor, row stride, rows per gate
    row) over the flattened [M, N] output: trailing lead dims the gate broadcasts over
    (stride 0 once expanded) become rows_per_gate, the others must step through the gate's
    rows at one stride.  Gates of any other form are expanded into a contiguous [M, N] copy."""
    n = out_shape[-1]
    try:
        g = gate.expand(out_shape)
    except RuntimeError as e:
        raise ValueError(f"gate {tuple(gate.shape)} does not broadcast to the output {tuple(out_shape)}") from e
    lead, strides = out_shape[:-1], g.stride()[:-1]
    i = len(lead)
    while i > 0 and (strides[i - 1] == 0 or lead[i - 1] == 1):
        i -= 1
    rows_per_gate = math.prod(lead[i:])
    prefix = [(lead[j], strides[j]) for j in range(i) if lead[j] != 1]
    stride = prefix[-1][1] if prefix else n
    nested = all(prefix[j][1] == prefix[j + 1][1] * prefix[j + 1][0] for j in range(len(prefix) - 1))
    if (n > 1 and g.stride(-1) != 1) or not nested or stride < n or g.data_ptr() % 16:
        return g.reshape(-1, n).contiguous(), n, 1
    return g, stride, max(1, rows_per_gate)


def _gated_residual(residual: torch.Tensor, gate: torch.Tensor | None, out_shape: tuple,
                    dtype: torch.dtype, inplace: bool = False) -> GatedResidual:
    """Validate `residual + gate * linear` operands against the linear's output."""
    if tuple(residual.shape) != tuple(out_shape):
        raise ValueError(f"residual {tuple(residual.shape)} must have the output shape {tuple(out_shape)}")
    if residual.dtype != dtype or (gate is not None and gate.dtype != dtype):
        raise ValueError(f"residual and gate must have the output dtype {dtype}")
    nat.require_device(residual, gate)
    if inplace and not residual.is_contiguous():
        raise ValueError("an in-place gated residual must be contiguous")
    res = residual if residual.is_contiguous() else residual.contiguous()
    if res.data_ptr() % 16:
        if inplace:
            raise ValueError("an in-place gated residual must be 16-byte aligned")
        res = res.clone()
    if gate is None:
        return GatedResidual(res, None, 0, 1, inplace)
    g, stride, rpg = _gate_rows(gate, tuple(out_shape))
    return GatedResidual(res, g, stride, rpg, inplace)


# Stream-K workspaces, one per (device index, stream handle), shared by the
# W4A4 GEMM (stream-K plans) and the W4A16 GEMM (split-K plans): allocated by
# torch (zero-filled, stream-ordered) on the stream's first eager launch and
# kept, so the library itself allocates nothing on these paths.
_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


def _workspace(device: torch.device) -> torch.Tensor | None:
    """The stream-K workspace of `device`'s current stream, or None under graph capture
    before one exists (the W4A4 GEMM then runs a data-parallel plan, same results bit for
    bit; the W4A16 GEMM its unsplit plan)."""
    stream = torch.cuda.current_stream(device)
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream.cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is None:
        if torch.cuda.is_current_stream_capturing():
            return None
        ws = torch.zeros(int(nat.load().convrot_w4a4_workspace_bytes()), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def w4a4_status(device=None) -> None:
    """Raise ConvRotNativeError if a stream-K W4A4 GEMM on the current stream of `device`
    gave up waiting for a partial tile since the last check (its output tile holds NaN).
    Synchronizes the stream; not for use under graph capture."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    stream = torch.cuda.current_stream(device)
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream.cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is not None:
        nat.check(nat.load().convrot_w4a4_status(nat.ptr(ws), nat.stream_of(device)))


def _w4a4(act: torch.Tensor, act_format: int, k: int, qweight, xscales, wscales, bias, output_dtype, n=None,
          gr: GatedResidual | None = None):
    m = act.shape[0]
    n_layout = _weight_n(qweight, k)
    n = n if n is not None else n_layout
    if k % 32:
        raise ValueError(f"MPP W4 TensorOp requires K divisible by 32, got {k}")
    _validate_mpp_epilogue(m, n, xscales, wscales, bias)
    nat.require_device(act, qweight, xscales, wscales, bias)
    w = _as_cdna4(qweight, n, k)
    xs, ws, b = _f32(xscales), _f32(wscales), _f32(bias)
    if gr is not None and gr.residual.numel() != m * n:
        raise ValueError(f"residual has {gr.residual.numel()} elements, the output {m * n}")
    if gr is not None and gr.inplace:
        out = gr.residual.view(m, n)
    else:
        out = torch.empty((m, n), dtype=output_dtype, device=act.device)
    work = _workspace(act.device)
    nat.check(
        nat.load().convrot_w4a4_gemm_ws(
            nat.ptr(act), act_format, nat.ptr(xs), nat.ptr(w), nat.ptr(ws), nat.ptr(b), m, n, k,
            nat.ptr(gr.residual if gr is not None else None), nat.ptr(gr.gate if gr is not None else None),
            gr.stride if gr is not None else 0, gr.rows_per_gate if gr is not None else 1,
            nat.ptr(work), work.numel() if work is not None else 0,
            nat.ptr(out), nat.dtype_code(output_dtype), nat.stream_of(act.device),
        )
    )
    return out


def _residual_arg(m: int, qweight, k: int, out_features, output_dtype, residual, gate, inplace):
    if residual is None:
        if gate is not None or inplace:
            raise ValueError("gate and inplace need a residual")
        return None
    n = out_features if out_features is not None else _weight_n(qweight, k)
    if residual.ndim < 1 or residual.shape[-1] != n or residual.numel() != m * n:
        raise ValueError(f"residual {tuple(residual.shape)} must hold the [{m}, {n}] output as [..., {n}]")
    # [*lead, N] residuals (e.g. [B, L, N]) let the gate broadcast over their leading dims
    return _gated_residual(residual, gate, tuple(residual.shape), output_dtype, inplace)


def hip_w4a4_matmul(qact, qweight, xscales, wscales, bias, *, output_dtype, out_features=None, residual=None,
                    gate=None, inplace=False):
    """Packed-A4 activations [M, K/2] x W4 weight -> output_dtype [M, N] (core.py:1061-1085).

    qweight: CDNA4 blocks (3-D; pass out_features when N is not a multiple of
    16) or the reference's K x packed-N layout (2-D).  With `residual` ([M, N],
    output_dtype) the kernel returns residual + gate * product (see
    ConvRotLinear.forward), in place into `residual` when `inplace`; the residual
    may be shaped [..., N] (M rows in all) for the gate to broadcast against.

    The packed codes are first unpacked to int8 (one HBM pass over M*K/2 + M*K
    bytes) so that the product runs in the int8 kernels: direct-to-LDS tiles
    and the few-row kernel.  The integer dots are exact either way, so the
    output is the same bits as convrot_w4a4_gemm(ACT_PACKED), whose
    register-staged kernel reads the packed codes itself without a buffer.
    """
    if qact.ndim != 2:
        raise ValueError(f"MPP W4A4 activation must be 2D, got {tuple(qact.shape)}")
    k = qact.shape[1] * 2
    gr = _residual_arg(qact.shape[0], qweight, k, out_features, output_dtype, residual, gate, inplace)
    if k % 32:
        raise ValueError(f"MPP W4 TensorOp requires K divisible by 32, got {k}")
    return _w4a4(unpack_signed_int4(qact), nat.ACT_INT8, k, qweight, xscales, wscales, bias, output_dtype,
                 out_features, gr)


def hip_w4a4_int8_matmul(activations, qweight, xscales, wscales, bias, *, output_dtype, out_features=None,
                         residual=None, gate=None, inplace=False):
    """int8 A4 activations [M, K] x W4 weight -> output_dtype [M, N] (core.py:1088-1120);
    residual, gate and inplace as in hip_w4a4_matmul."""
    if activations.ndim != 2 or activations.dtype != torch.int8:
        raise ValueError(
            f"MPP W4A4 requires a 2D int8 activation, got {tuple(activations.shape)} {activations.dtype}"
        )
    k = activations.shape[1]
    gr = _residual_arg(activations.shape[0], qweight, k, out_features, output_dtype, residual, gate, inplace)
    return _w4a4(activations.contiguous(), nat.ACT_INT8, k, qweight, xscales, wscales, bias, output_dtype,
                 out_features, gr)


# ------------------------------------------------------------------ FP6 operands
#
# A code v is stored as the FP6 (e2m3) encoding of v/8, and gfx950's FP6 matrix
# instruction, with both operand scales 2^3, sums the exact products v*w at
# twice the INT8 instruction's rate: the same GEMM with the same outputs bit
# for bit (layout and encoding in include/convrot_amd.h).  ConvRotLinear
# takes this path at FP6_MIN_ROWS rows and above when in_features % 128 == 0;
# below that the few-row INT8 kernels, which stream half a byte of weight per
# code instead of three quarters, are as fast or faster.
FP6_MIN_ROWS = 256
FP6_MAX_FEATURES = 262144  # exclusive: sums of K products of |v*w| <= 64 stay below 2^24
# The FP6 GEMM addresses each operand with 32-bit buffer offsets (include/convrot_amd.h):
# larger products run on INT8 operands instead.
FP6_MAX_OPERAND_BYTES = (1 << 32) - (1 << 20)
_fp6_operands = os.getenv("CONVROT_FP6_OPERANDS", "1") != "0"
# Which FP6 weight form ConvRotLinear caches: "compact" (0.5 byte per weight, each
# fragment expanded in registers inside the GEMM), "full" (the 0.75-byte operand
# blocks), or "auto" (the library's choice: compact, see fp6_weight_form).
FP6_WEIGHT_FORMS = ("auto", "compact", "full")
_fp6_weight_form = os.getenv("CONVROT_FP6_WEIGHTS", "auto")


def set_fp6_operands(enabled: bool) -> None:
    """Turn the FP6 operand path of ConvRotLinear on or off (default on; the environment
    variable CONVROT_FP6_OPERANDS=0 turns it off at import).  Outputs are the same bits
    either way."""
    global _fp6_operands
    _fp6_operands = bool(enabled)


def fp6_operands_enabled() -> bool:
    return _fp6_operands


def set_fp6_weight_form(form: str) -> None:
    """Choose the FP6 weight form ConvRotLinear caches ("auto", "compact" or "full"; the
    environment variable CONVROT_FP6_WEIGHTS sets it at import).  Outputs are the same bits
    with every form; caches built under another form are rebuilt on the next product."""
    global _fp6_weight_form
    if form not in FP6_WEIGHT_FORMS:
        raise ValueError(f"FP6 weight form must be one of {FP6_WEIGHT_FORMS}, got {form!r}")
    _fp6_weight_form = form


def fp6_weight_form(rows: int, out_features: int) -> str:
    """The FP6 weight form ("compact" or "full") ConvRotLinear caches for a layer whose first
    FP6 product has `rows` rows and `out_features` output features, under the current setting.

    "auto" is the compact form on every tile.  Timed with the weights streamed from HBM, as a
    model's step reads them, it wins on the 128-row tiles too (config 2: 1818 -> 1927 TOPS;
    the FLUX.1-dev DiT step: 32.25 -> 31.64 ms, bit-identical), although an isolated GEMM
    with its weights warm in the Infinity Cache runs the 128-row compact tiles ~10 % slower."""
    del rows, out_features  # one form for every shape (the arguments keep the per-layer query)
    return "compact" if _fp6_weight_form == "auto" else _fp6_weight_form


def fp6_bytes(rows: int, features: int) -> int:
    """Bytes of the FP6 operand blocks of a [rows, features] operand (features % 128 == 0)."""
    return math.prod(fp6_shape(rows, features))


def fp6_eligible(m: int, n: int, k: int, output_dtype: torch.dtype) -> bool:
    """Whether a W4A4 product of this shape runs on FP6 operands in ConvRotLinear."""
    return (_fp6_operands and m >= FP6_MIN_ROWS and k % 128 == 0 and 0 < k < FP6_MAX_FEATURES
            and output_dtype in (torch.bfloat16, torch.float16, torch.float32)
            and max(fp6_bytes(m, k), fp6_bytes(n, k)) <= FP6_MAX_OPERAND_BYTES)


def fp6_weight(qweight: torch.Tensor, out_features: int, in_features: int) -> torch.Tensor:
    """CDNA4 W4 weight -> FP6 operand blocks [K/128, ceil(N/16), 1536] (an offline
    conversion; every int4 code, -8 included, has an FP6 field)."""
    if in_features % 128:
        raise ValueError(f"FP6 operands require in_features divisible by 128, got {in_features}")
    nat.require_device(qweight)
    _check_cdna4(qweight, out_features, in_features)
    out = torch.empty(fp6_shape(out_features, in_features), dtype=torch.uint8, device=qweight.device)
    nat.check(nat.load().convrot_weight_fp6(nat.ptr(qweight.contiguous()), nat.ptr(out), out_features, in_features,
                                            nat.stream_of(qweight.device)))
    return out


def fp6_weight_compact(qweight: torch.Tensor, out_features: int, in_features: int) -> torch.Tensor | None:
    """CDNA4 W4 weight -> compact FP6 blocks [K/128, ceil(N/16), 1024] (the FP6 fields
    without their exponent bits, 0.5 byte per weight; include/convrot_amd.h), or None when
    a code is -8, which has no compact field (fp6_weight holds it).  Reads a flag back from
    the device, so it synchronizes the stream (an offline conversion)."""
    if in_features % 128:
        raise ValueError(f"FP6 operands require in_features divisible by 128, got {in_features}")
    nat.require_device(qweight)
    _check_cdna4(qweight, out_features, in_features)
    out = torch.empty(cdna4_shape(out_features, in_features), dtype=torch.uint8, device=qweight.device)
    flag = torch.empty((1,), dtype=torch.int32, device=qweight.device)
    nat.check(nat.load().convrot_weight_fp6_compact(nat.ptr(qweight.contiguous()), nat.ptr(out), nat.ptr(flag),
                                                    out_features, in_features, nat.stream_of(qweight.device)))
    return None if int(flag.item()) else out


def hip_fused_prepare_convrot_activation_fp6(x: torch.Tensor, group_size: int = CONVROT_GROUP_SIZE):
    """The fused preparation with FP6 output: (FP6 blocks [K/128, ceil(M/16), 1536] of the
    A4 codes, float32 row scales).  Rows of a ragged last 16-row block are left unwritten
    (they only reach product rows that are never stored)."""
    _validate_fused(x, group_size, "FP6")
    if x.shape[-1] % 128:
        raise ValueError(f"FP6 operands require features divisible by 128, got {x.shape[-1]}")
    return _prepare(x, group_size, nat.PREP_FP6)


def _w4a4_fp6(act6, w6, xscales, wscales, bias, output_dtype, m: int, n: int, k: int,
              gr: GatedResidual | None = None):
    if k % 128 or not 0 < k < FP6_MAX_FEATURES or output_dtype not in (torch.bfloat16, torch.float16,
                                                                         torch.float32):
        raise ValueError(f"FP6 W4A4 product needs K % 128 == 0 with K < {FP6_MAX_FEATURES} and a float32, "
                         f"float16 or bfloat16 output; got M={m} N={n} K={k} {output_dtype}")
    compact = tuple(w6.shape) == cdna4_shape(n, k)  # 1024-byte blocks: the compact weight layout
    if tuple(act6.shape) != fp6_shape(m, k) or (tuple(w6.shape) != fp6_shape(n, k) and not compact):
        raise ValueError(f"FP6 operands must be {fp6_shape(m, k)} and {fp6_shape(n, k)} (or compact "
                         f"{cdna4_shape(n, k)}), got {tuple(act6.shape)} and {tuple(w6.shape)}")
    _validate_mpp_epilogue(m, n, xscales, wscales, bias)
    nat.require_device(act6, w6, xscales, wscales, bias)
    xs, ws, b = _f32(xscales), _f32(wscales), _f32(bias)
    if gr is not None and gr.residual.numel() != m * n:
        raise ValueError(f"residual has {gr.residual.numel()} elements, the output {m * n}")
    if gr is not None and gr.inplace:
        out = gr.residual.view(m, n)
    else:
        out = torch.empty((m, n), dtype=output_dtype, device=act6.device)
    lib, stream = nat.load(), nat.stream_of(act6.device)
    if compact:
        nat.check(lib.convrot_w4a4_gemm_fp6_compact(
            nat.ptr(act6), nat.ptr(xs), nat.ptr(w6), nat.ptr(ws), nat.ptr(b), m, n, k,
            nat.ptr(gr.residual if gr is not None else None), nat.ptr(gr.gate if gr is not None else None),
            gr.stride if gr is not None else 0, gr.rows_per_gate if gr is not None else 1, nat.ptr(out),
            nat.dtype_code(output_dtype), stream))
    elif gr is None:
        nat.check(lib.convrot_w4a4_gemm_fp6(nat.ptr(act6), nat.ptr(xs), nat.ptr(w6), nat.ptr(ws), nat.ptr(b), m, n, k,
                                            nat.ptr(out), nat.dtype_code(output_dtype), stream))
    else:
        nat.check(lib.convrot_w4a4_gemm_fp6_residual(
            nat.ptr(act6), nat.ptr(xs), nat.ptr(w6), nat.ptr(ws), nat.ptr(b), m, n, k, nat.ptr(gr.residual),
            nat.ptr(gr.gate), gr.stride, gr.rows_per_gate, nat.ptr(out), nat.dtype_code(output_dtype), stream))
    return out


def hip_w4a4_fp6_matmul(act6, w6, xscales, wscales, bias, *, output_dtype, rows: int, out_features: int,
                        in_features: int, residual=None, gate=None, inplace=False):
    """FP6 A4 activations x FP6 W4 weight -> output_dtype [rows, out_features]: the product
    and epilogue of hip_w4a4_int8_matmul (core.py:1088-1120), same bits; residual, gate and
    inplace as in hip_w4a4_matmul.  w6 is fp6_weight's [K/128, ceil(N/16), 1536] blocks or
    fp6_weight_compact's [K/128, ceil(N/16), 1024]."""
    m, n = rows, out_features
    gr = None
    if residual is not None:
        if residual.ndim < 1 or residual.shape[-1] != n or residual.numel() != m * n:
            raise ValueError(f"residual {tuple(residual.shape)} must hold the [{m}, {n}] output as [..., {n}]")
        gr = _gated_residual(residual, gate, tuple(residual.shape), output_dtype, inplace)
    elif gate is not None or inplace:
        raise ValueError("gate and inplace need a residual")
    return _w4a4_fp6(act6, w6, xscales, wscales, bias, output_dtype, m, n, in_features, gr)


def hip_w4a16_matmul(activations, qweight, wscales, bias, *, output_dtype, out_features=None, residual=None,
                     gate=None, inplace=False):
    """Rotated bf16/f16 activations x W4 weight -> output_dtype (core.py:1123-1152);
    residual, gate and inplace as in hip_w4a4_matmul (applied in the GEMM's epilogue)."""
    if activations.ndim != 2:
        raise ValueError(f"MPP W4A16 activation must be 2D, got {tuple(activations.shape)}")
    if activations.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"MPP W4A16 requires float16 or bfloat16 activation, got {activations.dtype}")
    m, k = activations.shape
    n_layout = _weight_n(qweight, k)
    n = out_features if out_features is not None else n_layout
    if k % 32:
        raise ValueError(f"MPP W4 TensorOp requires K divisible by 32, got {k}")
    _validate_mpp_epilogue(m, n, None, wscales, bias)
    gr = _residual_arg(m, qweight, k, n, output_dtype, residual, gate, inplace)
    nat.require_device(activations, qweight, wscales, bias)
    act = activations.contiguous()
    w = _as_cdna4(qweight, n, k)
    ws, b = _f32(wscales), _f32(bias)
    if gr is not None and gr.inplace:
        out = gr.residual.view(m, n)
    else:
        out = torch.empty((m, n), dtype=output_dtype, device=act.device)
    # the stream's W4A4 workspace lets the weight-streaming kernel split K over
    # workgroups (few output tiles, long K, M <= 32); none under graph capture
    # before it exists (the unsplit plan)
    work = _workspace(act.device)
    nat.check(
        nat.load().convrot_w4a16_gemm_ws(
            nat.ptr(act), nat.dtype_code(act.dtype), nat.ptr(w), nat.ptr(ws), nat.ptr(b), m, n, k,
            nat.ptr(gr.residual if gr is not None else None), nat.ptr(gr.gate if gr is not None else None),
            gr.stride if gr is not None else 0, gr.rows_per_gate if gr is not None else 1,
            nat.ptr(work), work.numel() if work is not None else 0,
            nat.ptr(out), nat.dtype_code(output_dtype), nat.stream_of(act.device),
        )
    )
    return out


# Reference names (the reference's Metal/MPP entry points) -> the gfx950 kernels.
metal_fused_prepare_convrot_activation = hip_fused_prepare_convrot_activation
metal_fused_prepare_convrot_activation_i8 = hip_fused_prepare_convrot_activation_i8
metal_fused_rotate_convrot_activation = hip_fused_rotate_convrot_activation
metal_unpack_signed_int4 = unpack_signed_int4
mpp_w4a4_matmul = hip_w4a4_matmul
mpp_w4a4_int8_matmul = hip_w4a4_int8_matmul
mpp_w4a16_matmul = hip_w4a16_matmul
# core.py:174-175 are MLX-compiled graphs of the same contract; the fused
# kernel is this build's compiled form.
compiled_prepare_convrot_activation = prepare_convrot_activation
compiled_regular_hadamard = regular_hadamard


# ------------------------------------------------------------------ module


class ConvRotLinear(nn.Module):
    """A linear layer stored and executed under the ConvRot W4A4 contract (core.py:1210-1313).

    Same constructor, attributes and defaults as the reference: `qweight`
    (uint8), `scales` (float32 [N], ones), `bias` (float32 [N], zeros -- one
    fixed signature for biased and biasless layers, core.py:1255-1258),
    `group_size`, `backend`, `preprocessor`, `weight_layout`,
    `source_has_bias`; the output dtype is the input dtype.

    Backends: "hip-w4a4" (default) / "hip-w4a16" hold qweight in the CDNA4
    tile layout; "mpp-w4a4" / "mpp-w4a16" keep the reference's K x packed-N
    contract for qweight (so reference checkpoints and repacks load
    unchanged) and run the same kernels on a cached CDNA4 repack.  A hip-*
    layer given a K x packed-N qweight by assignment, as reference code does,
    runs it the same way (a CDNA4 repack cached per tensor version).
    The default comes from $CONVROT_BACKEND, then $CONVROT_MLX_BACKEND.
    """

    def __init__(
        self,
        in_features: int,
        out_features: int,
        *,
        bias: bool = True,
        group_size: int = CONVROT_GROUP_SIZE,
        backend: str | None = None,
        preprocessor: str | None = None,
        device=None,
    ):
        super().__init__()
        if in_features % group_size:
            raise ValueError(f"in_features {in_features} not divisible by ConvRot group size {group_size}")
        _validate_group_size(group_size)
        if group_size not in SUPPORTED_FUSED_GROUP_SIZES:
            raise ValueError(
                f"fused ConvRot activation preparation supports groups {sorted(SUPPORTED_FUSED_GROUP_SIZES)}, "
                f"got {group_size}"
            )
        self.in_features = in_features
        self.out_features = out_features
        self.group_size = group_size
        self.backend = backend or os.getenv("CONVROT_BACKEND") or os.getenv("CONVROT_MLX_BACKEND") or "hip-w4a4"
        if self.backend not in SUPPORTED_BACKENDS:
            raise ValueError(
                f"Unknown ConvRot backend {self.backend!r}; expected one of {sorted(SUPPORTED_BACKENDS)}"
            )
        self.preprocessor = preprocessor or os.getenv("CONVROT_PREPROCESSOR") or os.getenv(
            "CONVROT_MLX_PREPROCESSOR", "hip-fused"
        )
        if self.preprocessor not in SUPPORTED_PREPROCESSORS:
            raise ValueError(
                f"Unknown ConvRot preprocessor {self.preprocessor!r}; "
                f"expected one of {sorted(SUPPORTED_PREPROCESSORS)}"
            )
        if self.backend.startswith("mpp-"):
            if out_features % 2:
                raise ValueError(f"MPP packed weights require even out_features, got {out_features}")
            qweight = torch.zeros((in_features, out_features // 2), dtype=torch.uint8, device=device)
            self.weight_layout = WEIGHT_LAYOUT_KN
        else:
            qweight = torch.zeros(cdna4_shape(out_features, in_features), dtype=torch.uint8, device=device)
            self.weight_layout = WEIGHT_LAYOUT_CDNA4
        self.register_buffer("qweight", qweight)
        self.register_buffer("scales", torch.ones((out_features,), dtype=torch.float32, device=device))
        self.register_buffer("bias", torch.zeros((out_features,), dtype=torch.float32, device=device))
        self.source_has_bias = bias
        self._cdna4_cache: tuple | None = None
        self._fp6_cache: tuple | None = None

    @property
    def a4(self) -> bool:
        return self.backend.endswith("w4a4")

    def load_nk_weight(self, qweight_nk: torch.Tensor, scales: torch.Tensor, bias: torch.Tensor | None = None):
        """Install an NK-packed weight (as quantize_convrot_weight returns) in this layer's layout."""
        if tuple(qweight_nk.shape) != (self.out_features, self.in_features // 2):
            raise ValueError(
                f"NK weight must have shape {(self.out_features, self.in_features // 2)}, got {tuple(qweight_nk.shape)}"
            )
        if self.weight_layout == WEIGHT_LAYOUT_KN:
            self.qweight = repack_nk_weight_for_mpp(qweight_nk)
        else:
            self.qweight = repack_nk_weight_for_cdna4(qweight_nk)
        self.scales = scales.to(torch.float32)
        if bias is not None:
            self.bias = bias.to(torch.float32)
        return self

    def _device_weight(self) -> torch.Tensor:
        """The CDNA4 weight the kernels read.  A hip-* layer holds it as `qweight`; an mpp-*
        layer, and a hip-* layer given a reference-style K x packed-N `qweight` (the
        reference's assignment, core.py:1244-1250), repack theirs once per tensor version."""
        q = self.qweight
        if self.weight_layout == WEIGHT_LAYOUT_CDNA4 and q.ndim != 2:
            _check_cdna4(q, self.out_features, self.in_features)
            return q
        key = (q.data_ptr(), q._version, tuple(q.shape), q.device)
        if self._cdna4_cache is None or self._cdna4_cache[0] != key:
            _validate_mpp_weight_layout(q, self.in_features)
            if q.shape[1] * 2 != self.out_features:
                raise ValueError(
                    f"MPP W4 weight must use K x packed-N layout; activation K={self.in_features}, "
                    f"weight={tuple(q.shape)}"
                )
            self._cdna4_cache = (key, repack_mpp_weight_for_cdna4(q))
        return self._cdna4_cache[1]

    def _fp6_weight(self, w: torch.Tensor, rows: int) -> torch.Tensor | None:
        """The FP6 form of the CDNA4 weight `w`, converted once and cached per tensor version
        (and weight-form setting, see set_fp6_weight_form): the compact layout (0.5 byte per
        weight) or the FP6 operand blocks (0.75 byte), which also hold a weight with a -8 code
        (no compact field).  The compact conversion reads a flag back from the device; under
        graph capture, where it cannot, a layer without a cached form returns None and the
        product runs on INT8 operands (the same bits)."""
        key = (w.data_ptr(), w._version, tuple(w.shape), w.device, _fp6_weight_form)
        if self._fp6_cache is None or self._fp6_cache[0] != key:
            form = fp6_weight_form(rows, self.out_features)
            if form == "compact" and torch.cuda.is_current_stream_capturing():
                return None
            w6 = fp6_weight_compact(w, self.out_features, self.in_features) if form == "compact" else None
            if w6 is None:
                w6 = fp6_weight(w, self.out_features, self.in_features)
            self._fp6_cache = (key, w6)
        return self._fp6_cache[1]

    def _project(self, prep, lead: tuple, dtype: torch.dtype, residual, gate, inplace: bool) -> torch.Tensor:
        """Run the prepared activation `prep(mode)` through this layer's GEMM, then the
        optional gated residual (residual + gate * linear) in the GEMM's epilogue."""
        if residual is None and (gate is not None or inplace):
            raise ValueError("gate and inplace need a residual")
        out_shape = (*lead, self.out_features)
        w = self._device_weight()
        rows = math.prod(lead)
        if self.a4:
            gr = None if residual is None else _gated_residual(residual, gate, out_shape, dtype, inplace)
        w6 = (self._fp6_weight(w, rows) if self.a4 and fp6_eligible(rows, self.out_features, self.in_features, dtype)
              else None)
        if w6 is not None:
            act6, xscales = prep(nat.PREP_FP6)
            out = _w4a4_fp6(act6, w6, xscales, self.scales, self.bias, dtype, rows, self.out_features,
                            self.in_features, gr)
        elif self.a4:
            qact, xscales = prep(nat.PREP_INT8)
            out = _w4a4(qact, nat.ACT_INT8, self.in_features, w, xscales, self.scales, self.bias, dtype,
                        self.out_features, gr)
        else:
            if residual is not None:
                _gated_residual(residual, gate, out_shape, dtype, inplace)  # checks before any launch
            rotated = prep(nat.PREP_ROTATE)[0]
            out = hip_w4a16_matmul(rotated, w, self.scales, self.bias, output_dtype=dtype,
                                   out_features=self.out_features, residual=residual, gate=gate, inplace=inplace)
        return residual if inplace else out.reshape(out_shape)

    def forward(self, x: torch.Tensor, *, residual: torch.Tensor | None = None, gate: torch.Tensor | None = None,
                inplace: bool = False) -> torch.Tensor:
        """linear(x); with `residual`, residual + gate * linear(x) (gate None: residual +
        linear(x)), each op rounded to x.dtype as torch evaluates it eagerly.  The gate
        broadcasts to the output ([B, 1, N] per image, [N], or full); `inplace` writes the
        result into `residual` and returns it."""
        if x.shape[-1] != self.in_features:
            raise ValueError(f"ConvRotLinear expected K={self.in_features}, got {x.shape[-1]}")
        x2d = x.reshape(-1, self.in_features)
        return self._project(lambda mode: _prepare(x2d, self.group_size, mode), x.shape[:-1], x.dtype,
                             residual, gate, inplace)

    def forward_modulated(self, x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor,
                          eps: float = 1e-6, *, residual: torch.Tensor | None = None,
                          gate: torch.Tensor | None = None, inplace: bool = False) -> torch.Tensor:
        """self((1 + scale) * layer_norm(x) + shift) with the normalization and modulation
        fused into the activation preparation (see hip_fused_modulated_prepare); residual,
        gate and inplace as in forward."""
        if x.shape[-1] != self.in_features:
            raise ValueError(f"ConvRotLinear expected K={self.in_features}, got {x.shape[-1]}")
        x2d = x.reshape(-1, self.in_features)
        return self._project(lambda mode: _prepare_modulated(x2d, shift, scale, self.group_size, mode, eps),
                             x.shape[:-1], x.dtype, residual, gate, inplace)

    def forward_gelu(self, x: torch.Tensor, head: torch.Tensor | None = None, *,
                     residual: torch.Tensor | None = None, gate: torch.Tensor | None = None,
                     inplace: bool = False) -> torch.Tensor:
        """self(cat([head, gelu(x)], -1)) (or self(gelu(x))) with the tanh GELU and the
        concatenation fused into the activation preparation (see hip_fused_gelu_prepare);
        residual, gate and inplace as in forward."""
        head_features = 0 if head is None else head.shape[-1]
        if head_features + x.shape[-1] != self.in_features:
            raise ValueError(f"ConvRotLinear expected K={self.in_features}, got {head_features} + {x.shape[-1]}")
        if head is not None and head.shape[:-1] != x.shape[:-1]:
            raise ValueError(f"GELU producer head {tuple(head.shape)} and x {tuple(x.shape)} differ in leading shape")
        x2d = x.reshape(-1, x.shape[-1])
        h2d = None if head is None else head.reshape(-1, head_features)
        return self._project(lambda mode: _prepare_gelu(x2d, h2d, self.group_size, mode), x.shape[:-1], x.dtype,
                             residual, gate, inplace)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, group_size={self.group_size}, "
                f"backend={self.backend!r}, weight_layout={self.weight_layout!r}")


def eligible_linear(module: object, group_size: int = CONVROT_GROUP_SIZE) -> bool:
    """core.py:1316-1321: a Linear with a 2-D weight whose in_features divide into groups."""
    return (
        isinstance(module, nn.Linear)
        and module.weight.ndim == 2
        and module.weight.shape[1] % group_size == 0
    )
