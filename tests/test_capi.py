"""CPU: the C-ABI library loads, exports every symbol include/convrot_amd.h declares,
and rejects invalid arguments with the documented status codes and messages before any
launch (no GPU is touched by these calls)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "convrot_amd.h"


def header_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(convrot_[a-z0-9_]+)\s*\(", text)))


def header_constants() -> dict[str, int]:
    return {k: int(v, 0) for k, v in re.findall(r"#define\s+(CONVROT_[A-Z0-9_]+)\s+(0x[0-9a-fA-F]+|\d+)", HEADER.read_text())}


@pytest.fixture(scope="module")
def lib():
    from convrot_mlx_amd import _native

    return _native.load()


def test_every_declared_symbol_is_exported(lib):
    from convrot_mlx_amd import _native

    names = header_functions()
    assert len(names) >= 9
    for name in names:
        assert hasattr(lib, name), f"{name} missing from {_native.LIB_PATH.name}"
    assert set(names) == set(_native.SIGNATURES), "ctypes binding and header disagree"


def test_integration_stub_binds_every_entry_point():
    """The reference-side ctypes stub in INTEGRATION.md sets argtypes for every function the
    header declares, with as many arguments as the package's own binding."""
    from convrot_mlx_amd import _native

    doc = (ROOT / "INTEGRATION.md").read_text()
    stub = doc[doc.index("# convrot_mlx/_amd.py"):]
    stub = stub[: stub.index("```")]
    for name in header_functions():
        if name in ("convrot_last_error", "convrot_version"):
            assert name in stub
            continue
        m = re.search(rf"_lib\.{name}\.argtypes = \[([^\]]*)\]", stub)
        assert m, f"{name} has no argtypes in the INTEGRATION.md stub"
        n_args = len([a for a in m.group(1).replace("\n", " ").split(",") if a.strip()])
        assert n_args == len(_native.SIGNATURES[name][1]), f"{name}: stub binds {n_args} arguments"


def test_constants_match_binding():
    from convrot_mlx_amd import _native as n

    c = header_constants()
    assert (c["CONVROT_DTYPE_F32"], c["CONVROT_DTYPE_F16"], c["CONVROT_DTYPE_BF16"]) == (n.DTYPE_F32, n.DTYPE_F16, n.DTYPE_BF16)
    assert (c["CONVROT_PREP_PACKED"], c["CONVROT_PREP_INT8"], c["CONVROT_PREP_ROTATE"], c["CONVROT_PREP_FP6"],
            c["CONVROT_PREP_NO_ROTATE"]) == (n.PREP_PACKED, n.PREP_INT8, n.PREP_ROTATE, n.PREP_FP6, n.PREP_NO_ROTATE)
    assert (c["CONVROT_LAYOUT_NK"], c["CONVROT_LAYOUT_KN"], c["CONVROT_LAYOUT_CDNA4"]) == (n.LAYOUT_NK, n.LAYOUT_KN, n.LAYOUT_CDNA4)
    assert (c["CONVROT_ACT_PACKED"], c["CONVROT_ACT_INT8"]) == (n.ACT_PACKED, n.ACT_INT8)
    assert (c["CONVROT_OK"], c["CONVROT_ERR_INVALID"], c["CONVROT_ERR_UNSUPPORTED"], c["CONVROT_ERR_LAUNCH"]) == (
        n.OK, n.ERR_INVALID, n.ERR_UNSUPPORTED, n.ERR_LAUNCH)


def test_version_and_sizes(lib):
    assert b"gfx950" in lib.convrot_version()
    assert lib.convrot_cdna4_bytes(3072, 12288) == 12288 * 3072 // 2
    assert lib.convrot_cdna4_bytes(46, 64) == 3 * 1 * 1024  # N padded to 48, K to 128
    assert lib.convrot_cdna4_bytes(-1, 5) == -1


def _err(lib):
    return lib.convrot_last_error().decode()


BF16 = 2


@pytest.mark.parametrize("G,msg", [(128, "Regular Hadamard size must be a power of 4, got 128"),
                                    (2, "Regular Hadamard size must be a power of 4, got 2"),
                                    (4096, "fused ConvRot supports groups [4, 16, 64, 256, 1024], got 4096")])
def test_prepare_rejects_group_sizes(lib, G, msg):
    rc = lib.convrot_prepare(None, BF16, 4, 4096, G, 0, None, None, None)
    assert rc in (1, 2) and _err(lib) == msg


def test_prepare_rejects_shapes(lib):
    assert lib.convrot_prepare(None, BF16, 4, 320, 256, 0, None, None, None) == 1
    assert _err(lib) == "features 320 not divisible by ConvRot group size 256"
    assert lib.convrot_prepare(None, BF16, 4, 8, 4, 0, None, None, None) == 2
    assert "divisible by 16" in _err(lib)
    assert lib.convrot_prepare(None, BF16, 1, 131072, 256, 0, None, None, None) == 2
    assert "at most 65536 features" in _err(lib)
    assert lib.convrot_prepare(None, 7, 1, 256, 256, 0, None, None, None) == 1
    assert lib.convrot_prepare(None, BF16, 1, 256, 256, 9, None, None, None) == 1
    assert lib.convrot_prepare(None, BF16, 1, 256, 256, 2 | 0x10, None, None, None) == 1
    # valid shape, nothing to do
    assert lib.convrot_prepare(None, BF16, 0, 256, 256, 0, None, None, None) == 0
    # valid shape, null buffers
    assert lib.convrot_prepare(None, BF16, 2, 256, 256, 0, None, None, None) == 1
    assert _err(lib) == "null pointer argument"


def test_gemm_validation(lib):
    assert lib.convrot_w4a4_gemm(None, 1, None, None, None, None, 4, 8, 48, None, BF16, None) == 1
    assert _err(lib) == "W4A4 GEMM requires K divisible by 32, got 48"
    assert lib.convrot_w4a4_gemm(None, 5, None, None, None, None, 4, 8, 64, None, BF16, None) == 1
    assert lib.convrot_w4a4_gemm(None, 1, None, None, None, None, 0, 8, 64, None, BF16, None) == 0
    assert lib.convrot_w4a16_gemm(None, 0, None, None, None, 4, 8, 64, None, BF16, None) == 1
    assert _err(lib) == "MPP W4A16 requires float16 or bfloat16 activation, got float32"
    assert lib.convrot_w4a16_gemm(None, BF16, None, None, None, 4, 8, 65600, None, BF16, None) == 2
    # packed weights of 2 GiB or more: the kernels' buffer offsets are 32-bit signed
    big_n = (1 << 31) // ((65536 // 128) * 1024) * 16  # ceil(K/128) * ceil(N/16) KB == 2 GiB
    assert lib.convrot_w4a16_gemm(None, BF16, None, None, None, 4, big_n, 65536, None, BF16, None) == 2
    assert _err(lib) == f"W4A16 GEMM packed weights are limited to 2 GiB (N={big_n} K=65536)"
    assert lib.convrot_w4a4_gemm(None, 1, None, None, None, None, 4, big_n, 65536, None, BF16, None) == 2
    assert lib.convrot_w4a4_gemm(None, 1, None, None, None, None, 4, big_n - 16, 65536, None, BF16, None) == 1
    assert _err(lib) == "null pointer argument"


def test_prepare_gelu_validation(lib):
    """convrot_prepare_gelu(head, Kh, head_stride, x, Kx, x_stride, dtype, rows, G, mode, out, scales, stream)."""
    g = lib.convrot_prepare_gelu
    assert g(None, 0, 0, None, 64, 64, BF16, 4, 64, 1 | 0x10, None, None, None) == 1
    assert _err(lib) == "the GELU producer always rotates (no CONVROT_PREP_NO_ROTATE)"
    assert g(None, 8, 8, None, 56, 56, BF16, 4, 64, 1, None, None, None) == 2
    assert _err(lib) == "the GELU producer requires head and x features divisible by 16, got 8 and 56"
    assert g(None, 16, 16, None, 64, 64, BF16, 4, 64, 1, None, None, None) == 1
    assert _err(lib) == "features 80 not divisible by ConvRot group size 64"
    assert g(None, 0, 0, None, 128, 64, BF16, 4, 64, 1, None, None, None) == 1
    assert _err(lib) == "row strides (head 0, x 64) shorter than the rows"
    assert g(None, 0, 0, None, 128, 128, BF16, 0, 64, 1, None, None, None) == 0  # no rows: nothing to do
    assert g(None, 0, 0, None, 128, 128, BF16, 4, 64, 1, None, None, None) == 1
    assert _err(lib) == "null pointer argument"


def test_gemm_residual_validation(lib):
    """convrot_w4a4_gemm_residual(act, fmt, xs, qw, ws, bias, M, N, K, residual, gate, gate_stride,
    rows_per_gate, out, dtype, stream): every call below fails its checks before any launch
    (the non-null pointers are placeholders that are never dereferenced)."""
    g = lib.convrot_w4a4_gemm_residual
    p = 0x10000  # 16-byte aligned placeholder
    assert g(None, 1, None, None, None, None, 4, 32, 48, None, None, 0, 1, None, BF16, None) == 1
    assert _err(lib) == "W4A4 GEMM requires K divisible by 32, got 48"
    assert g(p, 1, p, p, p, None, 4, 32, 64, p, p, 32, 0, p, BF16, None) == 1
    assert _err(lib) == "rows_per_gate must be positive, got 0"
    assert g(p, 1, p, p, p, None, 0, 32, 64, None, None, 0, 1, p, BF16, None) == 0  # no rows: nothing to do
    assert g(p, 1, p, p, p, None, 4, 32, 64, None, None, 0, 1, p, BF16, None) == 1
    assert _err(lib) == "null pointer argument"
    assert g(p, 1, p, p, p, None, 4, 32, 64, p + 8, None, 0, 1, p, BF16, None) == 1
    assert _err(lib) == "residual and gate must be 16-byte aligned"
    assert g(p, 1, p, p, p, None, 4, 32, 64, p, p + 4, 32, 2, p, BF16, None) == 1
    assert _err(lib) == "residual and gate must be 16-byte aligned"
    assert g(p, 1, p, p, p, None, 4, 32, 64, p, p, 16, 2, p, BF16, None) == 1
    assert _err(lib) == "gate rows 16 elements apart overlap (N=32)"
    assert g(p, 1, p, p, p, None, 4, 32, 64, p, p, 16, 2, p + 4, BF16, None) == 1
    assert _err(lib) == "act, qweight and out must be 16-byte aligned"
    # the W4A16 variant: its own GEMM checks, then the same residual checks
    h = lib.convrot_w4a16_gemm_residual
    assert h(p, 0, p, p, None, 4, 32, 64, p, None, 0, 1, p, BF16, None) == 1
    assert _err(lib) == "MPP W4A16 requires float16 or bfloat16 activation, got float32"
    assert h(p, BF16, p, p, None, 4, 32, 64, p, p, 32, 0, p, BF16, None) == 1
    assert _err(lib) == "rows_per_gate must be positive, got 0"
    assert h(p, BF16, p, p, None, 4, 32, 64, None, None, 0, 1, p, BF16, None) == 1
    assert _err(lib) == "null pointer argument"
    assert h(p, BF16, p, p, None, 4, 32, 64, p, p, 16, 2, p, BF16, None) == 1
    assert _err(lib) == "gate rows 16 elements apart overlap (N=32)"


def test_w4a16_gemm_ws_validation(lib):
    """convrot_w4a16_gemm_ws runs convrot_w4a16_gemm's checks, then the workspace and residual
    checks of convrot_w4a4_gemm_ws, before anything is launched."""
    g = lib.convrot_w4a16_gemm_ws
    p = 0x10000
    assert g(p, 0, p, p, None, 4, 32, 64, None, None, 0, 1, None, 0, p, BF16, None) == 1
    assert _err(lib) == "MPP W4A16 requires float16 or bfloat16 activation, got float32"
    assert g(p, BF16, p, p, None, 4, 32, 48, None, None, 0, 1, None, 0, p, BF16, None) == 1
    assert _err(lib) == "W4A16 GEMM requires K divisible by 32, got 48"
    assert g(p, BF16, p, p, None, 4, 32, 64, None, None, 0, 1, None, 4096, p, BF16, None) == 1
    assert _err(lib) == "invalid workspace (4096 bytes)"
    assert g(p, BF16, p, p, None, 4, 32, 64, None, None, 0, 1, p + 16, 4096, p, BF16, None) == 1
    assert _err(lib) == "workspace must be 256-byte aligned"
    assert g(p, BF16, p, p, None, 4, 32, 64, None, p, 32, 1, None, 0, p, BF16, None) == 1
    assert _err(lib) == "a gate needs a residual"
    assert g(p, BF16, p, p, None, 4, 32, 64, p, p, 32, 0, None, 0, p, BF16, None) == 1
    assert _err(lib) == "rows_per_gate must be positive, got 0"
    assert g(p, BF16, p, p, None, 0, 32, 64, None, None, 0, 1, None, 0, p, BF16, None) == 0  # M = 0: nothing to do


def test_gemm_noalloc_validation(lib):
    """convrot_w4a4_gemm_noalloc (arguments of convrot_w4a4_gemm_residual; residual NULL: the
    plain GEMM) rejects bad arguments before it touches its scratch or launches anything."""
    g = lib.convrot_w4a4_gemm_noalloc
    p = 0x10000
    assert g(None, 1, None, None, None, None, 4, 32, 48, None, None, 0, 1, None, BF16, None) == 1
    assert _err(lib) == "W4A4 GEMM requires K divisible by 32, got 48"
    assert g(p, 1, p, p, p, None, 0, 32, 64, None, None, 0, 1, p, BF16, None) == 0  # no rows: nothing to do
    assert g(p, 1, p, p, p, None, 4, 32, 64, None, p, 32, 1, p, BF16, None) == 1
    assert _err(lib) == "a gate needs a residual"
    assert g(p, 1, p, p, p, None, 4, 32, 64, p, p, 32, 0, p, BF16, None) == 1
    assert _err(lib) == "rows_per_gate must be positive, got 0"
    assert g(p, 1, p, p, p, None, 4, 32, 64, p + 8, None, 0, 1, p, BF16, None) == 1
    assert _err(lib) == "residual and gate must be 16-byte aligned"
    assert g(None, 1, p, p, p, None, 4, 32, 64, None, None, 0, 1, p, BF16, None) == 1
    assert _err(lib) == "null pointer argument"


def test_repack_validation(lib):
    assert lib.convrot_repack_weight(None, 0, None, 1, 33, 64, None) == 1
    assert _err(lib) == "MPP int4 packing requires even out_features, got 33"
    assert lib.convrot_repack_weight(None, 1, None, 0, 34, 63, None) == 1
    assert lib.convrot_repack_weight(None, 0, None, 5, 34, 64, None) == 1
    assert lib.convrot_pack_int4(None, 0, 8, None, None) == 0


def test_errors_are_thread_local(lib):
    import threading

    lib.convrot_w4a4_gemm(None, 1, None, None, None, None, 4, 8, 48, None, BF16, None)
    seen = {}

    def other():
        seen["msg"] = lib.convrot_last_error().decode()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == "" and _err(lib).startswith("W4A4 GEMM requires")


def test_fp6_validation(lib):
    """The FP6 entry points reject what their kernels cannot address before any launch: a
    weight conversion with in_features not divisible by 128 (no FP6 layout, no GEMM accepts
    it), and operands whose FP6 blocks pass 2^32 - 2^20 bytes (the GEMM's buffer offsets are
    32-bit; e.g. 373k rows at K = 15360).  ConvRotLinear sends such products to INT8."""
    import ctypes

    import torch

    from convrot_mlx_amd import core

    p = 0x10000
    assert lib.convrot_weight_fp6(None, None, 64, 192, None) == 2
    assert _err(lib) == "FP6 operands require in_features divisible by 128, got 192"
    assert lib.convrot_weight_fp6(p, p, 0, 256, None) == 0  # valid, nothing to do
    g = lib.convrot_w4a4_gemm_fp6
    limit = core.FP6_MAX_OPERAND_BYTES
    assert limit == (1 << 32) - (1 << 20)
    big_m = (limit // (120 * 1536) + 1) * 16  # first 16-row count past the limit at K = 15360
    assert lib.convrot_fp6_bytes(big_m, 15360) > limit >= lib.convrot_fp6_bytes(big_m - 16, 15360)
    assert g(p, p, p, p, None, big_m, 3072, 15360, p, BF16, None) == 2
    assert "exceeds" in _err(lib) and "INT8" in _err(lib)
    assert g(p, p, p, p, None, 4608, big_m, 15360, p, BF16, None) == 2  # a weight with that many columns
    assert g(None, p, p, p, None, big_m - 16, 3072, 15360, p, BF16, None) == 1  # in range: next check
    assert _err(lib) == "null pointer argument"
    assert not core.fp6_eligible(big_m, 3072, 15360, torch.bfloat16)
    assert core.fp6_eligible(big_m - 16, 3072, 15360, torch.bfloat16) == core.fp6_operands_enabled()
    assert core.fp6_bytes(4608, 3072) == lib.convrot_fp6_bytes(4608, 3072) == 24 * 288 * 1536
    bm, bn = ctypes.c_int(0), ctypes.c_int(0)
    assert lib.convrot_w4a4_fp6_tile(0, 64, ctypes.byref(bm), ctypes.byref(bn)) == 1
    # compact weights: the same shape rules, and a gate needs a residual
    assert lib.convrot_weight_fp6_compact(None, None, None, 64, 192, None) == 2
    assert _err(lib) == "FP6 operands require in_features divisible by 128, got 192"
    assert lib.convrot_weight_fp6_compact(p, p, p + 2, 64, 256, None) == 1
    assert "4-byte aligned" in _err(lib)
    c = lib.convrot_w4a4_gemm_fp6_compact
    assert c(p, p, p, p, None, big_m, 3072, 15360, None, None, 0, 1, p, BF16, None) == 2
    assert c(p, p, p, p, None, 64, 64, 256, None, p, 64, 1, p, BF16, None) == 1
    assert _err(lib) == "a gate needs a residual"
    assert c(p, p, p, p, None, 64, 64, 256, p, p, 64, 0, p, BF16, None) == 1
    assert _err(lib) == "rows_per_gate must be positive, got 0"
    assert c(p, p, p, p, None, 0, 64, 256, None, None, 0, 1, p, BF16, None) == 0


@pytest.mark.parametrize("name,value", [("fp6_tile", "64x64"), ("fp6_tile", "256x256x"), ("fp6_tile", "256x192"),
                                        ("gemm_tile", "100x100"), ("gemm_tile", "192x128w2x2"),
                                        ("gemm_tile", "256x256w4x2s3"), ("w4a16_tile", "192x128"),
                                        ("w4a4_smallm_cfg", "T"), ("prep_ni", "x")])
def test_tuning_rejects_unbuilt_tiles(lib, name, value):
    """A tile override the library does not build is an error, not a silent fallback to the
    automatic plan (256x256w4x2 exists only in the register-staged kernel, which has no ring
    depth)."""
    assert lib.convrot_set_tuning(name.encode(), value.encode()) == 1
    assert _err(lib) == f"invalid value '{value}' for tuning override '{name}'"


@pytest.mark.parametrize("name,value", [("fp6_tile", "128x192"), ("gemm_tile", "288x192w2x2"),
                                        ("gemm_tile", "256x256w4x2"), ("gemm_tile", "128x256w2x4s4"),
                                        ("w4a16_tile", "256x128")])
def test_tuning_accepts_built_tiles(lib, name, value):
    import ctypes

    try:
        assert lib.convrot_set_tuning(name.encode(), value.encode()) == 0
        if name == "fp6_tile":  # the forced tile is what the plan query reports (no device needed)
            bm, bn = ctypes.c_int(0), ctypes.c_int(0)
            assert lib.convrot_w4a4_fp6_tile(4608, 3072, ctypes.byref(bm), ctypes.byref(bn)) == 0
            assert f"{bm.value}x{bn.value}" == value
    finally:
        assert lib.convrot_set_tuning(name.encode(), None) == 0


# The automatic FP6 tile on a 256-CU device (the query falls back to 256 CUs without a GPU):
# the 8-wave 256x256 tile at every config-3 shape, 128x192 at config 2's N = 3072 and
# 3072 -> 12288 taken by 128x128 once four or more of its tiles fall to each CU.
@pytest.mark.parametrize("M,N,tile", [(4608, 9216, "256x256"), (4608, 3072, "256x256"), (4608, 12288, "256x256"),
                                      (4608, 21504, "256x256"), (1536, 3072, "128x192"), (1536, 9216, "256x256"),
                                      (1536, 12288, "128x128"), (512, 3072, "128x128"), (512, 9216, "128x192"),
                                      (1024, 12288, "256x256")])
def test_fp6_plan(lib, M, N, tile):
    import ctypes

    bm, bn = ctypes.c_int(0), ctypes.c_int(0)
    assert lib.convrot_w4a4_fp6_tile(M, N, ctypes.byref(bm), ctypes.byref(bn)) == 0
    assert f"{bm.value}x{bn.value}" == tile
