"""ctypes binding of libconvrot_amd.so (the C ABI in include/convrot_amd.h).

There is exactly one compute path: the gfx950 HIP kernels behind this
library.  If the library is missing, or a tensor is not on a ROCm device,
calls raise -- there is no CPU or PyTorch fallback.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_NAME = "libconvrot_amd.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

# include/convrot_amd.h
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_LAUNCH = 0, 1, 2, 3
PREP_PACKED, PREP_INT8, PREP_ROTATE, PREP_FP6, PREP_NO_ROTATE = 0, 1, 2, 3, 0x10
LAYOUT_NK, LAYOUT_KN, LAYOUT_CDNA4 = 0, 1, 2
ACT_PACKED, ACT_INT8 = 0, 1

# Every symbol the header declares, with its ctypes signature.
_vp, _i64, _i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
SIGNATURES = {
    "convrot_prepare": (_i32, [_vp, _i32, _i64, _i64, _i32, _i32, _vp, _vp, _vp]),
    "convrot_prepare_modulated": (_i32, [_vp, _i32, _i64, _i64, _i32, _i32, _vp, _vp, _i64, ctypes.c_float, _vp,
                                         _vp, _vp]),
    "convrot_prepare_gelu": (_i32, [_vp, _i64, _i64, _vp, _i64, _i64, _i32, _i64, _i32, _i32, _vp, _vp, _vp]),
    "convrot_w4a4_gemm": (_i32, [_vp, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i32, _vp]),
    "convrot_w4a4_gemm_residual": (_i32, [_vp, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64,
                                          _vp, _i32, _vp]),
    "convrot_w4a4_workspace_bytes": (_i64, []),
    "convrot_w4a4_gemm_ws": (_i32, [_vp, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _vp,
                                    _i64, _vp, _i32, _vp]),
    "convrot_w4a4_status": (_i32, [_vp, _vp]),
    "convrot_w4a4_gemm_noalloc": (_i32, [_vp, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64,
                                         _vp, _i32, _vp]),
    "convrot_w4a16_gemm": (_i32, [_vp, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i32, _vp]),
    "convrot_w4a16_gemm_residual": (_i32, [_vp, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _vp,
                                           _i32, _vp]),
    "convrot_w4a16_gemm_ws": (_i32, [_vp, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _i64,
                                     _vp, _i32, _vp]),
    "convrot_pack_int4": (_i32, [_vp, _i64, _i64, _vp, _vp]),
    "convrot_unpack_int4": (_i32, [_vp, _i64, _i64, _vp, _vp]),
    "convrot_repack_weight": (_i32, [_vp, _i32, _vp, _i32, _i64, _i64, _vp]),
    "convrot_cdna4_bytes": (_i64, [_i64, _i64]),
    "convrot_fp6_bytes": (_i64, [_i64, _i64]),
    "convrot_w4a4_fp6_tile": (_i32, [_i64, _i64, _vp, _vp]),
    "convrot_weight_fp6": (_i32, [_vp, _vp, _i64, _i64, _vp]),
    "convrot_w4a4_gemm_fp6": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i32, _vp]),
    "convrot_w4a4_gemm_fp6_residual": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _vp,
                                              _i32, _vp]),
    "convrot_weight_fp6_compact": (_i32, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "convrot_w4a4_gemm_fp6_compact": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _vp,
                                             _i32, _vp]),
    "convrot_last_error": (ctypes.c_char_p, []),
    "convrot_set_tuning": (_i32, [ctypes.c_char_p, ctypes.c_char_p]),
    "convrot_version": (ctypes.c_char_p, []),
}

_TORCH_DTYPES = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}

_lib: ctypes.CDLL | None = None


class ConvRotNativeError(RuntimeError):
    """The HIP library reported a launch/device failure."""


def load() -> ctypes.CDLL:
    """Load the library (once) and bind every declared symbol."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_NAME} is not built ({LIB_PATH}); run `make -C convrot-mlx_amd` or "
            "`python -c 'import __graft_entry__ as g; g.build()'` at the repository root. "
            "There is no fallback compute path."
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def version() -> str:
    return load().convrot_version().decode()


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _TORCH_DTYPES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16") from None


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one ROCm device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"ConvRot HIP kernels need ROCm device tensors, got a {t.device.type} tensor; "
                "this build has no CPU fallback"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def stream_of(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None else None)


def check(status: int) -> None:
    if status == OK:
        return
    msg = load().convrot_last_error().decode()
    if status in (ERR_INVALID, ERR_UNSUPPORTED):
        raise ValueError(msg)
    raise ConvRotNativeError(msg)


def set_tuning(name: str, value: str | None) -> None:
    """Force one of the library's kernel / plan choices (tuning sweeps and tests); None or ""
    restores the automatic choice.  Names: gemm_tile ("BMxBN[wWMxWN[sS]]"), gemm_sk (0/1),
    gemm_sk_min, gemm_no_dma, gemm_smallm_max, w4a4_smallm_cfg (A/B/C/F), w4a16_cfg
    (A/B/C/D/E/F, S: split K, T), w4a16_tile ("BMxBN"), prep_ni (1/3/4), sk_spin_limit, gemm_persist (0: never;
    G: always, on G workgroups), gemm_mfma32 (0/1), fp6_tile ("BMxBN": 256x256, 256x224, 128x256, 128x192, 128x128)."""
    check(load().convrot_set_tuning(name.encode(), None if value is None else str(value).encode()))


def cdna4_bytes(n: int, k: int) -> int:
    return int(load().convrot_cdna4_bytes(n, k))


def fp6_bytes(rows: int, k: int) -> int:
    return int(load().convrot_fp6_bytes(rows, k))


def fp6_tile(m: int, n: int) -> tuple[int, int]:
    """The (BM, BN) tile the FP6 W4A4 GEMM runs for an m x n product."""
    bm, bn = ctypes.c_int(0), ctypes.c_int(0)
    check(load().convrot_w4a4_fp6_tile(m, n, ctypes.byref(bm), ctypes.byref(bn)))
    return bm.value, bn.value
