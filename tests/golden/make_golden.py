#!/usr/bin/env python3
"""Write the golden fixtures under tests/golden/ from the CPU oracle.

The reference (Lumenbeing/convrot-mlx) holds no golden data beyond the literal
pack bytes of test_core.py:186-192, and its MLX runtime is not importable here,
so these vectors come from the oracle (oracle/), itself pinned by
tests/test_oracle.py.  Inputs reuse the seeds and shapes of
/root/reference/tests/test_core.py so that they are the reference tests' own
inputs (numpy default_rng streams, float32 -> bf16 RNE).  Run from the
repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import oracle as orc  # noqa: E402

OUT = Path(__file__).resolve().parent


def bf16_normal(seed, shape):
    rng = np.random.default_rng(seed)
    return orc.from_f32(rng.normal(size=shape).astype(np.float32), "bfloat16")


def main() -> None:
    orc.build()
    fx = {}
    # test_core.py:65-74 (seed 18, 19x512, G=256): fused packed preparation
    x = bf16_normal(18, (19, 512))
    q, s = orc.prepare_convrot_activation(x, "bfloat16", 256)
    fx["prep_s18"] = dict(x=x, qact=q, scales=s, group_size=np.array(256))
    # test_core.py:98-126 (seed 2026082305, 17x2688, G=64): packed, i8 and rotation
    x = bf16_normal(2026082305, (17, 2688))
    q, s = orc.prepare_convrot_activation(x, "bfloat16", 64)
    fx["prep_h3"] = dict(x=x, qact=q, scales=s, rotated=orc.regular_hadamard(x, "bfloat16", 64), group_size=np.array(64))
    # test_core.py:88-96 (seed 1802): rotation only
    x = bf16_normal(1802, (19, 512))
    fx["rotate_s1802"] = dict(x=x, rotated=orc.regular_hadamard(x, "bfloat16", 256), group_size=np.array(256))
    # test_core.py:213-283 (seed 2026082302, M=37 K=64 N=46): integer GEMM + epilogue
    rng = np.random.default_rng(2026082302)
    a = rng.integers(-7, 8, size=(37, 64), dtype=np.int8)
    w = rng.integers(-7, 8, size=(46, 64), dtype=np.int8)
    xs = rng.uniform(0.01, 0.2, size=(37,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(46,)).astype(np.float32)
    b = rng.normal(size=(46,)).astype(np.float32)
    fx["gemm_edges"] = dict(
        qact=orc.pack_signed_int4(a), qweight_nk=orc.pack_signed_int4(w), xscales=xs, wscales=ws, bias=b,
        out_f32=orc.w4a4_matmul_codes(a, w, xs, ws, b, "float32"),
        out_bf16=orc.w4a4_matmul_codes(a, w, xs, ws, b, "bfloat16"),
        qweight_kn=orc.repack_nk_weight_for_mpp(orc.pack_signed_int4(w)),
    )
    # test_core.py:375-402 (seed 29): layer (2,7,256) -> 33, bf16, bias
    rng = np.random.default_rng(29)
    dense_w = orc.from_f32(rng.normal(size=(33, 256)).astype(np.float32), "bfloat16")
    dense_b = rng.normal(size=(33,)).astype(np.float32)
    values = orc.from_f32(rng.normal(size=(2, 7, 256)).astype(np.float32), "bfloat16")
    wc, wsc = orc.prepare_codes(dense_w, "bfloat16", 256)
    ac, xsc = orc.prepare_codes(values.reshape(-1, 256), "bfloat16", 256)
    fx["layer_33"] = dict(dense_w=dense_w, dense_b=dense_b, values=values,
                          out=orc.w4a4_matmul_codes(ac, wc, xsc, wsc, dense_b, "bfloat16").reshape(2, 7, 33))
    # test_core.py:186-192 literal bytes (the reference's own known answer)
    fx["pack_literal"] = dict(values=np.array([[-8, -7, -1, 0, 1, 7, 3, -4]], np.int8),
                              packed=np.array([[0x98, 0x0F, 0x71, 0xC3]], np.uint8))
    for name, arrays in fx.items():
        np.savez_compressed(OUT / f"{name}.npz", **arrays)
        print(f"wrote {name}.npz")


if __name__ == "__main__":
    main()
