"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py):
the oracle must keep reproducing them (CPU), and the HIP path must match them (GPU)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from _util import from_dev, to_dev

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_oracle_reproduces_fixtures(orc):
    f = load("prep_s18")
    q, s = orc.prepare_convrot_activation(f["x"], "bfloat16", int(f["group_size"]))
    assert np.array_equal(q, f["qact"]) and np.array_equal(s, f["scales"])
    f = load("prep_h3")
    q, s = orc.prepare_convrot_activation(f["x"], "bfloat16", 64)
    assert np.array_equal(q, f["qact"]) and np.array_equal(s, f["scales"])
    assert np.array_equal(orc.regular_hadamard(f["x"], "bfloat16", 64), f["rotated"])
    f = load("gemm_edges")
    out = orc.reference_w4a4_matmul(f["qact"], f["qweight_nk"], f["xscales"], f["wscales"], f["bias"], "float32")
    assert np.array_equal(out.view(np.uint32), f["out_f32"].view(np.uint32))
    assert np.array_equal(orc.repack_nk_weight_for_mpp(f["qweight_nk"]), f["qweight_kn"])
    f = load("pack_literal")
    assert np.array_equal(orc.pack_signed_int4(f["values"]), f["packed"])


@pytest.mark.gpu
def test_hip_matches_fixtures(dev):
    import convrot_mlx_amd as api

    f = load("prep_s18")
    q, s = api.metal_fused_prepare_convrot_activation(to_dev(f["x"], "bfloat16", dev))
    assert np.array_equal(from_dev(q), f["qact"]) and np.array_equal(from_dev(s), f["scales"])
    f = load("prep_h3")
    xd = to_dev(f["x"], "bfloat16", dev)
    q, s = api.metal_fused_prepare_convrot_activation(xd, 64)
    assert np.array_equal(from_dev(q), f["qact"]) and np.array_equal(from_dev(s), f["scales"])
    assert np.array_equal(from_dev(api.metal_fused_rotate_convrot_activation(xd, 64)), f["rotated"])
    f = load("rotate_s1802")
    assert np.array_equal(from_dev(api.regular_hadamard(to_dev(f["x"], "bfloat16", dev))), f["rotated"])
    f = load("gemm_edges")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    out = api.mpp_w4a4_matmul(t(f["qact"]), t(f["qweight_kn"]), t(f["xscales"]), t(f["wscales"]), t(f["bias"]),
                              output_dtype=torch.float32)
    assert np.array_equal(from_dev(out).view(np.uint32), f["out_f32"].view(np.uint32))
    out = api.mpp_w4a4_matmul(t(f["qact"]), t(f["qweight_kn"]), t(f["xscales"]), t(f["wscales"]), t(f["bias"]),
                              output_dtype=torch.bfloat16)
    assert np.array_equal(from_dev(out), f["out_bf16"])
    f = load("layer_33")
    qw, ws = api.quantize_convrot_weight(to_dev(f["dense_w"], "bfloat16", dev))
    layer = api.ConvRotLinear(256, 33, device=dev).load_nk_weight(qw, ws, t(f["dense_b"]))
    assert np.array_equal(from_dev(layer(to_dev(f["values"], "bfloat16", dev))), f["out"])
    f = load("pack_literal")
    assert np.array_equal(from_dev(api.pack_signed_int4(t(f["values"]))), f["packed"])
