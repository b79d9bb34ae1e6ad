"""GPU parity of the gated-residual W4A4 GEMM epilogue against the oracle, bit for bit:
out = dt(residual + dt(gate * dt(linear))) through every W4A4 kernel (few-row, DMA
data-parallel tiles, stream-K, register-staged, packed activations), every output dtype,
each gate form a DiT uses (per image, a chunk of a modulation vector, one vector, full,
none) plus an odd gate row stride, ragged N, in place into the residual, and through
ConvRotLinear's forward / forward_gelu / forward_modulated against the unfused
composition torch evaluates."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import TORCH_DT, from_dev, to_dev

pytestmark = pytest.mark.gpu


def _api():
    import convrot_mlx_amd as api

    return api


# name: (environment, images B, rows per image L, K, N, activation format)
PATHS = {
    "smallm_A": ({"w4a4_smallm_cfg": "A"}, 1, 7, 256, 196, "int8"),
    "smallm_C": ({"gemm_smallm_max": "64", "w4a4_smallm_cfg": "C"}, 2, 20, 384, 70, "int8"),
    "dma_128x128": ({"gemm_smallm_max": "0", "gemm_tile": "128x128w2x2", "gemm_sk": "0"},
                    2, 150, 512, 200, "int8"),
    "dma_256x256": ({"gemm_smallm_max": "0", "gemm_tile": "256x256w2x4", "gemm_sk": "0"},
                    3, 100, 384, 260, "int8"),
    "dma_192x128": ({"gemm_smallm_max": "0", "gemm_tile": "192x128w4x2", "gemm_sk": "0"},
                    2, 150, 256, 136, "int8"),
    "dma_288x192": ({"gemm_smallm_max": "0", "gemm_tile": "288x192w2x2", "gemm_sk": "0"},
                    2, 330, 512, 400, "int8"),
    "dma_288x192_odd": ({"gemm_smallm_max": "0", "gemm_tile": "288x192w2x2", "gemm_sk": "0"},
                        3, 101, 256, 202, "int8"),
    "stream_k": ({"gemm_smallm_max": "0", "gemm_tile": "128x256w2x4", "gemm_sk": "1",
                  "gemm_sk_min": "1"}, 2, 130, 1024, 270, "int8"),
    "register": ({"gemm_smallm_max": "0", "gemm_no_dma": "1"}, 2, 90, 256, 100, "int8"),
    "packed": ({"gemm_smallm_max": "0"}, 2, 90, 256, 102, "packed"),
    "packed_kernel": ({}, 2, 90, 256, 102, "packed_kernel"),
    "fp6_256x256": ({"fp6_tile": "256x256"}, 2, 150, 384, 270, "fp6"),
    "fp6_256x224": ({"fp6_tile": "256x224"}, 3, 101, 256, 460, "fp6"),
    "fp6_128x256": ({"fp6_tile": "128x256"}, 2, 130, 640, 202, "fp6"),
    "fp6_128x128": ({"fp6_tile": "128x128"}, 3, 101, 384, 330, "fp6"),
    "fp6_128x192": ({"fp6_tile": "128x192"}, 2, 130, 512, 410, "fp6"),
}
_ENV_KEYS = ("w4a4_smallm_cfg", "gemm_smallm_max", "gemm_tile", "gemm_sk",
             "gemm_sk_min", "gemm_no_dma", "fp6_tile")


def _set_env(tuning, env):
    for key in _ENV_KEYS:
        tuning.set(key, None)
    for key, value in env.items():
        tuning.set(key, value)


def _operands(orc, seed, M, K, N, dtype):
    rng = np.random.default_rng(seed)
    a = rng.integers(-8, 8, size=(M, K), dtype=np.int8)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    xs = rng.uniform(0.01, 0.2, size=(M,)).astype(np.float32)
    ws = rng.uniform(0.01, 0.2, size=(N,)).astype(np.float32)
    b = rng.normal(size=(N,)).astype(np.float32)
    res = orc.from_f32((rng.normal(size=(M, N)) * 8.0).astype(np.float32), dtype)
    lin = orc.w4a4_matmul_codes(a, w, xs, ws, b, dtype)
    return rng, a, w, xs, ws, b, res, lin


def _gate(orc, rng, form, B, L, N, dtype, dev):
    """(device gate or None, oracle gate rows [G, N] or None, rows per gate row)."""
    if form == "none":
        return None, None, 1
    rows_g = {"per_image": B, "chunk": B, "odd_stride": B, "vector": 1, "full": B * L}[form]
    g = orc.from_f32(rng.normal(size=(rows_g, N)).astype(np.float32), dtype)
    rpg = {"full": 1, "vector": B * L}.get(form, L)
    if form == "per_image":
        gd = to_dev(g, dtype, dev).reshape(B, 1, N)
    elif form == "chunk":  # one of three gates cut from a [B, 3N] modulation output
        wide = np.zeros((B, 3 * N), g.dtype)
        wide[:, N:2 * N] = g
        gd = to_dev(wide, dtype, dev)[:, None, :].chunk(3, dim=-1)[1]
    elif form == "odd_stride":  # rows N + 3 elements apart: the kernel's element-wise gate loads
        wide = np.zeros((B, N + 3), g.dtype)
        wide[:, :N] = g
        gd = to_dev(wide, dtype, dev)[:, None, :N]
    elif form == "vector":
        gd = to_dev(g, dtype, dev).reshape(N)
    else:
        gd = to_dev(g, dtype, dev).reshape(B, L, N)
    return gd, g, rpg


def _call(api, orc, dev, fmt, a, w, xs, ws, b, dtype, residual, gate, inplace=False):
    N = w.shape[0]
    wq = torch.from_numpy(orc.codes_to_cdna4(w)).to(dev)
    args = (torch.from_numpy(xs).to(dev), torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev))
    kw = dict(output_dtype=TORCH_DT[dtype], out_features=N, residual=residual, gate=gate, inplace=inplace)
    if fmt == "packed":
        qact = torch.from_numpy(orc.pack_signed_int4(a)).to(dev)
        return api.hip_w4a4_matmul(qact, wq, *args, **kw)
    if fmt == "fp6":  # FP6 operands (the same epilogue)
        a6 = torch.from_numpy(orc.codes_to_fp6(a)).to(dev)
        w6 = torch.from_numpy(orc.codes_to_fp6(w)).to(dev)
        kw.pop("out_features")
        return api.hip_w4a4_fp6_matmul(a6, w6, *args, rows=a.shape[0], out_features=N, in_features=a.shape[1], **kw)
    if fmt == "packed_kernel":  # the C ABI's register-staged kernel on the packed codes
        from convrot_mlx_amd import _native as nat

        qact = torch.from_numpy(orc.pack_signed_int4(a)).to(dev)
        M = a.shape[0]
        res = residual.reshape(M, N)
        g = gate.expand(residual.shape) if gate is not None else None
        assert g is None or g.stride(-2) == 0, "per-image gates only"
        out = res if inplace else torch.empty((M, N), dtype=TORCH_DT[dtype], device=dev)
        gp = nat.ptr(g) if g is not None else nat.ptr(None)
        gstride = g.stride(0) if g is not None else 0
        rpg = residual.shape[1] if residual.dim() == 3 else M
        nat.check(nat.load().convrot_w4a4_gemm_residual(
            nat.ptr(qact), nat.ACT_PACKED, nat.ptr(args[0]), nat.ptr(wq), nat.ptr(args[1]), nat.ptr(args[2]),
            M, N, a.shape[1], nat.ptr(res), gp, gstride, rpg, nat.ptr(out), nat.dtype_code(TORCH_DT[dtype]),
            nat.stream_of(dev)))
        return out
    return api.hip_w4a4_int8_matmul(torch.from_numpy(a).to(dev), wq, *args, **kw)


def _assert_exact(got, want, label):
    if want.dtype == np.float32:
        bad = int((got.view(np.uint32) != want.view(np.uint32)).sum())
    else:
        bad = int((got != want).sum())
    assert bad == 0, f"{label}: {bad} of {want.size} outputs differ"


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("path", list(PATHS))
def test_every_kernel_path(orc, dev, tuning, path, dtype):
    """Per-image gates ([B, 1, N]) on every W4A4 kernel; out of place, then in place."""
    api = _api()
    env, B, L, K, N, fmt = PATHS[path]
    _set_env(tuning, env)
    M = B * L
    rng, a, w, xs, ws, b, res, lin = _operands(orc, 101, M, K, N, dtype)
    gd, g, rpg = _gate(orc, rng, "per_image", B, L, N, dtype, dev)
    want = orc.gated_residual(lin, res, g, rpg, dtype)
    rd = to_dev(res, dtype, dev).reshape(B, L, N)
    out = _call(api, orc, dev, fmt, a, w, xs, ws, b, dtype, rd, gd)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (M, N)
    _assert_exact(from_dev(out), want, f"{path} {dtype}")
    assert np.array_equal(from_dev(rd).reshape(M, N), res)  # out of place leaves the residual
    back = _call(api, orc, dev, fmt, a, w, xs, ws, b, dtype, rd, gd, inplace=True)
    torch.cuda.synchronize()
    assert back.data_ptr() == rd.data_ptr()
    _assert_exact(from_dev(rd).reshape(M, N), want, f"{path} {dtype} in place")


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("form", ["chunk", "odd_stride", "vector", "full", "none"])
@pytest.mark.parametrize("path", ["smallm_A", "dma_128x128", "register", "dma_288x192", "fp6_256x224"])
def test_gate_forms(orc, dev, tuning, path, form, dtype):
    api = _api()
    env, B, L, K, N, fmt = PATHS[path]
    _set_env(tuning, env)
    M = B * L
    rng, a, w, xs, ws, b, res, lin = _operands(orc, 202, M, K, N, dtype)
    gd, g, rpg = _gate(orc, rng, form, B, L, N, dtype, dev)
    want = orc.gated_residual(lin, res, g, rpg, dtype)
    rd = to_dev(res, dtype, dev).reshape(B, L, N)
    out = _call(api, orc, dev, fmt, a, w, xs, ws, b, dtype, rd, gd)
    torch.cuda.synchronize()
    _assert_exact(from_dev(out), want, f"{path} {form} {dtype}")
    # and the unfused composition torch would evaluate on the plain GEMM output
    plain = _call(api, orc, dev, fmt, a, w, xs, ws, b, dtype, None, None).reshape(B, L, N)
    ref = rd + plain if gd is None else rd + gd * plain
    torch.cuda.synchronize()
    assert torch.equal(out.reshape(B, L, N), ref)


def test_residual_argument_errors(dev):
    api = _api()
    a = torch.zeros((4, 128), dtype=torch.int8, device=dev)
    wq = torch.zeros(api.cdna4_shape(32, 128), dtype=torch.uint8, device=dev)
    xs = torch.ones(4, device=dev)
    ws = torch.ones(32, device=dev)
    res = torch.zeros((4, 32), dtype=torch.bfloat16, device=dev)
    kw = dict(output_dtype=torch.bfloat16, out_features=32)
    with pytest.raises(ValueError, match="residual"):
        api.hip_w4a4_int8_matmul(a, wq, xs, ws, None, residual=res[:, :16], **kw)
    with pytest.raises(ValueError, match="dtype"):
        api.hip_w4a4_int8_matmul(a, wq, xs, ws, None, residual=res.float(), **kw)
    with pytest.raises(ValueError, match="broadcast"):
        api.hip_w4a4_int8_matmul(a, wq, xs, ws, None, residual=res, gate=torch.zeros((3, 32), dtype=torch.bfloat16,
                                                                                     device=dev), **kw)
    with pytest.raises(ValueError, match="need a residual"):
        api.hip_w4a4_int8_matmul(a, wq, xs, ws, None, gate=res, **kw)
    with pytest.raises(ValueError, match="contiguous"):
        api.hip_w4a4_int8_matmul(a, wq, xs, ws, None, residual=torch.zeros((32, 4), dtype=torch.bfloat16,
                                                                           device=dev).t(), inplace=True, **kw)


def _layer(api, orc, dev, backend, K, N, G, seed):
    rng = np.random.default_rng(seed)
    dense_w = orc.from_f32(rng.normal(0, 0.02, size=(N, K)).astype(np.float32), "bfloat16")
    dense_b = rng.normal(size=(N,)).astype(np.float32)
    qw, ws = api.quantize_convrot_weight(to_dev(dense_w, "bfloat16", dev), G)
    return api.ConvRotLinear(K, N, group_size=G, backend=backend, device=dev).load_nk_weight(
        qw, ws, torch.from_numpy(dense_b).to(dev))


@pytest.mark.parametrize("backend", ["hip-w4a4", "hip-w4a16"])
def test_layer_forwards(orc, dev, backend):
    """ConvRotLinear.forward / forward_gelu / forward_modulated with residual and gate equal
    residual + gate * (the same call without them), evaluated by torch, bit for bit."""
    api = _api()
    B, L, K, N, G = 2, 24, 256, 192, 64
    layer = _layer(api, orc, dev, backend, K, N, G, 5)
    gen = torch.Generator(device=dev).manual_seed(9)
    x = torch.randn(B, L, K, device=dev, generator=gen).to(torch.bfloat16)
    res = (torch.randn(B, L, N, device=dev, generator=gen) * 4).to(torch.bfloat16)
    mod = torch.randn(B, 3 * N, device=dev, generator=gen).to(torch.bfloat16)
    gate = mod[:, None, :].chunk(3, dim=-1)[2]
    shift = torch.randn(B, 1, K, device=dev, generator=gen).to(torch.bfloat16)
    scale = torch.randn(B, 1, K, device=dev, generator=gen).to(torch.bfloat16)
    calls = {
        "forward": lambda **kw: layer(x, **kw),
        "forward_gelu": lambda **kw: layer.forward_gelu(x[..., 64:], head=x[..., :64], **kw),
        "forward_modulated": lambda **kw: layer.forward_modulated(x, shift, scale, **kw),
    }
    for name, call in calls.items():
        plain = call()
        want = res + gate * plain
        got = call(residual=res, gate=gate)
        assert torch.equal(got, want), name
        assert torch.equal(call(residual=res), res + plain), name
        r2 = res.clone()
        assert call(residual=r2, gate=gate, inplace=True) is r2
        assert torch.equal(r2, want), name


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("cfg,B,L,K,N", [("A", 1, 5, 256, 200), ("A", 2, 12, 384, 200), ("B", 2, 4, 384, 70),
                                         ("C", 2, 20, 256, 136), ("D", 2, 7, 384, 200), ("E", 2, 13, 256, 330),
                                         ("F", 1, 40, 512, 96), ("T", 2, 100, 384, 260)])
def test_w4a16_kernels(orc, dev, tuning, cfg, B, L, K, N, dtype):
    """The W4A16 GEMM's gated-residual epilogue on each of its kernels (splits A to F and
    the tiled kernel, forced; split A below and from 8 rows, i.e. both activation load orders),
    per-image gates, ragged N: residual + gate * linear equals
    torch's composition on the same kernel's plain output, bit for bit, out of place and in
    place (the product itself is W4A16 arithmetic, checked against the oracle elsewhere)."""
    api = _api()
    tuning.set("w4a16_cfg", cfg)
    M = B * L
    rng = np.random.default_rng(303)
    act_dt = "float16" if dtype == "float16" else "bfloat16"
    act = to_dev(orc.from_f32(rng.normal(size=(M, K)).astype(np.float32), act_dt), act_dt, dev)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    wq = torch.from_numpy(orc.codes_to_cdna4(w)).to(dev)
    ws = torch.from_numpy(rng.uniform(0.001, 0.01, size=N).astype(np.float32)).to(dev)
    b = torch.from_numpy(rng.normal(size=N).astype(np.float32)).to(dev)
    res = to_dev(orc.from_f32((rng.normal(size=(M, N)) * 4).astype(np.float32), dtype), dtype, dev).reshape(B, L, N)
    gate = to_dev(orc.from_f32(rng.normal(size=(B, N)).astype(np.float32), dtype), dtype, dev).reshape(B, 1, N)
    kw = dict(output_dtype=TORCH_DT[dtype], out_features=N)
    plain = api.hip_w4a16_matmul(act, wq, ws, b, **kw).reshape(B, L, N)
    fused = api.hip_w4a16_matmul(act, wq, ws, b, residual=res, gate=gate, **kw)
    torch.cuda.synchronize()
    want = res + gate * plain
    assert torch.equal(fused.reshape(B, L, N), want)
    assert torch.equal(api.hip_w4a16_matmul(act, wq, ws, b, residual=res, **kw).reshape(B, L, N), res + plain)
    r2 = res.clone()
    api.hip_w4a16_matmul(act, wq, ws, b, residual=r2, gate=gate, inplace=True, **kw)
    torch.cuda.synchronize()
    assert torch.equal(r2, want)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("gate_kind", ["per_image", "chunked"])
def test_w4a16_tiled_vector_residual(orc, dev, tuning, dtype, gate_kind):
    """The tiled W4A16 kernel's 16-byte residual and gate loads (N and the gate stride
    multiples of 8): a per-image [B, 1, N] gate and a chunk of a [B, 1, 3N] modulation
    output, out of place and in place, equal torch's composition on the plain output."""
    api = _api()
    tuning.set("w4a16_cfg", "T")
    B, L, K, N = 2, 160, 384, 256
    M = B * L
    rng = np.random.default_rng(404)
    act = to_dev(orc.from_f32(rng.normal(size=(M, K)).astype(np.float32), dtype), dtype, dev)
    w = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    wq = torch.from_numpy(orc.codes_to_cdna4(w)).to(dev)
    ws = torch.from_numpy(rng.uniform(0.001, 0.01, size=N).astype(np.float32)).to(dev)
    b = torch.from_numpy(rng.normal(size=N).astype(np.float32)).to(dev)
    res = to_dev(orc.from_f32((rng.normal(size=(M, N)) * 4).astype(np.float32), dtype), dtype, dev).reshape(B, L, N)
    if gate_kind == "per_image":
        gate = to_dev(orc.from_f32(rng.normal(size=(B, N)).astype(np.float32), dtype), dtype, dev).reshape(B, 1, N)
    else:
        mod = to_dev(orc.from_f32(rng.normal(size=(B, 3 * N)).astype(np.float32), dtype), dtype, dev)
        gate = mod[:, None, :].chunk(3, dim=-1)[2]
    kw = dict(output_dtype=TORCH_DT[dtype], out_features=N)
    plain = api.hip_w4a16_matmul(act, wq, ws, b, **kw).reshape(B, L, N)
    want = res + gate * plain
    fused = api.hip_w4a16_matmul(act, wq, ws, b, residual=res, gate=gate, **kw)
    torch.cuda.synchronize()
    assert torch.equal(fused.reshape(B, L, N), want)
    r2 = res.clone()
    api.hip_w4a16_matmul(act, wq, ws, b, residual=r2, gate=gate, inplace=True, **kw)
    torch.cuda.synchronize()
    assert torch.equal(r2, want)
