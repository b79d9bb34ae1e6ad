"""Random-init FLUX.1-dev-architecture DiT in torch, and the config-5 measurement.

The reference runs FLUX.1 Dev through Apple's MLX example runtime and swaps its
Linears for ConvRotLinear (/root/reference/examples/flux1_dev/adapter.py:45-70,
load_flow_convrot :73-106).  That runtime, the checkpoints and diffusers are
not available here, so this module restates the public FLUX.1 architecture
(the published "flux-dev" parameters: 19 double-stream and 38 single-stream
blocks, hidden 3072, 24 heads of 128, MLP ratio 4, 3-axis RoPE (16, 56, 56),
guidance embedding) with random weights, enough to time one denoising step and
measure how far the W4A4 model drifts from the dense one (benchmark config 5).

On the GPU attention is torch's fused flash / memory-efficient SDPA kernel in
bf16 (the unfused math backend, which issues batched bf16 products on transposed
views, is excluded); on the CPU it is written out in float32.  Everything else
runs in bf16.

    python examples/flux1_dev/dit.py            # prints one JSON line
"""

from __future__ import annotations

import argparse
import json
import math
import sys
import time
from dataclasses import dataclass, field
from pathlib import Path

import torch
import torch.nn.functional as F
from torch import nn
from torch.nn.attention import SDPBackend, sdpa_kernel

ROOT = Path(__file__).resolve().parents[2]
if str(ROOT / "convrot-mlx_amd") not in sys.path:
    sys.path.insert(0, str(ROOT / "convrot-mlx_amd"))


@dataclass
class FluxParams:
    in_channels: int = 64
    vec_in_dim: int = 768
    context_in_dim: int = 4096
    hidden_size: int = 3072
    mlp_ratio: float = 4.0
    num_heads: int = 24
    depth: int = 19
    depth_single_blocks: int = 38
    axes_dim: tuple = field(default=(16, 56, 56))
    theta: int = 10000
    qkv_bias: bool = True
    guidance_embed: bool = True


def timestep_embedding(t: torch.Tensor, dim: int, max_period: float = 10000.0, time_factor: float = 1000.0):
    t = time_factor * t.float()
    half = dim // 2
    freqs = torch.exp(-math.log(max_period) * torch.arange(half, dtype=torch.float32, device=t.device) / half)
    args = t[:, None] * freqs[None]
    return torch.cat([torch.cos(args), torch.sin(args)], dim=-1)


def rope(pos: torch.Tensor, dim: int, theta: int) -> torch.Tensor:
    """[B, L] positions -> [B, L, dim/2, 2, 2] rotation matrices (float32)."""
    scale = torch.arange(0, dim, 2, dtype=torch.float64, device=pos.device) / dim
    omega = 1.0 / (theta ** scale)
    ang = pos.to(torch.float64)[..., None] * omega  # outer product, no batched matmul
    rot = torch.stack([torch.cos(ang), -torch.sin(ang), torch.sin(ang), torch.cos(ang)], dim=-1)
    return rot.reshape(*ang.shape, 2, 2).float()


def apply_rope(x: torch.Tensor, freqs: torch.Tensor) -> torch.Tensor:
    """x [B, H, L, D] -> float32, rotated pairwise by freqs [B, 1, L, D/2, 2, 2]."""
    xf = x.float().reshape(*x.shape[:-1], -1, 1, 2)
    out = freqs[..., 0] * xf[..., 0] + freqs[..., 1] * xf[..., 1]
    return out.reshape(*x.shape)


def attention(q, k, v, pe):
    """Joint attention over [B, H, L, D] heads, RoPE applied in float32, heads merged.

    On the GPU this is torch's fused scaled-dot-product attention restricted to its flash /
    memory-efficient kernels (the unfused math backend is excluded, so an unsupported case
    raises instead of falling back).  Elsewhere it is written out in float32."""
    q, k = apply_rope(q, pe).to(v.dtype), apply_rope(k, pe).to(v.dtype)
    if q.is_cuda:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            out = F.scaled_dot_product_attention(q, k, v)
    else:
        scores = torch.matmul(q.float(), k.float().transpose(-1, -2).contiguous()) / math.sqrt(q.shape[-1])
        out = torch.matmul(torch.softmax(scores, dim=-1), v.float()).to(v.dtype)
    b, h, l, d = out.shape
    return out.transpose(1, 2).reshape(b, l, h * d)


class EmbedND(nn.Module):
    def __init__(self, theta: int, axes_dim):
        super().__init__()
        self.theta, self.axes_dim = theta, axes_dim

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        emb = torch.cat([rope(ids[..., i], self.axes_dim[i], self.theta) for i in range(ids.shape[-1])], dim=-3)
        return emb.unsqueeze(1)


class MLPEmbedder(nn.Module):
    def __init__(self, in_dim: int, hidden: int):
        super().__init__()
        self.in_layer = nn.Linear(in_dim, hidden)
        self.out_layer = nn.Linear(hidden, hidden)

    def forward(self, x):
        return self.out_layer(F.silu(self.in_layer(x)))


class RMSNorm(nn.Module):
    def __init__(self, dim: int):
        super().__init__()
        self.scale = nn.Parameter(torch.ones(dim))

    def forward(self, x):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(x.dtype) * self.scale


class QKNorm(nn.Module):
    def __init__(self, dim: int):
        super().__init__()
        self.query_norm, self.key_norm = RMSNorm(dim), RMSNorm(dim)

    def forward(self, q, k):
        return self.query_norm(q), self.key_norm(k)


class Modulation(nn.Module):
    def __init__(self, dim: int, double: bool):
        super().__init__()
        self.multiplier = 6 if double else 3
        self.lin = nn.Linear(dim, self.multiplier * dim)

    def forward(self, vec):
        out = self.lin(F.silu(vec))[:, None, :].chunk(self.multiplier, dim=-1)
        first = out[:3]
        second = out[3:] if self.multiplier == 6 else None
        return first, second  # (shift, scale, gate)


def modulated(linear: nn.Module, x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, fused: bool):
    """linear((1 + scale) * layer_norm(x) + shift).  With `fused` and a ConvRotLinear the
    normalization and modulation run inside its activation preparation (one kernel);
    otherwise as torch ops."""
    if fused and hasattr(linear, "forward_modulated"):
        return linear.forward_modulated(x, shift, scale, eps=1e-6)
    return linear((1 + scale) * F.layer_norm(x, (x.shape[-1],), eps=1e-6) + shift)


def set_fused_modulation(model: nn.Module, on: bool) -> None:
    """Route every adaLN-modulated Linear input through modulated(..., fused=on)."""
    for m in model.modules():
        if hasattr(m, "fused_modulation"):
            m.fused_modulation = on


def set_fused_gelu(model: nn.Module, on: bool) -> None:
    """With `on`, every MLP-down Linear takes its input through ConvRotLinear.forward_gelu: the
    tanh GELU (and, in the single blocks, the concatenation with the attention output, read
    from linear1's output in place) runs inside the activation preparation."""
    for m in model.modules():
        if hasattr(m, "fused_gelu"):
            m.fused_gelu = on


def set_fused_residual(model: nn.Module, on: bool) -> None:
    """With `on`, every gated residual `x + gate * linear(...)` that closes a block branch runs
    in the ConvRotLinear's GEMM epilogue (residual=, gate=) instead of two torch ops."""
    for m in model.modules():
        if hasattr(m, "fused_residual"):
            m.fused_residual = on


def project(linear: nn.Module, x: torch.Tensor, *, gelu: bool = False, head: torch.Tensor | None = None,
            residual: torch.Tensor | None = None, gate: torch.Tensor | None = None,
            fused_gelu: bool = False, fused_residual: bool = False) -> torch.Tensor:
    """residual + gate * linear(input) (or linear(input) without a residual), where input is
    x, gelu_tanh(x) (`gelu`) or cat([head, gelu_tanh(x)]).  The GELU / concatenation and the
    gated residual move into a ConvRotLinear's preparation and epilogue when their flags are
    set; otherwise they are the torch ops FLUX uses."""
    convrot = hasattr(linear, "forward_gelu")
    kw = dict(residual=residual, gate=gate) if fused_residual and convrot and residual is not None else {}
    if gelu and fused_gelu and convrot:
        out = linear.forward_gelu(x, head=head, **kw)
    else:
        if gelu:
            x = F.gelu(x, approximate="tanh")
        if head is not None:
            x = torch.cat([head, x], dim=-1)
        out = linear(x, **kw)
    if residual is None or kw:
        return out
    return residual + gate * out


def _split_heads(qkv: torch.Tensor, heads: int):
    b, l, _ = qkv.shape
    q, k, v = qkv.reshape(b, l, 3, heads, -1).permute(2, 0, 3, 1, 4).unbind(0)
    return q, k, v


class DoubleStreamBlock(nn.Module):
    def __init__(self, hidden: int, heads: int, mlp_ratio: float, qkv_bias: bool):
        super().__init__()
        mlp_hidden = int(hidden * mlp_ratio)
        self.heads = heads
        self.fused_modulation = self.fused_gelu = self.fused_residual = False
        for side in ("img", "txt"):
            setattr(self, f"{side}_mod", Modulation(hidden, double=True))
            setattr(self, f"{side}_qkv", nn.Linear(hidden, 3 * hidden, bias=qkv_bias))
            setattr(self, f"{side}_qknorm", QKNorm(hidden // heads))
            setattr(self, f"{side}_proj", nn.Linear(hidden, hidden))
            setattr(self, f"{side}_mlp", nn.Sequential(nn.Linear(hidden, mlp_hidden), nn.GELU(approximate="tanh"),
                                                       nn.Linear(mlp_hidden, hidden)))

    def forward(self, img, txt, vec, pe):
        (i_shift1, i_scale1, i_gate1), (i_shift2, i_scale2, i_gate2) = self.img_mod(vec)
        (t_shift1, t_scale1, t_gate1), (t_shift2, t_scale2, t_gate2) = self.txt_mod(vec)
        fu = self.fused_modulation
        iq, ik, iv = _split_heads(modulated(self.img_qkv, img, i_shift1, i_scale1, fu), self.heads)
        tq, tk, tv = _split_heads(modulated(self.txt_qkv, txt, t_shift1, t_scale1, fu), self.heads)
        iq, ik = self.img_qknorm(iq, ik)
        tq, tk = self.txt_qknorm(tq, tk)
        attn = attention(torch.cat([tq, iq], 2), torch.cat([tk, ik], 2), torch.cat([tv, iv], 2), pe)
        t_attn, i_attn = attn[:, : txt.shape[1]], attn[:, txt.shape[1]:]
        flags = dict(fused_gelu=self.fused_gelu, fused_residual=self.fused_residual)
        # img_mlp[1] / txt_mlp[1] are nn.GELU(approximate="tanh"): project applies it (gelu=True)
        img = project(self.img_proj, i_attn, residual=img, gate=i_gate1, **flags)
        img = project(self.img_mlp[2], modulated(self.img_mlp[0], img, i_shift2, i_scale2, fu), gelu=True,
                      residual=img, gate=i_gate2, **flags)
        txt = project(self.txt_proj, t_attn, residual=txt, gate=t_gate1, **flags)
        txt = project(self.txt_mlp[2], modulated(self.txt_mlp[0], txt, t_shift2, t_scale2, fu), gelu=True,
                      residual=txt, gate=t_gate2, **flags)
        return img, txt


class SingleStreamBlock(nn.Module):
    def __init__(self, hidden: int, heads: int, mlp_ratio: float):
        super().__init__()
        self.hidden, self.heads = hidden, heads
        self.mlp_hidden = int(hidden * mlp_ratio)
        self.linear1 = nn.Linear(hidden, 3 * hidden + self.mlp_hidden)
        self.linear2 = nn.Linear(hidden + self.mlp_hidden, hidden)
        self.norm = QKNorm(hidden // heads)
        self.modulation = Modulation(hidden, double=False)
        self.fused_modulation = self.fused_gelu = self.fused_residual = False

    def forward(self, x, vec, pe):
        (shift, scale, gate), _ = self.modulation(vec)
        h = modulated(self.linear1, x, shift, scale, self.fused_modulation)
        qkv, mlp = torch.split(h, [3 * self.hidden, self.mlp_hidden], dim=-1)
        q, k, v = _split_heads(qkv, self.heads)
        q, k = self.norm(q, k)
        attn = attention(q, k, v, pe)
        return project(self.linear2, mlp, gelu=True, head=attn, residual=x, gate=gate,
                       fused_gelu=self.fused_gelu, fused_residual=self.fused_residual)


class Flux(nn.Module):
    def __init__(self, p: FluxParams):
        super().__init__()
        self.p = p
        h = p.hidden_size
        self.pe_embedder = EmbedND(p.theta, p.axes_dim)
        self.img_in = nn.Linear(p.in_channels, h)
        self.time_in = MLPEmbedder(256, h)
        self.vector_in = MLPEmbedder(p.vec_in_dim, h)
        self.guidance_in = MLPEmbedder(256, h) if p.guidance_embed else None
        self.txt_in = nn.Linear(p.context_in_dim, h)
        self.double_blocks = nn.ModuleList(
            [DoubleStreamBlock(h, p.num_heads, p.mlp_ratio, p.qkv_bias) for _ in range(p.depth)])
        self.single_blocks = nn.ModuleList(
            [SingleStreamBlock(h, p.num_heads, p.mlp_ratio) for _ in range(p.depth_single_blocks)])
        self.final_adaln = nn.Linear(h, 2 * h)
        self.final_linear = nn.Linear(h, p.in_channels)
        self.fused_modulation = False

    def forward(self, img, img_ids, txt, txt_ids, timesteps, y, guidance=None):
        img = self.img_in(img)
        vec = self.time_in(timestep_embedding(timesteps, 256).to(img.dtype))
        if self.guidance_in is not None:
            vec = vec + self.guidance_in(timestep_embedding(guidance, 256).to(img.dtype))
        vec = vec + self.vector_in(y)
        txt = self.txt_in(txt)
        pe = self.pe_embedder(torch.cat([txt_ids, img_ids], dim=1))
        for block in self.double_blocks:
            img, txt = block(img, txt, vec, pe)
        x = torch.cat([txt, img], dim=1)
        for block in self.single_blocks:
            x = block(x, vec, pe)
        img = x[:, txt.shape[1]:]
        shift, scale = self.final_adaln(F.silu(vec))[:, None, :].chunk(2, dim=-1)
        return modulated(self.final_linear, img, shift, scale, self.fused_modulation)


def make_inputs(p: FluxParams, img_tokens: int, txt_tokens: int, device, seed: int = 5):
    """Latent tokens ~N(0,1) on a square patch grid, text embeddings ~N(0,1), pooled vector
    ~N(0,1), timestep 0.5, guidance 3.5 (batch 1)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    side = int(math.isqrt(img_tokens))
    assert side * side == img_tokens, "image tokens must form a square grid"
    img_ids = torch.zeros((side, side, 3), device=device)
    img_ids[..., 1] = torch.arange(side, device=device)[:, None]
    img_ids[..., 2] = torch.arange(side, device=device)[None, :]
    return dict(
        img=torch.randn((1, img_tokens, p.in_channels), generator=g, device=device).to(torch.bfloat16),
        img_ids=img_ids.reshape(1, img_tokens, 3),
        txt=torch.randn((1, txt_tokens, p.context_in_dim), generator=g, device=device).to(torch.bfloat16),
        txt_ids=torch.zeros((1, txt_tokens, 3), device=device),
        timesteps=torch.full((1,), 0.5, device=device),
        y=torch.randn((1, p.vec_in_dim), generator=g, device=device).to(torch.bfloat16),
        guidance=torch.full((1,), 3.5, device=device),
    )


def build(p: FluxParams, device, seed: int = 0) -> Flux:
    """torch's default Linear init, drawn directly in bf16 on `device` (no float32 copy of
    the 12B parameters)."""
    torch.manual_seed(seed)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(device):
            model = Flux(p)
    finally:
        torch.set_default_dtype(prev)
    return model.eval()


def _median_ms(fn, steps: int) -> float:
    times = []
    for _ in range(steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2] * 1e3


def time_step(model, inputs, steps: int) -> tuple[torch.Tensor, float, float]:
    """(eager output, eager ms, HIP-graph replay ms) of one forward, medians over `steps`.

    The graph is captured on the stream the warm-up ran on (so any per-stream workspace
    already exists) and every replay is checked bit-for-bit against the eager output."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.no_grad(), torch.cuda.stream(stream):
        for _ in range(2):
            out = model(**inputs)
        eager_ms = _median_ms(lambda: model(**inputs), steps)
        out = model(**inputs)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            static = model(**inputs)
        graph_ms = _median_ms(graph.replay, steps)
        torch.cuda.synchronize()
        if not torch.equal(static, out):
            raise RuntimeError("HIP-graph replay of the step differs from the eager step")
    torch.cuda.current_stream().wait_stream(stream)
    del graph, static
    return out, eager_ms, graph_ms


def linear_weight_bytes(model: nn.Module) -> dict:
    """Device bytes the model's Linears hold: dense weights and biases, or a ConvRotLinear's
    qweight, scales and bias plus the derived forms it caches (the FP6 operand weight, and the
    CDNA4 repack of a K x packed-N qweight), and the weight count they serve."""
    from convrot_mlx_amd import ConvRotLinear

    stored = derived = weights = 0
    for m in model.modules():
        if isinstance(m, ConvRotLinear):
            weights += m.in_features * m.out_features
            stored += sum(t.numel() * t.element_size() for t in (m.qweight, m.scales, m.bias))
            for cache in (m._fp6_cache, m._cdna4_cache):
                if cache is not None:
                    derived += cache[1].numel() * cache[1].element_size()
        elif isinstance(m, nn.Linear):
            weights += m.weight.numel()
            stored += sum(t.numel() * t.element_size() for t in (m.weight, m.bias) if t is not None)
    return {"weights": weights, "stored_bytes": stored, "derived_bytes": derived,
            "bytes_per_weight": round((stored + derived) / max(1, weights), 4)}


def allocated_baseline() -> int:
    """Bytes torch's allocator holds on the device now (what the process held before a model)."""
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return torch.cuda.memory_allocated()


def step_peak_memory(model: nn.Module, inputs: dict, base: int = 0) -> dict:
    """Device memory around one eager step (torch's allocator): resident before it and the peak
    during it, in GiB, net of `base` bytes held by the process before the model was built."""
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats()
    resident = torch.cuda.memory_allocated()
    with torch.no_grad():
        model(**inputs)
    torch.cuda.synchronize()
    gib = float(1 << 30)
    return {"resident_GiB": round((resident - base) / gib, 3),
            "step_peak_GiB": round((torch.cuda.max_memory_allocated() - base) / gib, 3)}


def config5_figure(p: FluxParams | None = None, img_tokens: int = 1024, txt_tokens: int = 512,
                   group_size: int = 64, steps: int = 5) -> dict:
    """One denoising step, dense bf16 vs every eligible Linear as W4A4 ConvRotLinear."""
    from convrot_mlx_amd import replace_convrot_linears

    p = p or FluxParams()
    dev = torch.device("cuda:0")
    base = allocated_baseline()
    model = build(p, dev)
    inputs = make_inputs(p, img_tokens, txt_tokens, dev)
    dense_weights = linear_weight_bytes(model)
    dense_memory = step_peak_memory(model, inputs, base)
    dense, dense_ms, dense_graph_ms = time_step(model, inputs, steps)
    dense = dense.float()
    linears = sum(1 for m in model.modules() if isinstance(m, nn.Linear))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    names = replace_convrot_linears(model, backend="hip-w4a4", group_size=group_size)
    torch.cuda.synchronize()
    convert_s = time.perf_counter() - t0
    torch.cuda.empty_cache()
    quant, quant_ms, quant_graph_ms = time_step(model, inputs, steps)
    quant = quant.float()
    set_fused_modulation(model, True)
    fused, fused_ms, fused_graph_ms = time_step(model, inputs, steps)
    fused = fused.float()
    set_fused_gelu(model, True)
    both, both_ms, both_graph_ms = time_step(model, inputs, steps)
    both = both.float()
    set_fused_residual(model, True)
    allf, all_ms, all_graph_ms = time_step(model, inputs, steps)
    allf = allf.float()
    convrot_weights = linear_weight_bytes(model)
    convrot_memory = step_peak_memory(model, inputs, base)
    # The same fused model with the 0.75-byte FP6 operand blocks cached instead of the compact
    # 0.5-byte form (the automatic choice), then on INT8 operands only (no FP6 weight form
    # cached): the same output bits, other weight memory.
    from convrot_mlx_amd import ConvRotLinear, set_fp6_operands, set_fp6_weight_form

    set_fp6_weight_form("full")
    try:
        full, full_ms, full_graph_ms = time_step(model, inputs, steps)
        full_weights = linear_weight_bytes(model)
        full_memory = step_peak_memory(model, inputs, base)
    finally:
        set_fp6_weight_form("auto")
    set_fp6_operands(False)
    try:
        for m in model.modules():
            if isinstance(m, ConvRotLinear):
                m._fp6_cache = None
        torch.cuda.empty_cache()
        int8, int8_ms, int8_graph_ms = time_step(model, inputs, steps)
        int8_weights = linear_weight_bytes(model)
        int8_memory = step_peak_memory(model, inputs, base)
    finally:
        set_fp6_operands(True)

    def dev_stats(out):
        diff = out - dense
        return (round((diff.norm() / dense.norm()).item(), 4),
                round(F.cosine_similarity(out.flatten(), dense.flatten(), dim=0).item(), 5),
                round(diff.abs().max().item(), 4))

    rel, cos, mad = dev_stats(quant)
    frel, fcos, _ = dev_stats(fused)
    brel, bcos, _ = dev_stats(both)
    arel, acos, _ = dev_stats(allf)
    return {
        "what": "random-init FLUX.1-dev DiT, one denoising step, batch 1, "
                f"{img_tokens} image + {txt_tokens} text tokens, bf16",
        "linears": linears, "converted": len(names), "group_size": group_size,
        "dense_bf16_ms": round(dense_ms, 2), "convrot_w4a4_ms": round(quant_ms, 2),
        "speedup": round(dense_ms / quant_ms, 3),
        "dense_bf16_graph_ms": round(dense_graph_ms, 2), "convrot_w4a4_graph_ms": round(quant_graph_ms, 2),
        "graph_speedup": round(dense_graph_ms / quant_graph_ms, 3), "convert_s": round(convert_s, 3),
        "rel_l2_vs_dense": rel, "cosine_vs_dense": cos, "max_abs_diff": mad,
        "fused_modulation": {
            "what": "adaLN LayerNorm + modulation fused into the ConvRot activation preparation (115 sites: 4 per double block, 1 per single block, the final layer)",
            "eager_ms": round(fused_ms, 2), "graph_ms": round(fused_graph_ms, 2),
            "graph_speedup_vs_dense": round(dense_graph_ms / fused_graph_ms, 3),
            "rel_l2_vs_dense": frel, "cosine_vs_dense": fcos,
            "rel_l2_vs_unfused": round(((fused - quant).norm() / quant.norm()).item(), 5),
        },
        "fused_modulation_and_gelu": {
            "what": "as fused_modulation, and every MLP-down Linear's tanh GELU (with the single blocks' "
                    "concatenation) fused into its activation preparation (76 sites)",
            "eager_ms": round(both_ms, 2), "graph_ms": round(both_graph_ms, 2),
            "graph_speedup_vs_dense": round(dense_graph_ms / both_graph_ms, 3),
            "rel_l2_vs_dense": brel, "cosine_vs_dense": bcos,
            "rel_l2_vs_fused_modulation": round(((both - fused).norm() / fused.norm()).item(), 5),
        },
        "fused_producers_and_residual": {
            "what": "as fused_modulation_and_gelu, and every gated residual x + gate * linear(...) in the "
                    "W4A4 GEMM epilogue (114 sites: 4 per double block, 1 per single block)",
            "eager_ms": round(all_ms, 2), "graph_ms": round(all_graph_ms, 2),
            "graph_speedup_vs_dense": round(dense_graph_ms / all_graph_ms, 3),
            "rel_l2_vs_dense": arel, "cosine_vs_dense": acos,
            "identical_to_fused_modulation_and_gelu": bool(torch.equal(allf, both)),
        },
        "memory": {
            "what": "torch allocator bytes on the device: the Linears' weights (dense bf16 weight + bias, or "
                    "ConvRotLinear qweight + scales + bias as stored, plus the derived FP6 operand weights "
                    "cached for products of 256+ rows), and the resident / peak bytes of one eager step of "
                    "the whole model (dense, and W4A4 with every fusion on), net of what the process held "
                    "before the model was built",
            "dense_linears": dense_weights, "w4a4_linears": convrot_weights,
            "dense_step": dense_memory, "w4a4_step": convrot_memory,
            "step_peak_reduction_pct": round(100.0 * (1.0 - convrot_memory["step_peak_GiB"] /
                                                      dense_memory["step_peak_GiB"]), 1),
            "reference": "M4 Pro, MLX allocator peak over a whole 20-step generation: 24.603 GiB dense vs "
                         "9.296 GiB ConvRot, 62.2 % less (docs/benchmarks/m4-pro.md:23-31)",
            "full_fp6_weights": {
                "what": "the fused model with set_fp6_weight_form('full'): every FP6 layer caches the "
                        "0.75-byte FP6 operand blocks instead of the 0.5-byte compact form",
                "linears": full_weights, "step": full_memory, "graph_ms": round(full_graph_ms, 2),
                "graph_speedup_vs_dense": round(dense_graph_ms / full_graph_ms, 3),
                "identical_output": bool(torch.equal(full.float(), allf)),
            },
            "int8_operands_only": {
                "what": "the fused model with set_fp6_operands(False): every product on the INT8 kernels, "
                        "no FP6 weight form cached (int4 qweight only)",
                "linears": int8_weights, "step": int8_memory, "graph_ms": round(int8_graph_ms, 2),
                "graph_speedup_vs_dense": round(dense_graph_ms / int8_graph_ms, 3),
                "identical_output": bool(torch.equal(int8.float(), allf)),
            },
        },
    }


def profile_variant(variant: str, steps: int, group_size: int = 64) -> dict:
    """Eager steps of one variant only (for a kernel trace whose statistics cover one model)."""
    from convrot_mlx_amd import replace_convrot_linears

    p = FluxParams()
    dev = torch.device("cuda:0")
    model = build(p, dev)
    inputs = make_inputs(p, 1024, 512, dev)
    if variant in ("convrot", "fused", "fused_gelu", "fused_all"):
        replace_convrot_linears(model, backend="hip-w4a4", group_size=group_size)
        set_fused_modulation(model, variant in ("fused", "fused_gelu", "fused_all"))
        set_fused_gelu(model, variant in ("fused_gelu", "fused_all"))
        set_fused_residual(model, variant == "fused_all")
    with torch.no_grad():
        model(**inputs)
        torch.cuda.synchronize()
        torch.cuda._sleep(1000)  # a marker kernel: the timed steps are the dispatches after it
        ms = _median_ms(lambda: model(**inputs), steps)
    return {"variant": variant, "timed_steps": steps, "eager_ms": round(ms, 2)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--group-size", type=int, default=64)
    ap.add_argument("--variant", choices=["both", "dense", "convrot", "fused", "fused_gelu", "fused_all"],
                    default="both",
                    help="'dense', 'convrot', 'fused' (convrot with fused modulation), 'fused_gelu' (and the "
                         "MLP GELUs fused too) or 'fused_all' (and the gated residuals in the GEMM epilogue) "
                         "runs eager steps of that model only, for profiling")
    args = ap.parse_args()
    if args.variant == "both":
        print(json.dumps(config5_figure(group_size=args.group_size, steps=args.steps)), flush=True)
    else:
        print(json.dumps(profile_variant(args.variant, args.steps, args.group_size)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
