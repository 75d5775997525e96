"""Seeded synthetic MoE layers for the benchmark configurations (there are no
checkpoints offline; every config is synthetic random-init).

Draw order, all in fp32 from one generator seeded with ``seed``:
x [B, h] ~ N(0, 1); router [E, h] ~ N(0, router_std); then for each expert e:
gate [I, h], up [I, h], down [h, I] ~ N(0, expert_std).  The expert matrices
are cast to ``weight_dtype`` straight into the packed expert layout
(src/expert_layout.cuh:5-18), so a full layer never exists in fp32; for
float8_e4m3fn each matrix is quantized with ``quantize_fp8`` (same draws, so
an fp8 layer is the quantized fp16 layer of the same seed).
"""
from __future__ import annotations

import dataclasses
import math
from dataclasses import dataclass
from typing import Optional

import torch

from .functional import MX_BLOCK, quantize_fp8, quantize_mxfp4, weight_layout, zeros_weights


@dataclass(frozen=True)
class MoEConfig:
    name: str
    num_experts: int
    hidden_dim: int
    intermediate_dim: int
    top_k: int
    weight_dtype: torch.dtype
    renormalize: bool
    router_std: float
    expert_std: float = 0.02

    @property
    def selected_bytes(self) -> int:
        """Weight bytes of k distinct experts: the algorithmic traffic of one
        batch-1 call (3 * h * I * elem_bytes per expert, plus 12 I bytes of
        scales for fp8)."""
        return self.top_k * expert_weight_bytes(self.hidden_dim, self.intermediate_dim,
                                                self.weight_dtype)

    def with_weights(self, dtype: torch.dtype) -> "MoEConfig":
        return dataclasses.replace(self, weight_dtype=dtype)


def expert_weight_bytes(hidden_dim: int, intermediate_dim: int, dtype: torch.dtype) -> int:
    """Bytes a kernel must read for one selected expert: its three matrices,
    and for fp8 and MXFP4 their scales."""
    n = 3 * hidden_dim * intermediate_dim
    if dtype == torch.float4_e2m1fn_x2:
        return n // 2 + n // MX_BLOCK
    es = torch.empty((), dtype=dtype).element_size()
    return n * es + (4 * (2 * intermediate_dim + hidden_dim) if dtype == torch.float8_e4m3fn
                     else 0)


CONFIGS = {
    # Toy: the CPU-runnable plumbing case (fp32, reference routing).
    "toy": MoEConfig("toy", 8, 256, 512, 2, torch.float32, False, 1.0 / 16.0),
    # Mixtral-8x7B layer: softmax-then-top2 with renormalised weights.
    "mixtral": MoEConfig("mixtral", 8, 4096, 14336, 2, torch.float16, True, 1.0 / 64.0),
    # DeepSeek-MoE layer: 64 small experts, top-6.
    "deepseek": MoEConfig("deepseek", 64, 2048, 1408, 6, torch.float16, False,
                          1.0 / math.sqrt(2048)),
    # DBRX layer: 16 experts, top-4, renormalised.
    "dbrx": MoEConfig("dbrx", 16, 6144, 10752, 4, torch.float16, True, 1.0 / math.sqrt(6144)),
}


def make_layer(num_experts: int, hidden_dim: int, intermediate_dim: int,
               weight_dtype: torch.dtype = torch.float32, router_std: float = 0.02,
               expert_std: float = 0.02, seed: int = 0, batch: Optional[int] = None,
               device="cpu", gen_device="cpu", x_dtype: torch.dtype = torch.float32):
    """Returns (x, gate_w, weight_buf) on ``device``.  x is [h] when ``batch``
    is None, else [batch, h].  Random numbers are drawn on ``gen_device``
    ("cpu" is reproducible across machines with the same torch build;
    "cuda" is fast for multi-GB layers)."""
    gen = torch.Generator(device=gen_device)
    gen.manual_seed(seed)
    shape_x = (hidden_dim,) if batch is None else (batch, hidden_dim)
    x = torch.randn(shape_x, generator=gen, device=gen_device, dtype=torch.float32)
    gate_w = torch.randn(num_experts, hidden_dim, generator=gen, device=gen_device,
                         dtype=torch.float32) * router_std
    off = weight_layout(num_experts, hidden_dim, intermediate_dim, weight_dtype)
    es = torch.empty((), dtype=weight_dtype).element_size()
    stride_el = off["expert_stride"] // es
    n = intermediate_dim * hidden_dim
    fp8 = weight_dtype == torch.float8_e4m3fn
    fp4 = weight_dtype == torch.float4_e2m1fn_x2
    buf = zeros_weights(num_experts * stride_el, weight_dtype, device)
    raw = buf.view(torch.uint8)
    I = intermediate_dim
    for e in range(num_experts):
        base = e * stride_el
        for j in range(3):
            shape = (intermediate_dim, hidden_dim) if j < 2 else (hidden_dim, intermediate_dim)
            w = torch.randn(shape, generator=gen, device=gen_device, dtype=torch.float32)
            w.mul_(expert_std)
            if fp4:
                q, sc = quantize_mxfp4(w)
                raw[base + j * n // 2:base + (j + 1) * n // 2].copy_(q.reshape(-1))
                s0 = base + off["scale_offset"] + j * (n // MX_BLOCK)
                raw[s0:s0 + n // MX_BLOCK].copy_(sc.reshape(-1))
                del q, sc
            elif fp8:
                # a scale per row: gate and up rows at j * I, down rows at 2 I
                q, sc = quantize_fp8(w, 1)
                buf[base + j * n:base + (j + 1) * n].copy_(q.reshape(-1))
                s0 = base + off["scale_offset"] + j * 4 * I
                raw[s0:s0 + 4 * sc.numel()].view(torch.float32).copy_(sc)
                del q, sc
            else:
                buf[base + j * n:base + (j + 1) * n].copy_(w.reshape(-1).to(weight_dtype))
            del w
    return (x.to(device=device, dtype=x_dtype), gate_w.to(device), buf)


def make_config_layer(cfg: MoEConfig, seed: int = 0, batch: Optional[int] = None,
                      device="cpu", gen_device="cpu", x_dtype: torch.dtype = torch.float32):
    return make_layer(cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.weight_dtype,
                      cfg.router_std, cfg.expert_std, seed, batch, device, gen_device, x_dtype)


def clustered_batch(gate_w: torch.Tensor, batch: int, pair=(0, 1), alpha: float = 4.0,
                    seed: int = 0, device="cpu") -> torch.Tensor:
    """[batch, h] tokens biased toward one expert pair: x_b = z_b + alpha *
    (R[a] + R[b]) / (||R[a]||^2 + ||R[b]||^2) * 2, z ~ N(0, 1).  With unit-norm
    router rows this adds about alpha to the logits of experts a and b, so
    tokens cluster on them (the batched-decode config's routing recipe)."""
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    h = gate_w.shape[1]
    z = torch.randn(batch, h, generator=gen, dtype=torch.float32)
    r = gate_w.detach().float().cpu()
    a, b = pair
    d = r[a] + r[b]
    scale = 2.0 * alpha / float((r[a] * r[a]).sum() + (r[b] * r[b]).sum())
    return (z + scale * d).to(device)
