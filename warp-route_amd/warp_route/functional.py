"""Functional entry points of the MI355X MoE layer (drop-in for
warp_route/functional.py of anishesg/warp-route).

Names and the seven positional arguments of ``fused_moe``, ``naive_moe`` and
``batched_fused_moe`` are the reference's (warp_route/functional.py:60-153);
trailing keyword arguments add:

  renormalize   divide the selected top-k weights by their sum (Mixtral /
                DBRX routing).  Default False: the weights are the softmax
                probabilities, as in the reference.
  topk_ids      optional preallocated int32 tensor ([k], or [B, k] for the
                batched op) that receives the selected expert indices
  topk_weights  optional preallocated float32 tensor of the same shape that
                receives their gate weights

``weight_buf`` may be float32 (the reference layout), float16, bfloat16 or
float8_e4m3fn (codes plus fp32 scales, see ``weight_layout``); ``x`` may be
float32 or float16 and the output has x's dtype.  Work runs on the current
HIP stream without a device synchronisation.  There is no CPU fallback: the
ops raise if the HIP extension is missing.
"""
from __future__ import annotations

import functools
from typing import List, Optional, Tuple

import torch

MAX_EXPERTS = 64  # src/gate.cuh:5
MAX_TOPK = 6      # src/gate.cuh:7
EXPERT_ALIGN = 128
FP8_MAX = 448.0   # largest finite OCP E4M3 value
WEIGHT_DTYPES = (torch.float32, torch.float16, torch.bfloat16, torch.float8_e4m3fn)


@functools.lru_cache(maxsize=1)
def _load_extension():
    """Import the compiled ``warp_route._C`` (warp_route/functional.py:9-18)."""
    try:
        from . import _C
    except ImportError as e:  # pragma: no cover - exercised only on broken installs
        raise ImportError(
            "warp_route._C extension not found. Build it with: "
            "python warp-route_amd/build.py (requires ROCm hipcc and PyTorch-ROCm)"
        ) from e
    return _C


def expert_layout(num_experts: int, hidden_dim: int, intermediate_dim: int,
                  elem_bytes: int = 4) -> dict:
    """Byte offsets of one packed expert block and its 128-byte aligned stride
    (compute_offsets, src/expert_layout.cuh:34-47, with the element size as a
    parameter)."""
    gateup = intermediate_dim * hidden_dim
    up = gateup * elem_bytes
    down = up + gateup * elem_bytes
    raw = down + hidden_dim * intermediate_dim * elem_bytes
    stride = (raw + EXPERT_ALIGN - 1) // EXPERT_ALIGN * EXPERT_ALIGN
    return {"gate_proj_offset": 0, "up_proj_offset": up, "down_proj_offset": down,
            "expert_stride": stride}


def weight_layout(num_experts: int, hidden_dim: int, intermediate_dim: int,
                  dtype: torch.dtype) -> dict:
    """Byte layout of one expert block for a weight dtype (wr_layout_dtype).

    float32 / float16 / bfloat16: ``expert_layout`` with the element size, no
    scales.  float8_e4m3fn: 1-byte codes at the same element offsets, then at
    ``scale_offset`` (3 I h rounded up to 16 bytes) one fp32 scale per output
    row, s_gate[I], s_up[I] and s_down[h], so that gate[r][c] = q * s_gate[r],
    up[r][c] = q * s_up[r] and down[r][c] = q * s_down[r]; the stride covers
    them, rounded up to 128."""
    if dtype not in WEIGHT_DTYPES:
        raise ValueError(f"weight dtype must be one of {WEIGHT_DTYPES}, got {dtype}")
    es = torch.empty((), dtype=dtype).element_size()
    if dtype != torch.float8_e4m3fn:
        out = expert_layout(num_experts, hidden_dim, intermediate_dim, es)
        out.update(scale_offset=-1, elem_bytes=es)
        return out
    n = intermediate_dim * hidden_dim
    sc = (3 * n + 15) // 16 * 16
    stride = ((sc + 4 * (2 * intermediate_dim + hidden_dim) + EXPERT_ALIGN - 1)
              // EXPERT_ALIGN * EXPERT_ALIGN)
    return {"gate_proj_offset": 0, "up_proj_offset": n, "down_proj_offset": 2 * n,
            "scale_offset": sc, "expert_stride": stride, "elem_bytes": 1}


def quantize_fp8(w: torch.Tensor, dim: int):
    """(codes, scales) of ``w`` in OCP E4M3 with one fp32 scale per slice
    along ``dim`` (dim=1: per row, dim=0: per column):
    scale = max|w| / 448 over the slice (1 for an all-zero slice), codes =
    round-to-nearest-even of w / scale, within +-448 by construction."""
    wf = w.to(torch.float32)
    amax = wf.abs().amax(dim=dim, keepdim=True)
    scale = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    q = (wf / scale).clamp_(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q, scale.reshape(-1)


def _pack_expert_weights(
    gate_proj: List[torch.Tensor],
    up_proj: List[torch.Tensor],
    down_proj: List[torch.Tensor],
    num_experts: int,
    hidden_dim: int,
    intermediate_dim: int,
    dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Pack per-expert weights into the flat expert layout
    (warp_route/functional.py:21-57).

    Per expert, row-major: [gate_proj I x h][up_proj I x h][down_proj h x I],
    each expert block zero-padded to a 128-byte boundary.  ``dtype`` selects
    float32 (the reference's only layout, the default), float16, bfloat16, or
    float8_e4m3fn, which quantizes every matrix with ``quantize_fp8`` per row
    (output channel) and stores the scales after the codes
    (``weight_layout``).  The buffer is created on the device of
    ``gate_proj[0]``.
    """
    off = weight_layout(num_experts, hidden_dim, intermediate_dim, dtype)
    es = off["elem_bytes"]
    stride_el = off["expert_stride"] // es
    n = intermediate_dim * hidden_dim
    buf = torch.zeros(num_experts * stride_el, dtype=dtype, device=gate_proj[0].device)
    if dtype != torch.float8_e4m3fn:
        for e in range(num_experts):
            base = e * stride_el
            buf[base:base + n] = gate_proj[e].reshape(-1)
            buf[base + n:base + 2 * n] = up_proj[e].reshape(-1)
            buf[base + 2 * n:base + 3 * n] = down_proj[e].reshape(-1)
        return buf
    raw = buf.view(torch.uint8)
    ns = 2 * intermediate_dim + hidden_dim
    for e in range(num_experts):
        base = e * stride_el
        qg, sg = quantize_fp8(gate_proj[e], 1)
        qu, su = quantize_fp8(up_proj[e], 1)
        qd, sd = quantize_fp8(down_proj[e], 1)
        buf[base:base + n] = qg.reshape(-1)
        buf[base + n:base + 2 * n] = qu.reshape(-1)
        buf[base + 2 * n:base + 3 * n] = qd.reshape(-1)
        sc = base + off["scale_offset"]
        raw[sc:sc + 4 * ns].view(torch.float32).copy_(torch.cat([sg, su, sd]))
    return buf


def fused_moe(
    x: torch.Tensor,
    gate_w: torch.Tensor,
    weight_buf: torch.Tensor,
    num_experts: int,
    hidden_dim: int,
    intermediate_dim: int,
    top_k: int,
    renormalize: bool = False,
    topk_ids: Optional[torch.Tensor] = None,
    topk_weights: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Single-token fused MoE forward (warp_route/functional.py:60-87).

    Args:
        x: hidden state [hidden_dim], float32 or float16, on the GPU.
        gate_w: router [num_experts, hidden_dim], float32.
        weight_buf: packed expert weights from ``_pack_expert_weights``.
        top_k: experts per token, 1 <= top_k <= min(6, num_experts).

    Returns the output [hidden_dim] in x's dtype.
    """
    _C = _load_extension()
    return _C.fused_moe_forward(x, gate_w, weight_buf, num_experts, hidden_dim,
                                intermediate_dim, top_k, renormalize, topk_ids, topk_weights)


def naive_moe(
    x: torch.Tensor,
    gate_w: torch.Tensor,
    weight_buf: torch.Tensor,
    num_experts: int,
    hidden_dim: int,
    intermediate_dim: int,
    top_k: int,
    renormalize: bool = False,
    topk_ids: Optional[torch.Tensor] = None,
    topk_weights: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Single-token naive multi-kernel MoE forward with host-side top-K
    (warp_route/functional.py:90-117).  Synchronises the current stream once."""
    _C = _load_extension()
    return _C.naive_moe_forward(x, gate_w, weight_buf, num_experts, hidden_dim,
                                intermediate_dim, top_k, renormalize, topk_ids, topk_weights)


def batched_fused_moe(
    x: torch.Tensor,
    gate_w: torch.Tensor,
    weight_buf: torch.Tensor,
    num_experts: int,
    hidden_dim: int,
    intermediate_dim: int,
    top_k: int,
    renormalize: bool = False,
    topk_ids: Optional[torch.Tensor] = None,
    topk_weights: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Batched fused MoE forward for B decode tokens
    (warp_route/functional.py:120-153).

    Args:
        x: [batch_size, hidden_dim], float32 or float16.

    Returns [batch_size, hidden_dim] in x's dtype.
    """
    if x.dim() != 2:
        raise ValueError(f"batched_fused_moe expects 2D input [batch, hidden], got shape {x.shape}")
    _, hd = x.shape
    if hd != hidden_dim:
        raise ValueError(f"Input hidden dim {hd} does not match hidden_dim={hidden_dim}")
    _C = _load_extension()
    return _C.batched_fused_moe_forward(x, gate_w, weight_buf, num_experts, hidden_dim,
                                        intermediate_dim, top_k, renormalize, topk_ids,
                                        topk_weights)


def gate_topk(
    x: torch.Tensor,
    gate_w: torch.Tensor,
    num_experts: int,
    hidden_dim: int,
    top_k: int,
    renormalize: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Router logits, softmax and top-K on the GPU (warp_gate_topk,
    src/gate.cu:103-116).  x is [hidden_dim] or [B, hidden_dim]; returns
    (ids int32, weights float32) of shape [k] or [B, k], experts in descending
    weight order, ties to the lower index."""
    _C = _load_extension()
    return _C.gate_topk(x, gate_w, num_experts, hidden_dim, top_k, renormalize)
