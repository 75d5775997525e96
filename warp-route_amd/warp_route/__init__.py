"""warp_route: decode-time fused Mixture-of-Experts layer for AMD MI355X
(gfx950), a drop-in for the Python package of anishesg/warp-route.

``MoELayer`` mirrors warp_route/__init__.py:10-105 of the reference: a router
plus per-expert gate/up/down parameter lists, dispatched to the fused kernel
for a single token and to the batched kernel for [B, hidden] inputs.  Unlike
the reference, which repacks every expert on every forward
(warp_route/__init__.py:81), the packed buffer is cached and rebuilt only when
a parameter has changed in place or been replaced (its identity, storage
pointer or version counter differ).  Writes made through ``p.data`` bypass
the version counter; call ``MoELayer.invalidate_packed()`` after them, or
construct the layer with ``cache_packed=False`` to repack on every forward
as the reference does.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from .functional import (MAX_EXPERTS, MAX_TOPK, WEIGHT_DTYPES, _pack_expert_weights,
                         batched_fused_moe, expert_layout, fused_moe, gate_topk, naive_moe,
                         quantize_fp8, quantize_mxfp4, weight_layout)

__all__ = ["MoELayer", "fused_moe", "naive_moe", "batched_fused_moe", "gate_topk",
           "expert_layout", "weight_layout", "quantize_fp8", "quantize_mxfp4",
           "_pack_expert_weights"]


class MoELayer(nn.Module):
    """Single MoE layer with per-expert SwiGLU FFN blocks
    (warp_route/__init__.py:10-61).

    Args:
        num_experts: total experts (<= 64).
        hidden_dim: hidden state dimension.
        intermediate_dim: per-expert intermediate dimension.
        top_k: experts per token, 1 <= top_k <= min(6, num_experts).
        renormalize: divide the selected weights by their sum.
        weight_dtype: dtype of the packed expert buffer the kernels read
            (torch.float32 as in the reference, torch.float16, torch.bfloat16,
            torch.float8_e4m3fn with per-row fp32 scales, or
            torch.float4_e2m1fn_x2 for MXFP4).
        cache_packed: keep the packed buffer between forwards, rebuilding it
            when a parameter is replaced or changed in place through autograd-
            visible ops (which bump its version counter).  Writes through
            ``p.data`` are not seen: call ``invalidate_packed()`` after them.
            False repacks on every forward, as the reference does.
    """

    def __init__(self, num_experts: int, hidden_dim: int, intermediate_dim: int,
                 top_k: int = 2, renormalize: bool = False,
                 weight_dtype: torch.dtype = torch.float32, cache_packed: bool = True) -> None:
        super().__init__()
        if not 1 <= num_experts <= MAX_EXPERTS:
            raise ValueError(f"num_experts must be in [1, {MAX_EXPERTS}], got {num_experts}")
        if not 1 <= top_k <= min(MAX_TOPK, num_experts):
            raise ValueError(
                f"top_k must be in [1, min({MAX_TOPK}, num_experts)], got {top_k}")
        if weight_dtype not in WEIGHT_DTYPES:
            raise ValueError(f"weight_dtype must be one of {WEIGHT_DTYPES}, got {weight_dtype}")
        self.num_experts = num_experts
        self.hidden_dim = hidden_dim
        self.intermediate_dim = intermediate_dim
        self.top_k = top_k
        self.renormalize = renormalize
        self.weight_dtype = weight_dtype
        self.cache_packed = cache_packed
        self.router = nn.Parameter(torch.empty(num_experts, hidden_dim))
        self.gate_proj = nn.ParameterList(
            [nn.Parameter(torch.empty(intermediate_dim, hidden_dim)) for _ in range(num_experts)])
        self.up_proj = nn.ParameterList(
            [nn.Parameter(torch.empty(intermediate_dim, hidden_dim)) for _ in range(num_experts)])
        self.down_proj = nn.ParameterList(
            [nn.Parameter(torch.empty(hidden_dim, intermediate_dim)) for _ in range(num_experts)])
        self._packed: Optional[torch.Tensor] = None
        self._packed_key = None
        self._init_weights()

    def _init_weights(self) -> None:
        """std-0.02 normal init of every parameter (warp_route/__init__.py:56-61)."""
        nn.init.normal_(self.router, std=0.02)
        for e in range(self.num_experts):
            nn.init.normal_(self.gate_proj[e], std=0.02)
            nn.init.normal_(self.up_proj[e], std=0.02)
            nn.init.normal_(self.down_proj[e], std=0.02)

    def _params(self):
        return list(self.gate_proj) + list(self.up_proj) + list(self.down_proj)

    def _cache_key(self):
        return tuple((id(p), p.data_ptr(), p._version, p.device) for p in self._params()) + (
            self.weight_dtype,)

    def invalidate_packed(self) -> None:
        """Drop the cached packed buffer; the next forward repacks.  Needed
        after writes through ``p.data`` (e.g. ``p.data.copy_(w)``), which do
        not bump the version counter the cache is keyed on."""
        self._packed = None
        self._packed_key = None

    def _pack_weights(self) -> torch.Tensor:
        """Packed expert buffer in ``weight_dtype`` (warp_route/__init__.py:63-69),
        rebuilt when a parameter changed since the last pack, after
        ``invalidate_packed()``, and on every call with cache_packed=False."""
        key = self._cache_key()
        if not self.cache_packed or self._packed is None or key != self._packed_key:
            with torch.no_grad():
                self._packed = _pack_expert_weights(
                    [p.data for p in self.gate_proj], [p.data for p in self.up_proj],
                    [p.data for p in self.down_proj], self.num_experts, self.hidden_dim,
                    self.intermediate_dim, dtype=self.weight_dtype)
            self._packed_key = key
        return self._packed

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """[hidden_dim] -> fused kernel; [B, hidden_dim] -> batched kernel
        (warp_route/__init__.py:71-105).  Output has x's shape and dtype."""
        weight_buf = self._pack_weights()
        router_w = self.router.data.float().contiguous()
        if x.dim() == 1:
            return fused_moe(x.contiguous(), router_w, weight_buf, self.num_experts,
                             self.hidden_dim, self.intermediate_dim, self.top_k,
                             self.renormalize)
        if x.dim() == 2:
            return batched_fused_moe(x.contiguous(), router_w, weight_buf, self.num_experts,
                                     self.hidden_dim, self.intermediate_dim, self.top_k,
                                     self.renormalize)
        raise ValueError(f"Input must be 1D or 2D, got shape {x.shape}")
