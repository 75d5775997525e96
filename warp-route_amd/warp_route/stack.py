"""A stack of MoE layers driven one decode step at a time, eagerly or replayed
from one captured HIP graph.

This is the decode loop of the benchmark's 32-layer configuration.  The
reference has no such driver: its callers step through the layers from
Python, one op launch at a time (warp_route/__init__.py:71-105 per layer).
Here a whole step, every layer's router and FFN launches and the residual adds
between them, is captured once with ``torch.cuda.CUDAGraph`` (a hipGraph on
ROCm) and replayed with a single launch from the host.

The ops are capture-safe: they launch only kernels on the current stream,
allocate their workspace from torch's caching allocator (the graph's private
pool while capturing), record no memset nodes, and never synchronise.
"""
from __future__ import annotations

from typing import List, Sequence, Tuple

import torch

from .functional import batched_fused_moe, fused_moe

__all__ = ["MoEStack", "GraphedStack"]


class MoEStack:
    """Layers l = 0..L-1, each a (gate_w [E, h] fp32, packed expert buffer)
    pair of the same shape.  One step maps x ([h] for one token, [B, h] for a
    batch) to h_L with h_0 = x and h_{l+1} = h_l + moe_l(h_l) (residual=True)
    or h_{l+1} = moe_l(h_l)."""

    def __init__(self, layers: Sequence[Tuple[torch.Tensor, torch.Tensor]], num_experts: int,
                 hidden_dim: int, intermediate_dim: int, top_k: int,
                 renormalize: bool = False, residual: bool = True) -> None:
        if len(layers) == 0:
            raise ValueError("MoEStack needs at least one layer")
        for i, (gw, buf) in enumerate(layers):
            if gw.dim() != 2 or gw.shape[0] != num_experts or gw.shape[1] != hidden_dim:
                raise ValueError(f"layer {i}: gate_w must be [{num_experts}, {hidden_dim}], "
                                 f"got {tuple(gw.shape)}")
            if buf.device != gw.device:
                raise ValueError(f"layer {i}: gate_w and weight_buf on different devices")
        self.layers: List[Tuple[torch.Tensor, torch.Tensor]] = list(layers)
        self.num_experts = num_experts
        self.hidden_dim = hidden_dim
        self.intermediate_dim = intermediate_dim
        self.top_k = top_k
        self.renormalize = renormalize
        self.residual = residual

    def _moe(self, h: torch.Tensor, gw: torch.Tensor, buf: torch.Tensor) -> torch.Tensor:
        args = (gw, buf, self.num_experts, self.hidden_dim, self.intermediate_dim, self.top_k,
                self.renormalize)
        if h.dim() == 1:
            return fused_moe(h, *args)
        if h.dim() == 2:
            return batched_fused_moe(h, *args)
        raise ValueError(f"Input must be 1D or 2D, got shape {tuple(h.shape)}")

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """One decode step, launched op by op."""
        h = x.contiguous()
        for gw, buf in self.layers:
            y = self._moe(h, gw, buf)
            h = h + y if self.residual else y
        return h

    __call__ = forward

    def capture(self, example: torch.Tensor, warmup: int = 2) -> "GraphedStack":
        """Capture one step for inputs shaped and typed like ``example`` (on
        the layers' device) and return the replayable step."""
        return GraphedStack(self, example, warmup)


class GraphedStack:
    """One captured step of a MoEStack.  Calling it copies x into the static
    input, replays the graph on the current stream and returns the static
    output tensor, which the next call overwrites (clone it to keep it)."""

    def __init__(self, stack: MoEStack, example: torch.Tensor, warmup: int) -> None:
        dev = stack.layers[0][0].device
        if example.device != dev:
            raise ValueError(f"example is on {example.device}, the layers on {dev}")
        self.stack = stack
        self.static_in = example.detach().clone().contiguous()
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(warmup):  # allocator and kernel warm-up outside the capture
                stack.forward(self.static_in)
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.static_out = stack.forward(self.static_in)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape != self.static_in.shape or x.dtype != self.static_in.dtype:
            raise ValueError(f"captured for {tuple(self.static_in.shape)} {self.static_in.dtype}, "
                             f"got {tuple(x.shape)} {x.dtype}")
        self.static_in.copy_(x)
        self.graph.replay()
        return self.static_out
