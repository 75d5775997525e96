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

``weight_buf`` may be float32 (the reference layout), float16, bfloat16,
float8_e4m3fn (codes plus fp32 row scales) or float4_e2m1fn_x2 (MXFP4: two
E2M1 codes per byte plus an E8M0 scale per 32 elements), see
``weight_layout``; ``x`` may be float32 or float16 and the output has x's
dtype.  Work runs on the current
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
WEIGHT_DTYPES = (torch.float32, torch.float16, torch.bfloat16, torch.float8_e4m3fn,
                 torch.float4_e2m1fn_x2)
MX_BLOCK = 32     # MXFP4 elements per E8M0 scale
E2M1_GRID = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)  # magnitudes of codes 0..7


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
    if dtype == torch.float4_e2m1fn_x2:
        if hidden_dim % MX_BLOCK or intermediate_dim % MX_BLOCK:
            raise ValueError(f"MXFP4 weights need hidden_dim and intermediate_dim to be multiples "
                             f"of {MX_BLOCK}, got {hidden_dim}, {intermediate_dim}")
        n = intermediate_dim * hidden_dim
        sc = (3 * n // 2 + 15) // 16 * 16
        stride = (sc + 3 * n // MX_BLOCK + EXPERT_ALIGN - 1) // EXPERT_ALIGN * EXPERT_ALIGN
        return {"gate_proj_offset": 0, "up_proj_offset": n // 2, "down_proj_offset": n,
                "scale_offset": sc, "expert_stride": stride, "elem_bytes": 0}
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


def zeros_weights(n: int, dtype: torch.dtype, device) -> torch.Tensor:
    """A zeroed 1-D weight buffer of n elements (torch has no fill kernel for
    float4_e2m1fn_x2, so its bytes are zeroed as uint8)."""
    if dtype == torch.float4_e2m1fn_x2:
        return torch.zeros(n, dtype=torch.uint8, device=device).view(dtype)
    return torch.zeros(n, dtype=dtype, device=device)


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


def quantize_mxfp4(w: torch.Tensor):
    """(codes, scales) of a [rows, cols] matrix in OCP MXFP4 (cols a multiple
    of 32): per block of 32 elements of a row, the shared E8M0 exponent is
    floor(log2(max|block|)) - 2 (E2M1's largest exponent; 0 for an all-zero
    block) plus the bias 127, and each element is w / 2^(exponent) rounded to
    the nearest E2M1 value, ties to an even code, saturating at 6.
    Returns codes as uint8 [rows, cols / 2] (element 2i in the low nibble) and
    scales as uint8 [rows, cols / 32]."""
    rows, cols = w.shape
    if cols % MX_BLOCK:
        raise ValueError(f"MXFP4 rows need a multiple of {MX_BLOCK} elements, got {cols}")
    wf = w.to(torch.float32).reshape(rows, cols // MX_BLOCK, MX_BLOCK)
    amax = wf.abs().amax(dim=-1)
    _, ex = torch.frexp(amax)  # amax = m * 2^ex, m in [0.5, 1): floor(log2(amax)) = ex - 1
    e8 = torch.where(amax > 0, (ex.to(torch.int32) - 1 - 2 + 127).clamp(0, 254),
                     torch.zeros_like(ex, dtype=torch.int32))
    scale = torch.ldexp(torch.ones_like(amax), (e8 - 127).to(torch.float32))
    v = wf / scale.unsqueeze(-1)
    a = v.abs().clamp(max=6.0)
    grid = torch.tensor(E2M1_GRID, dtype=torch.float32, device=w.device)
    dist = (a.unsqueeze(-1) - grid).abs()
    code = dist.argmin(dim=-1)  # the lower code on a tie
    # a tie between an odd code and the next one goes to the even code
    nxt = (code + 1).clamp(max=7)
    tie = (code % 2 == 1) & (dist.gather(-1, nxt.unsqueeze(-1)).squeeze(-1) ==
                             dist.gather(-1, code.unsqueeze(-1)).squeeze(-1))
    code = torch.where(tie, nxt, code)
    code = code | ((v < 0).to(code.dtype) << 3)
    code = code.to(torch.uint8).reshape(rows, cols)
    packed = code[:, 0::2] | (code[:, 1::2] << 4)
    return packed.contiguous(), e8.to(torch.uint8).contiguous()


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
    es = torch.empty((), dtype=dtype).element_size()  # bytes per buffer element
    stride_el = off["expert_stride"] // es
    n = intermediate_dim * hidden_dim
    buf = zeros_weights(num_experts * stride_el, dtype, gate_proj[0].device)
    raw = buf.view(torch.uint8)
    if dtype == torch.float4_e2m1fn_x2:
        gs = n // MX_BLOCK  # scale bytes per matrix
        for e in range(num_experts):
            base = e * stride_el
            for j, m in enumerate((gate_proj[e], up_proj[e], down_proj[e])):
                q, sc = quantize_mxfp4(m)
                raw[base + j * n // 2:base + (j + 1) * n // 2] = q.reshape(-1)
                s0 = base + off["scale_offset"] + j * gs
                raw[s0:s0 + gs] = sc.reshape(-1)
        return buf
    if dtype != torch.float8_e4m3fn:
        for e in range(num_experts):
            base = e * stride_el
            buf[base:base + n] = gate_proj[e].reshape(-1)
            buf[base + n:base + 2 * n] = up_proj[e].reshape(-1)
            buf[base + 2 * n:base + 3 * n] = down_proj[e].reshape(-1)
        return buf
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


_CODE_BITS = {torch.float32: 32, torch.float16: 16, torch.bfloat16: 16,
              torch.float8_e4m3fn: 8, torch.float4_e2m1fn_x2: 4}


def shard_expert_weights(weight_buf: torch.Tensor, num_experts: int, hidden_dim: int,
                         intermediate_dim: int, num_shards: int, shard: int) -> torch.Tensor:
    """One GPU's share of a tensor-parallel split over the intermediate
    dimension: a packed buffer (same dtype, same device) of the layer with
    I' = I / num_shards, holding rows [s I', (s+1) I') of every expert's gate
    and up matrices and the same columns of its down matrix.

    The codes are copied, not requantized: fp8 gate/up row scales are sliced
    with their rows and the down row scales kept whole; MXFP4 block scales
    move with their 32-element blocks (I' must be a multiple of 32).  So the
    shard holds exactly the original weights, each shard routes as the whole
    layer does (the router is replicated), and the whole layer's output is
    the sum of the shards' outputs."""
    E, h, I, G = num_experts, hidden_dim, intermediate_dim, num_shards
    if G < 1 or I % G or not 0 <= shard < G:
        raise ValueError(f"cannot take shard {shard} of {G} from intermediate_dim {I}")
    dt = weight_buf.dtype
    Is = I // G
    full = weight_layout(E, h, I, dt)
    part = weight_layout(E, h, Is, dt)  # raises for MXFP4 when I' % 32 != 0
    bits = _CODE_BITS[dt]
    if weight_buf.numel() * weight_buf.element_size() < E * full["expert_stride"]:
        raise ValueError("weight_buf is smaller than the packed layer")

    def nb(n):  # bytes of n codes
        return n * bits // 8

    src = weight_buf.reshape(-1).view(torch.uint8)[:E * full["expert_stride"]]
    src = src.view(E, full["expert_stride"])
    buf = zeros_weights(E * part["expert_stride"] // weight_buf.element_size(), dt,
                        weight_buf.device)
    dst = buf.view(torch.uint8).view(E, part["expert_stride"])
    r0, r1 = shard * Is, (shard + 1) * Is

    def rows(s_off, d_off, row_bytes):  # rows r0:r1 of a row-major block
        dst[:, d_off:d_off + Is * row_bytes] = src[:, s_off + r0 * row_bytes:
                                                   s_off + r1 * row_bytes]

    def cols(s_off, d_off, n_rows, full_bytes, lo, hi):  # columns lo:hi (bytes) of every row
        d = dst[:, d_off:d_off + n_rows * (hi - lo)].view(E, n_rows, hi - lo)
        d.copy_(src[:, s_off:s_off + n_rows * full_bytes].view(E, n_rows, full_bytes)[:, :, lo:hi])

    rows(full["gate_proj_offset"], part["gate_proj_offset"], nb(h))
    rows(full["up_proj_offset"], part["up_proj_offset"], nb(h))
    cols(full["down_proj_offset"], part["down_proj_offset"], h, nb(I), nb(r0), nb(r1))
    if dt == torch.float8_e4m3fn:  # s_gate[I], s_up[I], s_down[h] (fp32)
        sf, sp = full["scale_offset"], part["scale_offset"]
        rows(sf, sp, 4)
        rows(sf + 4 * I, sp + 4 * Is, 4)
        dst[:, sp + 8 * Is:sp + 8 * Is + 4 * h] = src[:, sf + 8 * I:sf + 8 * I + 4 * h]
    elif dt == torch.float4_e2m1fn_x2:  # E8M0 bytes: gate [I][h/32], up [I][h/32], down [h][I/32]
        sf, sp = full["scale_offset"], part["scale_offset"]
        hb = h // MX_BLOCK
        rows(sf, sp, hb)
        rows(sf + I * hb, sp + Is * hb, hb)
        cols(sf + 2 * I * hb, sp + 2 * Is * hb, h, I // MX_BLOCK,
             r0 // MX_BLOCK, r1 // MX_BLOCK)
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


def set_handoff_check(enabled: bool) -> None:
    """Make ``fused_moe`` check its kernel's hand-off after every call.

    The single-token kernel hands act from its gate/up blocks to its down
    blocks through arrival counters, with a bounded wait (about 0.2 s).  A
    wait that expires makes that block write NaN rows and sets a status word
    and a host-visible word of the library.  Every ``fused_moe`` call reads
    the host-visible word after its launch, without a synchronisation, and
    raises ``RuntimeError`` if it is set: that reports the expiries of the
    calls whose kernels have run by then, so possibly one call late.  With
    the check on, ``fused_moe`` also reads this call's status word after the
    call (a stream synchronisation, so not under graph capture) and raises
    ``RuntimeError`` if it is set.  ``WARP_ROUTE_CHECK_HANDOFF=1`` in the
    environment turns it on at import.  The reference has no such wait: its
    fused kernel is a single warp (src/fused_moe.cu:76-227)."""
    _load_extension().set_handoff_check(bool(enabled))


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
