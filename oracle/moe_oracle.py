"""CPU oracle for the decode-time MoE layer.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or, for the
CPU baseline, as the thing timed on the host).  The product path
(``warp_route``, ``libwarp_route_hip.so``) never imports it and has no CPU
fallback.

It restates, in numpy, the arithmetic of anishesg/warp-route for this path.
Citations are ``file:line`` into that repository:

  layout_offsets / total_weight_bytes   src/expert_layout.cuh:34-47, 74-77
  expert_views                          src/expert_layout.cuh:50-71
  pack_expert_weights                   warp_route/functional.py:21-57
  router_logits                         src/fused_moe.cu:100-112, src/naive_moe.cu:49-72
  softmax_topk                          src/naive_moe.cu:152-175 (host softmax +
                                        iterative argmax with strict '>')
  expert_ffn                            tests/test_python.py:32-35,
                                        src/fused_moe.cu:192-224
  moe_forward                           tests/test_python.py:15-37,
                                        src/naive_moe.cu:181-241
  torch_moe_reference_cpu               tests/test_python.py:15-37 (fp32 torch,
                                        plus the renormalise flag)
  decode_bf16 / decode_e4m3 /           no reference counterpart (its weights are
  weight_layout / expert_matrices       fp32 only): the bf16 and OCP fp8 E4M3
                                        weight formats of include/warp_route.h
                                        (wr_dtype, wr_layout_info), decoded
                                        from their published bit layouts

Every function is pinned by tests in ``tests/test_oracle.py`` against checks
that do not retype its formula (the decoders: every bf16 and E4M3 code
against torch's own dtype conversions; the fp8 layout: hand-computed byte
tables): hand-computed byte tables and padding cases
for the layout, pack/unpack round trips, math.fsum exact sums for the
logits, scipy's softmax and brute-force sorting for the selection,
constructed exact ties, pure-Python loops on tiny shapes and the identity /
linearity / zero-input special cases for the FFN, and torch's library
routines (the reference's own test formula) for the whole layer.
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional, Sequence

import numpy as np

MAX_EXPERTS = 64   # src/gate.cuh:5
MAX_TOPK = 6       # src/gate.cuh:7
EXPERT_ALIGN = 128  # src/expert_layout.cuh:43-45

FLT_MAX = np.float32(np.finfo(np.float32).max)


# ----------------------------------------------------------------------------
# Layout (src/expert_layout.cuh, warp_route/functional.py:21-57)
# ----------------------------------------------------------------------------
def layout_offsets(num_experts: int, hidden_dim: int, intermediate_dim: int,
                   elem_bytes: int) -> Dict[str, int]:
    """Byte offsets inside one expert block (src/expert_layout.cuh:34-47).

    The reference fixes the element size at sizeof(float); here it is a
    parameter (4 for fp32, 2 for fp16) and the formula is otherwise the same.
    """
    gateup = intermediate_dim * hidden_dim
    down = hidden_dim * intermediate_dim
    up_off = gateup * elem_bytes
    down_off = up_off + gateup * elem_bytes
    raw = down_off + down * elem_bytes
    stride = (raw + EXPERT_ALIGN - 1) // EXPERT_ALIGN * EXPERT_ALIGN
    return {"gate_proj_offset": 0, "up_proj_offset": up_off,
            "down_proj_offset": down_off, "expert_stride": stride}


def total_weight_bytes(num_experts: int, hidden_dim: int, intermediate_dim: int,
                       elem_bytes: int) -> int:
    """src/expert_layout.cuh:74-77."""
    return num_experts * layout_offsets(num_experts, hidden_dim, intermediate_dim,
                                        elem_bytes)["expert_stride"]


def pack_expert_weights(gate_proj: Sequence[np.ndarray], up_proj: Sequence[np.ndarray],
                        down_proj: Sequence[np.ndarray], num_experts: int,
                        hidden_dim: int, intermediate_dim: int,
                        dtype=np.float32) -> np.ndarray:
    """Flat zero-padded packed buffer (warp_route/functional.py:21-57).

    Returns a 1-D array of ``dtype`` holding ``num_experts * stride / itemsize``
    elements.  The expert stride is a multiple of 128 bytes, hence of the item
    size, so every block starts on an element boundary.
    """
    dt = np.dtype(dtype)
    off = layout_offsets(num_experts, hidden_dim, intermediate_dim, dt.itemsize)
    stride_el = off["expert_stride"] // dt.itemsize
    n = intermediate_dim * hidden_dim
    buf = np.zeros(num_experts * stride_el, dtype=dt)
    for e in range(num_experts):
        base = e * stride_el
        buf[base:base + n] = np.asarray(gate_proj[e], dtype=dt).reshape(-1)
        buf[base + n:base + 2 * n] = np.asarray(up_proj[e], dtype=dt).reshape(-1)
        buf[base + 2 * n:base + 3 * n] = np.asarray(down_proj[e], dtype=dt).reshape(-1)
    return buf


def expert_views(buf: np.ndarray, e: int, num_experts: int, hidden_dim: int,
                 intermediate_dim: int):
    """(gate [I,h], up [I,h], down [h,I]) views of expert e in a packed buffer
    (gate_proj_ptr / up_proj_ptr / down_proj_ptr, src/expert_layout.cuh:50-71)."""
    es = buf.dtype.itemsize
    off = layout_offsets(num_experts, hidden_dim, intermediate_dim, es)
    base = e * off["expert_stride"] // es
    n = intermediate_dim * hidden_dim
    g = buf[base + off["gate_proj_offset"] // es:][:n].reshape(intermediate_dim, hidden_dim)
    u = buf[base + off["up_proj_offset"] // es:][:n].reshape(intermediate_dim, hidden_dim)
    d = buf[base + off["down_proj_offset"] // es:][:n].reshape(hidden_dim, intermediate_dim)
    return g, u, d


# ----------------------------------------------------------------------------
# Reduced-precision weight formats (no reference counterpart)
# ----------------------------------------------------------------------------
WEIGHT_FORMATS = ("f32", "f16", "bf16", "fp8", "mxfp4")
MX_BLOCK = 32


def decode_bf16(bits: np.ndarray) -> np.ndarray:
    """bfloat16 bit patterns (uint16) -> float64: the 16 bits are the high
    half of an IEEE binary32."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)
    with np.errstate(invalid="ignore"):  # signalling NaN patterns stay NaN
        return b.view(np.float32).astype(np.float64)


def decode_e4m3(codes: np.ndarray) -> np.ndarray:
    """OCP 8-bit float E4M3 codes (uint8) -> float64.  Bits s.eeee.mmm,
    exponent bias 7: e = 0 is subnormal, (-1)^s * m/8 * 2^-6; otherwise
    (-1)^s * (1 + m/8) * 2^(e-7); s.1111.111 is NaN; there are no infinities
    (the largest finite value, s.1111.110, is 448)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = (c & 0x7).astype(np.float64)
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    mag = np.where((e == 0xF) & (m == 7), np.nan, mag)
    return sign * mag


def decode_e2m1(codes: np.ndarray) -> np.ndarray:
    """OCP FP4 E2M1 codes (0..15) -> float64.  Bits s.ee.m, exponent bias 1:
    e = 0 is subnormal, (-1)^s * m/2; otherwise (-1)^s * (1 + m/2) * 2^(e-1).
    Magnitudes 0, 0.5, 1, 1.5, 2, 3, 4, 6; no infinities or NaN."""
    c = np.asarray(codes).astype(np.int64) & 0xF
    sign = np.where(c & 0x8, -1.0, 1.0)
    e = (c >> 1) & 0x3
    m = (c & 0x1).astype(np.float64)
    mag = np.where(e == 0, m / 2.0, (1.0 + m / 2.0) * np.exp2(e - 1.0))
    return sign * mag


def decode_e8m0(codes: np.ndarray) -> np.ndarray:
    """OCP E8M0 scale bytes -> float64 2^(e - 127); 255 is NaN."""
    e = np.asarray(codes, dtype=np.uint8).astype(np.float64)
    return np.where(e == 255, np.nan, np.exp2(e - 127.0))


def weight_layout(num_experts: int, hidden_dim: int, intermediate_dim: int,
                  fmt: str) -> Dict[str, int]:
    """Expert block layout per weight format (wr_layout_dtype).  f32, f16 and
    bf16: layout_offsets with 4, 2, 2 bytes per element and no scales.  fp8:
    1-byte codes at element offsets 0, I h, 2 I h; scales at 3 I h rounded up
    to 16 bytes (fp32 s_gate[I], s_up[I], s_down[h], one per output row);
    stride rounded up to 128 bytes."""
    if fmt not in WEIGHT_FORMATS:
        raise ValueError(f"unknown weight format {fmt!r}")
    if fmt == "mxfp4":
        # codes half a byte per element; then E8M0 bytes, one per 32 elements
        # of a row: gate [I][h/32], up [I][h/32], down [h][I/32]
        n = intermediate_dim * hidden_dim
        sc = (3 * n // 2 + 15) // 16 * 16
        stride = (sc + 3 * n // MX_BLOCK + EXPERT_ALIGN - 1) // EXPERT_ALIGN * EXPERT_ALIGN
        return {"gate_proj_offset": 0, "up_proj_offset": n // 2, "down_proj_offset": n,
                "scale_offset": sc, "expert_stride": stride, "elem_bytes": 0}
    if fmt != "fp8":
        es = {"f32": 4, "f16": 2, "bf16": 2}[fmt]
        out = layout_offsets(num_experts, hidden_dim, intermediate_dim, es)
        out.update(scale_offset=-1, elem_bytes=es)
        return out
    n = intermediate_dim * hidden_dim
    sc = (3 * n + 15) // 16 * 16
    stride = ((sc + 4 * (2 * intermediate_dim + hidden_dim) + EXPERT_ALIGN - 1)
              // EXPERT_ALIGN * EXPERT_ALIGN)
    return {"gate_proj_offset": 0, "up_proj_offset": n, "down_proj_offset": 2 * n,
            "scale_offset": sc, "expert_stride": stride, "elem_bytes": 1}


def expert_matrices(raw: np.ndarray, e: int, num_experts: int, hidden_dim: int,
                    intermediate_dim: int, fmt: str):
    """(gate [I,h], up [I,h], down [h,I]) of expert e as float64, decoded from
    the raw bytes (uint8) of a packed buffer in weight format ``fmt``.  fp8
    matrices are dequantized: every row times its row scale."""
    raw = np.asarray(raw, dtype=np.uint8)
    lo = weight_layout(num_experts, hidden_dim, intermediate_dim, fmt)
    h, I = hidden_dim, intermediate_dim
    n = I * h
    base = e * lo["expert_stride"]
    es = lo["elem_bytes"]

    if fmt == "mxfp4":
        def mxmat(j, off, rows, cols):
            b = raw[base + off:base + off + n // 2]
            codes = np.empty(n, dtype=np.uint8)
            codes[0::2] = b & 0xF
            codes[1::2] = b >> 4
            s0 = base + lo["scale_offset"] + j * (n // MX_BLOCK)
            sc = decode_e8m0(raw[s0:s0 + n // MX_BLOCK]).reshape(rows, cols // MX_BLOCK)
            return decode_e2m1(codes).reshape(rows, cols) * np.repeat(sc, MX_BLOCK, axis=1)
        return (mxmat(0, lo["gate_proj_offset"], I, h), mxmat(1, lo["up_proj_offset"], I, h),
                mxmat(2, lo["down_proj_offset"], h, I))

    def mat(off, rows, cols):
        b = raw[base + off:base + off + n * es]
        if fmt == "f32":
            v = b.view(np.float32).astype(np.float64)
        elif fmt == "f16":
            v = b.view(np.float16).astype(np.float64)
        elif fmt == "bf16":
            v = decode_bf16(b.view(np.uint16))
        else:
            v = decode_e4m3(b)
        return v.reshape(rows, cols)

    g = mat(lo["gate_proj_offset"], I, h)
    u = mat(lo["up_proj_offset"], I, h)
    d = mat(lo["down_proj_offset"], h, I)
    if fmt == "fp8":
        ns = 2 * I + h
        sc = raw[base + lo["scale_offset"]:base + lo["scale_offset"] + 4 * ns]
        s = sc.view(np.float32).astype(np.float64)
        g = g * s[:I][:, None]
        u = u * s[I:2 * I][:, None]
        d = d * s[2 * I:][:, None]
    return g, u, d


# ----------------------------------------------------------------------------
# Gating (src/fused_moe.cu:100-150, src/naive_moe.cu:49-72, 152-175)
# ----------------------------------------------------------------------------
def router_logits(gate_w: np.ndarray, x: np.ndarray) -> np.ndarray:
    """fp64 logits[e] = sum_i gate_w[e,i] x[i] (src/fused_moe.cu:100-112)."""
    return np.asarray(gate_w, dtype=np.float64) @ np.asarray(x, dtype=np.float64)


def logit_error_bound(gate_w: np.ndarray, x: np.ndarray) -> np.ndarray:
    """Bound on |fp32 dot - exact dot| for any summation order:
    gamma_n * sum_i |w_i x_i| with gamma_n = n u / (1 - n u), u = 2^-24,
    plus the final rounding to fp32."""
    w = np.abs(np.asarray(gate_w, dtype=np.float64))
    a = np.abs(np.asarray(x, dtype=np.float64))
    n = w.shape[1]
    u = 2.0 ** -24
    gamma = n * u / (1.0 - n * u)
    s = w @ a
    return gamma * s + u * s


def softmax_topk(logits, top_k: int, renormalize: bool = False):
    """fp32 softmax over all experts, then top-k by iterative argmax.

    Follows cpu_softmax_topk (src/naive_moe.cu:152-175): subtract the max, exp,
    sequential fp32 sum, divide; then ``top_k`` rounds picking the first unused
    expert whose probability is strictly greater than the best so far
    (initialised to -FLT_MAX), so ties go to the lower index and an expert
    whose probability is NaN is never picked.  With ``renormalize`` the
    selected weights are divided by their fp32 sum (Mixtral / DBRX routing);
    the reference never renormalises.

    Returns (probs fp32 [E], ids int32 [k], weights fp32 [k]).
    """
    l = np.asarray(logits, dtype=np.float32)
    E = l.shape[0]
    vmax = -FLT_MAX
    for e in range(E):
        vmax = np.float32(max(vmax, l[e]))
    probs = np.empty(E, dtype=np.float32)
    s = np.float32(0.0)
    with np.errstate(over="ignore", invalid="ignore"):
        for e in range(E):
            probs[e] = np.float32(np.exp(np.float32(l[e] - vmax)))
            s = np.float32(s + probs[e])
        for e in range(E):
            probs[e] = np.float32(probs[e] / s)
    used = [False] * E
    ids = np.zeros(top_k, dtype=np.int32)
    ws = np.zeros(top_k, dtype=np.float32)
    for kk in range(top_k):
        best, bval = 0, -FLT_MAX
        for e in range(E):
            if not used[e] and probs[e] > bval:
                bval, best = probs[e], e
        ids[kk], ws[kk] = best, bval
        used[best] = True
    if renormalize:
        tot = np.float32(0.0)
        for kk in range(top_k):
            tot = np.float32(tot + ws[kk])
        ws = (ws / tot).astype(np.float32)
    return probs, ids, ws


def topk_margin(logits64: np.ndarray, top_k: int) -> float:
    """Gap between the k-th and (k+1)-th largest fp64 logit (inf when k == E)."""
    s = np.sort(np.asarray(logits64, dtype=np.float64))[::-1]
    if top_k >= s.shape[0]:
        return math.inf
    return float(s[top_k - 1] - s[top_k])


def selection_is_robust(gate_w: np.ndarray, x: np.ndarray, top_k: int) -> bool:
    """True when the top-k set and order cannot depend on fp32 rounding: every
    adjacent gap among the k+1 largest logits exceeds twice the logit error
    bound plus a relative allowance for the fp32 exp and division."""
    l = router_logits(gate_w, x)
    bound = float(np.max(logit_error_bound(gate_w, x)))
    s = np.sort(l)[::-1]
    m = min(top_k + 1, s.shape[0])
    for i in range(m - 1):
        gap = s[i] - s[i + 1]
        if not gap > 2.0 * bound + 1e-5 * (1.0 + abs(s[i])):
            return False
    return True


# ----------------------------------------------------------------------------
# Expert FFN and the whole layer
# ----------------------------------------------------------------------------
def silu(v: np.ndarray) -> np.ndarray:
    """silu(g) = g / (1 + exp(-g)) (src/fused_moe.cu:30-32)."""
    with np.errstate(over="ignore"):
        return v / (1.0 + np.exp(-v))


def expert_ffn(x: np.ndarray, g: np.ndarray, u: np.ndarray, d: np.ndarray) -> np.ndarray:
    """fp64 Wd (silu(Wg x) * (Wu x)) (tests/test_python.py:32-35)."""
    x64 = np.asarray(x, dtype=np.float64)
    gv = np.asarray(g, dtype=np.float64) @ x64
    uv = np.asarray(u, dtype=np.float64) @ x64
    act = silu(gv) * uv
    return np.asarray(d, dtype=np.float64) @ act


def moe_forward(x: np.ndarray, gate_w: np.ndarray, buf: np.ndarray, num_experts: int,
                hidden_dim: int, intermediate_dim: int, top_k: int,
                renormalize: bool = False) -> Dict[str, np.ndarray]:
    """One token through the layer (tests/test_python.py:15-37 with the
    renormalise flag; selection semantics of src/naive_moe.cu:152-175).

    The selection runs on fp32 logits (the rounded fp64 dot products); the
    FFN and the weighted sum run in fp64 with the fp64 softmax weights of the
    selected experts.  Returns out (fp64 [h]), ids, weights (fp32),
    weights64, logits64, probs (fp32).
    """
    logits64 = router_logits(gate_w, x)
    probs, ids, ws = softmax_topk(logits64.astype(np.float32), top_k, renormalize)
    m = np.max(logits64)
    p64 = np.exp(logits64 - m)
    p64 /= p64.sum()
    w64 = p64[ids]
    if renormalize:
        w64 = w64 / w64.sum()
    out = np.zeros(hidden_dim, dtype=np.float64)
    for kk in range(top_k):
        g, u, d = expert_views(buf, int(ids[kk]), num_experts, hidden_dim, intermediate_dim)
        out += w64[kk] * expert_ffn(x, g, u, d)
    return {"out": out, "ids": ids, "weights": ws, "weights64": w64,
            "logits64": logits64, "probs": probs}


def moe_forward_batch(x: np.ndarray, gate_w: np.ndarray, buf: np.ndarray, num_experts: int,
                      hidden_dim: int, intermediate_dim: int, top_k: int,
                      renormalize: bool = False) -> Dict[str, np.ndarray]:
    """Row-wise moe_forward over a [B, h] batch (tests/test_batched.py:33-59:
    every token equals the single-token result)."""
    outs, ids, ws = [], [], []
    for b in range(x.shape[0]):
        r = moe_forward(x[b], gate_w, buf, num_experts, hidden_dim, intermediate_dim,
                        top_k, renormalize)
        outs.append(r["out"])
        ids.append(r["ids"])
        ws.append(r["weights"])
    return {"out": np.stack(outs) if outs else np.zeros((0, hidden_dim)),
            "ids": np.stack(ids) if ids else np.zeros((0, top_k), np.int32),
            "weights": np.stack(ws) if ws else np.zeros((0, top_k), np.float32)}


# ----------------------------------------------------------------------------
# CPU baseline (fp32 torch on the host): restates tests/test_python.py:15-37.
# ----------------------------------------------------------------------------
def torch_moe_reference_cpu(hidden, gate_w, gate_proj: List, up_proj: List, down_proj: List,
                            top_k: int, renormalize: bool = False):
    """The reference's pure-torch MoE (tests/test_python.py:15-37) in fp32 on
    the CPU, with the renormalise flag.  Used as the CPU baseline and as a
    library-routine cross-check of ``moe_forward``.  Expert tensors are fp32
    [I,h], [I,h], [h,I] CPU tensors."""
    import torch
    logits = gate_w @ hidden
    probs = torch.softmax(logits, dim=0)
    weights, indices = torch.topk(probs, top_k)
    if renormalize:
        weights = weights / weights.sum()
    out = torch.zeros_like(hidden)
    for kk in range(top_k):
        e = int(indices[kk])
        g = gate_proj[e] @ hidden
        u = up_proj[e] @ hidden
        act = g * torch.sigmoid(g) * u
        out += weights[kk] * (down_proj[e] @ act)
    return out, indices, weights


def relative_error(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / max(|ref|) (tests/test_correctness.cu:121-130)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = max(float(np.max(np.abs(ref))) if ref.size else 0.0, 1e-30)
    return float(np.max(np.abs(got - ref))) / denom if ref.size else 0.0


def cosine(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, dtype=np.float64).reshape(-1)
    b = np.asarray(b, dtype=np.float64).reshape(-1)
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    if na == 0.0 and nb == 0.0:
        return 1.0
    return float(a @ b / (na * nb))
