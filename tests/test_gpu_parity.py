"""GPU parity: the HIP kernels (through warp_route._C and the C-ABI) against
the CPU oracle on the same seeded inputs.

Bar: selected expert ids bit-exact (fp32 gating, ties to
the lower index; every randomly drawn case must pass the oracle's margin
guard), gate weights within 1e-5, outputs within rtol = atol = 1e-2, and
within 1e-4 of max|ref| (max-abs error) where the output is fp32.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests._helpers import assert_parity, assert_same_up_to_order, f64, oracle_token

import warp_route
from warp_route import capi
from warp_route import functional as F
from warp_route.synthetic import CONFIGS, clustered_batch, make_config_layer, make_layer

pytestmark = pytest.mark.gpu

F32, F16 = torch.float32, torch.float16
BF16, FP8, MX4 = torch.bfloat16, torch.float8_e4m3fn, torch.float4_e2m1fn_x2
WNAME = {F32: "f32", F16: "f16", BF16: "bf16", FP8: "fp8", MX4: "mxfp4"}

# (E, h, I, k, weight dtype, renormalize)
SMALL = [
    (8, 256, 512, 1, F32, False),
    (8, 256, 512, 2, F32, False),
    (8, 512, 1024, 2, F16, True),
    (16, 256, 512, 2, F32, True),
    (8, 1024, 2048, 2, F16, False),
    (64, 256, 512, 6, F16, False),
    (16, 512, 256, 4, F32, True),
    (8, 256, 1408, 6, F16, True),
    (5, 100, 36, 2, F32, False),   # h % 4 != 0: scalar weight path
    (5, 100, 36, 2, F16, True),
    (3, 33, 17, 3, F16, False),    # odd shapes, k == E
    (1, 64, 64, 1, F16, False),    # single expert
    (8, 264, 520, 2, F16, True),   # x staged in LDS, partial last chunk of a row
    (4, 8200, 64, 2, F16, False),  # h above the LDS copy's bound: x from registers
    (8, 256, 8448, 2, F16, False), # 1056 gate/up blocks, over 4 per CU: x from registers
]


def ids_of(c):
    E, h, I, k, wd, rn = c
    return f"E{E}-h{h}-I{I}-k{k}-{WNAME[wd]}{'-renorm' if rn else ''}"


def robust_layer(E, h, I, wd, k, device, x_dtype=F32, batch=None, seed0=0):
    """First seed >= seed0 whose selection passes the oracle's margin guard
    for every token (decided on the CPU before anything runs on the GPU)."""
    for seed in range(seed0, seed0 + 50):
        x, gw, buf = make_layer(E, h, I, wd, router_std=h ** -0.5, expert_std=0.05, seed=seed,
                                batch=batch, device=device, x_dtype=x_dtype)
        xs = x.float().cpu().double().numpy().reshape(-1, h)
        gws = gw.cpu().double().numpy()
        if all(O.selection_is_robust(gws, xs[b], k) for b in range(xs.shape[0])):
            return x, gw, buf, seed
    raise AssertionError("no robust seed found")


def out_tol(x_dtype):
    return 2e-3 if x_dtype == F16 else 1e-4


@pytest.mark.parametrize("x_dtype", [F32, F16], ids=["xf32", "xf16"])
@pytest.mark.parametrize("cfg", SMALL, ids=ids_of)
@pytest.mark.parametrize("op", ["fused", "naive"])
def test_single_token_parity(cuda, op, cfg, x_dtype):
    E, h, I, k, wd, rn = cfg
    x, gw, buf, seed = robust_layer(E, h, I, wd, k, cuda, x_dtype)
    ids = torch.empty(k, dtype=torch.int32, device=cuda)
    ws = torch.empty(k, dtype=torch.float32, device=cuda)
    fn = F.fused_moe if op == "fused" else F.naive_moe
    print(f"[gpu] {op} {ids_of(cfg)} x={x_dtype} seed={seed}", flush=True)
    out = fn(x, gw, buf, E, h, I, k, rn, ids, ws)
    torch.cuda.synchronize()
    assert out.dtype == x_dtype and out.shape == (h,)
    ref = oracle_token(x, gw, buf, E, h, I, k, rn)
    assert_parity(out, ids, ws, ref, rel_tol=out_tol(x_dtype), label=f"{op} {ids_of(cfg)}")


# Reduced-precision weights: bf16, and fp8 E4M3 with per-channel scales.
LOWP = [
    (8, 256, 512, 2, BF16, False),
    (8, 256, 512, 2, FP8, True),
    (64, 256, 512, 6, FP8, False),
    (16, 512, 1024, 4, FP8, True),
    (8, 1024, 2048, 2, BF16, True),
    (8, 4096, 1024, 2, FP8, True),    # 4 KB fp8 rows
    (8, 6144, 512, 2, FP8, False),    # fp8 rows longer than 4 KB
    (8, 6144, 512, 2, BF16, False),   # bf16 rows longer than 4 KB: 2 rows per wave
    (5, 100, 36, 2, BF16, False),     # h % 8 != 0: scalar path
    (5, 100, 36, 2, FP8, True),       # h % 16 != 0: scalar path
    (3, 48, 40, 3, FP8, False),       # I % 16 != 0: scalar path, k == E
    (8, 256, 512, 2, MX4, True),      # MXFP4: blocks of 32 along rows
    (64, 256, 512, 6, MX4, False),
    (16, 512, 1024, 4, MX4, True),
    (8, 4096, 1024, 2, MX4, True),    # 2 KB code rows
    (8, 6144, 512, 2, MX4, False),    # 3 KB code rows: x staged in LDS up to h = 6144
    (4, 6176, 256, 2, MX4, True),     # h just above the MXFP4 LDS copy: x from registers
    (5, 96, 64, 2, MX4, False),       # three and two blocks per row, k == 2 of 5
    # MXFP4 at h = 2048 and 4096 (x staged in LDS with the block scales)
    (8, 2048, 256, 2, MX4, False),
    (64, 2048, 128, 6, MX4, True),
    (16, 4096, 512, 4, MX4, False),
]


@pytest.mark.parametrize("x_dtype", [F32, F16], ids=["xf32", "xf16"])
@pytest.mark.parametrize("cfg", LOWP, ids=ids_of)
@pytest.mark.parametrize("op", ["fused", "naive", "batched"])
def test_low_precision_weight_parity(cuda, op, cfg, x_dtype):
    """The oracle decodes the same bf16 / fp8 bytes (fp8: codes times their
    gate-row, up-row and down-column scales) and runs the fp64 layer; the bar
    is the same as for fp16 weights."""
    E, h, I, k, wd, rn = cfg
    B = 3 if op == "batched" else None
    x, gw, buf, seed = robust_layer(E, h, I, wd, k, cuda, x_dtype, batch=B)
    print(f"[gpu] lowp {op} {ids_of(cfg)} x={x_dtype} seed={seed}", flush=True)
    if op == "batched":
        ids = torch.empty(B, k, dtype=torch.int32, device=cuda)
        ws = torch.empty(B, k, dtype=torch.float32, device=cuda)
        out = F.batched_fused_moe(x, gw, buf, E, h, I, k, rn, ids, ws)
        torch.cuda.synchronize()
        for b in range(B):
            ref = oracle_token(x[b], gw, buf, E, h, I, k, rn)
            assert_parity(out[b], ids[b], ws[b], ref, rel_tol=out_tol(x_dtype),
                          label=f"batched {ids_of(cfg)} b={b}")
        return
    ids = torch.empty(k, dtype=torch.int32, device=cuda)
    ws = torch.empty(k, dtype=torch.float32, device=cuda)
    fn = F.fused_moe if op == "fused" else F.naive_moe
    out = fn(x, gw, buf, E, h, I, k, rn, ids, ws)
    torch.cuda.synchronize()
    assert out.dtype == x_dtype and out.shape == (h,)
    ref = oracle_token(x, gw, buf, E, h, I, k, rn)
    assert_parity(out, ids, ws, ref, rel_tol=out_tol(x_dtype), label=f"{op} {ids_of(cfg)}")


@pytest.mark.parametrize("op", ["fused", "naive", "batched"])
def test_mxfp4_unaligned_x_takes_the_byte_path(cuda, op):
    """x that is not 16-byte aligned (a view one element into a larger
    tensor) makes MXFP4 take its byte-at-a-time path (two codes per load)."""
    E, h, I, k = 8, 256, 512, 2
    B = 2 if op == "batched" else None
    xa, gw, buf, seed = robust_layer(E, h, I, MX4, k, cuda, batch=B)
    big = torch.empty(xa.numel() + 1, dtype=xa.dtype, device=cuda)
    big[1:] = xa.reshape(-1)
    x = big[1:].view(xa.shape)
    assert x.data_ptr() % 16 != 0
    print(f"[gpu] mxfp4 unaligned {op} seed={seed}", flush=True)
    if op == "batched":
        out = F.batched_fused_moe(x, gw, buf, E, h, I, k, True)
        torch.cuda.synchronize()
        for b in range(B):
            assert_parity(out[b], None, None, oracle_token(xa[b], gw, buf, E, h, I, k, True),
                          label=f"unaligned batched b={b}")
        return
    fn = F.fused_moe if op == "fused" else F.naive_moe
    out = fn(x, gw, buf, E, h, I, k, True)
    torch.cuda.synchronize()
    assert_parity(out, None, None, oracle_token(xa, gw, buf, E, h, I, k, True),
                  label=f"unaligned {op}")


@pytest.mark.parametrize("cfg", SMALL, ids=ids_of)
def test_gate_topk_parity(cuda, cfg):
    E, h, I, k, wd, rn = cfg
    x, gw, _, seed = robust_layer(E, h, 8, wd, k, cuda, batch=5)
    print(f"[gpu] gate_topk {ids_of(cfg)} seed={seed}", flush=True)
    ids, ws = F.gate_topk(x, gw, E, h, k, rn)
    torch.cuda.synchronize()
    for b in range(5):
        l64 = O.router_logits(f64(gw), f64(x[b]))
        _, rid, rw = O.softmax_topk(l64.astype(np.float32), k, rn)
        np.testing.assert_array_equal(ids[b].cpu().numpy(), rid)
        np.testing.assert_allclose(ws[b].cpu().numpy(), rw, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("op", ["fused", "naive", "gate"])
def test_exact_tie_known_answers(cuda, op):
    """Ties constructed so that GPU and oracle see bit-identical logits."""
    E, h, I, k = 8, 128, 64, 3
    _, gw, buf = make_layer(E, h, I, F16, router_std=0.1, seed=1, device=cuda)

    def run(x, g):
        if op == "gate":
            return F.gate_topk(x, g, E, h, k)
        ids = torch.empty(k, dtype=torch.int32, device=cuda)
        ws = torch.empty(k, dtype=torch.float32, device=cuda)
        fn = F.fused_moe if op == "fused" else F.naive_moe
        out = fn(x, g, buf, E, h, I, k, False, ids, ws)
        return ids, ws, out

    # 1. hidden == 0: all logits exactly 0 -> ids 0..k-1, weights 1/E, output 0.
    r = run(torch.zeros(h, device=cuda), gw)
    assert r[0].tolist() == [0, 1, 2]
    assert torch.all(r[1] == 0.125)
    if op != "gate":
        assert torch.all(r[2] == 0)
    # 2. all router rows identical -> ids 0..k-1 for any x.
    x = torch.randn(h, device=cuda)
    same = gw[0:1].expand(E, h).contiguous()
    assert run(x, same)[0].tolist() == [0, 1, 2]
    # 3. duplicate rows 2 and 6 forced to the top: 2 must come first.
    g3 = gw.clone()
    g3[2] = x / x.norm() * 4.0
    g3[6] = g3[2]
    ids3 = run(x, g3)[0].tolist()
    assert ids3[:2] == [2, 6]


@pytest.mark.parametrize("E", [8, 24], ids=["E8-rows", "E24-wave"])
@pytest.mark.parametrize("B", [3, 20], ids=["B3-in-kernel-route", "B20-route-kernel"])
def test_batched_exact_tie_known_answers(cuda, B, E):
    """The same ties through the grouped batched path (h and I multiples of
    128).  B = 3 routes inside the gate/up kernel, B = 20 in k_route; E = 8
    selects four tokens per wave (one per 16-lane row), E = 24 one token per
    wave.  Every token must get the answers the single-token op gives."""
    h, I, k = 128, 128, 3
    _, gw, buf = make_layer(E, h, I, F16, router_std=0.1, seed=1, device=cuda)
    print(f"[gpu] batched ties E={E} B={B}", flush=True)

    def run(x, g):
        ids = torch.empty(B, k, dtype=torch.int32, device=cuda)
        ws = torch.empty(B, k, dtype=torch.float32, device=cuda)
        out = F.batched_fused_moe(x, g, buf, E, h, I, k, False, ids, ws)
        torch.cuda.synchronize()
        return ids, ws, out

    # 1. x == 0: all logits exactly 0 -> ids 0..k-1, weights 1/E, output 0.
    ids, ws, out = run(torch.zeros(B, h, device=cuda), gw)
    assert ids.tolist() == [[0, 1, 2]] * B
    assert torch.all(ws == torch.tensor(1.0 / E, dtype=torch.float32))
    assert torch.all(out == 0)
    # 2. all router rows identical -> ids 0..k-1 for any x.
    x = torch.randn(B, h, device=cuda)
    same = gw[0:1].expand(E, h).contiguous()
    assert run(x, same)[0].tolist() == [[0, 1, 2]] * B
    # 3. duplicate rows 2 and 6 forced to the top for every token: 2 first.
    g3 = gw.clone()
    g3[2] = x[0] / x[0].norm() * 4.0
    g3[6] = g3[2]
    x3 = x[0:1].expand(B, h).contiguous()
    ids3 = run(x3, g3)[0]
    assert ids3[:, :2].tolist() == [[2, 6]] * B


@pytest.mark.parametrize("B", [1, 4, 16, 64])
@pytest.mark.parametrize("cfg", [(8, 256, 512, 1, F32, False), (8, 256, 512, 2, F32, False),
                                 (16, 512, 1024, 2, F16, True), (64, 256, 512, 6, F16, False)],
                         ids=ids_of)
def test_batched_parity(cuda, cfg, B):
    """Every row equals the oracle and the single-token op up to summation
    order, with identical ids and weights (tests/test_batched.py:33-59)."""
    E, h, I, k, wd, rn = cfg
    x, gw, buf, seed = robust_layer(E, h, I, wd, k, cuda, batch=B)
    ids = torch.empty(B, k, dtype=torch.int32, device=cuda)
    ws = torch.empty(B, k, dtype=torch.float32, device=cuda)
    print(f"[gpu] batched {ids_of(cfg)} B={B} seed={seed}", flush=True)
    out = F.batched_fused_moe(x, gw, buf, E, h, I, k, rn, ids, ws)
    torch.cuda.synchronize()
    assert out.shape == (B, h)
    for b in range(B):
        ref = oracle_token(x[b], gw, buf, E, h, I, k, rn)
        assert_parity(out[b], ids[b], ws[b], ref, label=f"batched b={b}")
        s_ids = torch.empty(k, dtype=torch.int32, device=cuda)
        s_ws = torch.empty(k, dtype=torch.float32, device=cuda)
        single = F.fused_moe(x[b].contiguous(), gw, buf, E, h, I, k, rn, s_ids, s_ws)
        assert torch.equal(s_ids, ids[b]) and torch.equal(s_ws, ws[b]), f"row {b} selection"
        assert_same_up_to_order(out[b], single, label=f"row {b} vs single-token op")


@pytest.mark.parametrize("scale,x_dtype", [(1.0, F32), (1e5, F32), (1e-6, F32), (3e-30, F32),
                                           (1.0, F16), (16.0, F16)],
                         ids=["x1", "x1e5", "x1e-6", "x3e-30", "xf16", "xf16-16"])
@pytest.mark.parametrize("h", [2048, 4096])
def test_mxfp4_single_token_x_range(cuda, h, scale, x_dtype):
    """MXFP4 single-token layers at h = 2048 and 4096 match the oracle at the
    usual bar for x scaled far from 1 (up to 1e5, down to near fp32's bottom)
    and for fp16 x (scaled by 16 at most: the fp16 output grows with the
    square of x).  The router is scaled inversely so that the routing stays
    the same."""
    E, I, k, rn = 8, 512, 2, True
    x, gw, buf = make_layer(E, h, I, MX4, router_std=h ** -0.5, expert_std=0.05, seed=7,
                            device=cuda)
    x = (x * scale).to(x_dtype)
    gw = (gw / scale).contiguous()
    assert torch.isfinite(x).all() and bool((x != 0).any())
    ref = oracle_token(x, gw, buf, E, h, I, k, rn)
    print(f"[gpu] mxfp4 single token h={h} x*{scale} {x_dtype} robust={ref['robust']}", flush=True)
    ids = torch.empty(k, dtype=torch.int32, device=cuda)
    ws = torch.empty(k, dtype=torch.float32, device=cuda)
    out = F.fused_moe(x, gw, buf, E, h, I, k, rn, ids, ws)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    np.testing.assert_array_equal(ids.cpu().numpy(), ref["ids"])
    err = O.relative_error(f64(out), ref["out"])
    assert err < out_tol(x_dtype), f"relative error {err:.3e}"


def test_batched_empty_batch(cuda):
    E, h, I, k = 8, 64, 64, 2
    _, gw, buf = make_layer(E, h, I, F16, seed=0, device=cuda)
    out = F.batched_fused_moe(torch.empty(0, h, device=cuda), gw, buf, E, h, I, k)
    assert out.shape == (0, h)


GROUPED = [(8, 256, 512, 2, False), (16, 512, 1024, 2, True), (64, 256, 512, 6, False),
           (8, 384, 640, 1, True)]


# (B, routing): tiles of 16 tokens for B <= 16 and of 32 for B <= 32; beyond
# that 32-token tiles when no expert has more than 32 (token, expert) pairs,
# else 64-token tiles.  Clustered batches of 33 and 80 put more than 32 pairs
# on one expert (E = 16 at B = 33 exactly 32: the 32-token class), random
# batches of 33 and 48 at most 18.
BATCHES = [(2, "clustered"), (5, "clustered"), (24, "clustered"), (33, "clustered"),
           (80, "clustered"), (33, "random"), (48, "random")]


@pytest.mark.parametrize("wd", [F16, FP8, BF16, MX4, F32], ids=["f16", "fp8", "bf16", "mxfp4", "f32"])
@pytest.mark.parametrize("x_dtype", [F32, F16], ids=["xf32", "xf16"])
@pytest.mark.parametrize("B,routing", BATCHES, ids=[f"B{b}-{r}" for b, r in BATCHES])
@pytest.mark.parametrize("cfg", GROUPED,
                         ids=lambda c: f"E{c[0]}-h{c[1]}-I{c[2]}-k{c[3]}" + ("-renorm" if c[4] else ""))
def test_grouped_batched_parity(cuda, cfg, B, routing, x_dtype, wd):
    """The grouped MFMA batched path (fp16, fp8, bf16 or MXFP4 weights, h and
    I multiples of 128; fp32 weights with exact fp32 MFMA products; fp8 and
    MXFP4 codes are staged raw and decoded per MFMA fragment, fp8 to fp16
    (row scales in the epilogue), MXFP4 to bf16 times its block scale; with
    16-token tiles (B <= 16) gate/up and down each take 256-byte K steps when
    h, respectively I, is a multiple of them: the shapes here give fp8 and
    MXFP4 both widths on both kernels;
    bf16 and MXFP4 weights take x and act as two bf16 terms, within 2^-18 of
    them, so their rows are compared with the single-token op at 5e-5 of
    max|out| instead of 1e-5).
    Tokens cluster on one expert pair, so experts get anywhere from 1 to B
    tokens (B = 80 puts more than 64 on one expert: two token passes), or
    route at random (x ~ N(0, 1)), which keeps every expert at 32 pairs or
    fewer and so pins the 32-token class beyond 32 tokens.  Every
    row's ids and weights are bit-identical to the single-token op and its
    output equals that op's up to summation order; a subset is checked against
    the oracle; two calls are bit-identical."""
    E, h, I, k, rn = cfg
    _, gw, buf = make_layer(E, h, I, wd, router_std=h ** -0.5, expert_std=0.05, seed=3,
                            device=cuda)
    pair = (1, 1) if k == 1 else (1, E - 1)  # k = 1: every token on one expert
    if routing == "clustered":
        x = clustered_batch(gw, B, pair=pair, alpha=4.0, seed=B, device=cuda).to(x_dtype)
    else:
        gen = torch.Generator(device="cpu").manual_seed(B)
        x = torch.randn(B, h, generator=gen).to(device=cuda, dtype=x_dtype)
    print(f"[gpu] grouped E{E}-h{h}-I{I}-k{k} B={B} {routing} {x_dtype} {WNAME[wd]}", flush=True)
    ids = torch.empty(B, k, dtype=torch.int32, device=cuda)
    ws = torch.empty(B, k, dtype=torch.float32, device=cuda)
    out = F.batched_fused_moe(x, gw, buf, E, h, I, k, rn, ids, ws)
    again = F.batched_fused_moe(x, gw, buf, E, h, I, k, rn)
    torch.cuda.synchronize()
    assert torch.equal(out, again), "grouped path is not deterministic"
    counts = np.bincount(ids.cpu().numpy().ravel(), minlength=E)
    assert counts.sum() == B * k
    if B == 80:
        assert counts.max() > 64, counts
    if routing == "random":
        assert counts.max() <= 32, counts  # 32-token tiles for B > 32
    elif B == 33:
        assert (counts.max() > 32) == (E != 16), counts  # 64-token tiles except at E = 16
    checked = 0
    for b in range(B):
        s_ids = torch.empty(k, dtype=torch.int32, device=cuda)
        s_ws = torch.empty(k, dtype=torch.float32, device=cuda)
        single = F.fused_moe(x[b].contiguous(), gw, buf, E, h, I, k, rn, s_ids, s_ws)
        assert torch.equal(s_ids, ids[b]) and torch.equal(s_ws, ws[b]), f"row {b} selection"
        tol = 5e-5 if (wd in (BF16, MX4) and out.dtype == torch.float32) else None
        assert_same_up_to_order(out[b], single, label=f"row {b} vs single-token op", tol=tol)
        if b % 8 == 0:
            ref = oracle_token(x[b], gw, buf, E, h, I, k, rn)
            if ref["robust"]:
                assert_parity(out[b], ids[b], ws[b], ref, rel_tol=out_tol(x_dtype),
                              label=f"grouped b={b}")
                checked += 1
    assert checked >= 1


@pytest.mark.parametrize("batch", [None, 4], ids=["token", "batch4"])
def test_graphed_stack_replays_match_eager(cuda, batch):
    """A 3-layer stack captured as one HIP graph: every replay equals the
    eager step bit for bit, for the captured input and for new inputs, with
    eager launches and host synchronisations between replays (a replay must
    not depend on state left by the capture or by the previous replay)."""
    from warp_route.stack import MoEStack
    E, h, I, k = 8, 256, 512, 2
    layers = []
    for s in range(3):
        _, gw, buf = make_layer(E, h, I, F16, router_std=h ** -0.5, expert_std=0.05, seed=20 + s,
                                device=cuda)
        layers.append((gw, buf))
    stack = MoEStack(layers, E, h, I, k, renormalize=True)
    shape = (h,) if batch is None else (batch, h)
    gen = torch.Generator(device="cpu").manual_seed(5)
    xs = [torch.randn(*shape, generator=gen).to(cuda) for _ in range(3)]
    want = [stack(x).clone() for x in xs]
    torch.cuda.synchronize()
    graphed = stack.capture(xs[0])
    for rep in range(3):
        for i, x in enumerate(xs):
            got = graphed(x).clone()
            torch.cuda.synchronize()
            assert torch.equal(got, want[i]), f"replay {rep}, input {i}"
            eager = stack(xs[(i + 1) % 3])  # eager work between replays
            torch.cuda.synchronize()
            assert torch.equal(eager, want[(i + 1) % 3])


def test_errors_are_python_exceptions(cuda):
    E, h, I, k = 8, 64, 64, 2
    x, gw, buf = make_layer(E, h, I, F16, seed=0, device=cuda)
    with pytest.raises(RuntimeError, match="weight_buf too small"):
        F.fused_moe(x, gw, buf[:-1], E, h, I, k)
    with pytest.raises(RuntimeError, match="top_k"):
        F.fused_moe(x, gw, buf, E, h, I, 7)
    with pytest.raises(RuntimeError, match="num_experts"):
        F.naive_moe(x, torch.randn(65, h, device=cuda), buf, 65, h, I, k)
    with pytest.raises(RuntimeError, match="gate_w must have shape"):
        F.fused_moe(x, gw[:4], buf, E, h, I, k)
    with pytest.raises(RuntimeError, match="float32"):
        F.fused_moe(x, gw.double(), buf, E, h, I, k)
    with pytest.raises(ValueError):
        F.batched_fused_moe(x, gw, buf, E, h, I, k)


def test_deterministic(cuda):
    cfg = CONFIGS["toy"]
    x, gw, buf = make_config_layer(cfg, seed=0, device=cuda)
    a = F.fused_moe(x, gw, buf, cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k)
    b = F.fused_moe(x, gw, buf, cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k)
    assert torch.equal(a, b)


def test_c_abi_direct_call_matches_extension(cuda):
    """wr_fused_moe through ctypes on torch-owned device memory."""
    E, h, I, k = 16, 512, 256, 4
    x, gw, buf, _ = robust_layer(E, h, I, F16, k, cuda)
    want = F.fused_moe(x, gw, buf, E, h, I, k, True)
    out = torch.empty_like(x)
    ids = torch.empty(k, dtype=torch.int32, device=cuda)
    ws = torch.empty(k, dtype=torch.float32, device=cuda)
    nws = capi.lib().wr_workspace_bytes(capi.WR_KIND_FUSED, E, h, I, k, 1)
    work = torch.empty(nws, dtype=torch.uint8, device=cuda)
    a = capi.WrMoeArgs()
    a.gate_w, a.weight_buf = gw.data_ptr(), buf.data_ptr()
    a.weight_bytes = buf.numel() * buf.element_size()
    a.weight_dtype, a.act_dtype = capi.WR_F16, capi.WR_F32
    a.num_experts, a.hidden_dim, a.intermediate_dim, a.top_k = E, h, I, k
    a.renormalize, a.batch_size = 1, 1
    a.x, a.out = x.data_ptr(), out.data_ptr()
    a.topk_ids, a.topk_weights = ids.data_ptr(), ws.data_ptr()
    a.workspace, a.workspace_bytes = work.data_ptr(), nws
    st = capi.call("wr_fused_moe", a, torch.cuda.current_stream().cuda_stream)
    assert st == capi.WR_OK, capi.status_str(st)
    torch.cuda.synchronize()
    assert torch.equal(out, want)


@pytest.mark.parametrize("wd", [F16, FP8], ids=["f16", "fp8"])
def test_split_route_ffn_matches_fused(cuda, wd):
    """wr_fused_moe_route then wr_fused_moe_ffn on one stream and workspace is
    bit-identical to wr_fused_moe, on a workspace that starts as junk and is
    reused for a second layer."""
    E, h, I, k = 8, 1024, 2048, 2
    stream = torch.cuda.current_stream().cuda_stream
    nws = capi.lib().wr_workspace_bytes(capi.WR_KIND_FUSED, E, h, I, k, 1)
    work = torch.full((nws,), 0x5A, dtype=torch.uint8, device=cuda)
    for seed in (4, 5):
        x, gw, buf, _ = robust_layer(E, h, I, wd, k, cuda, seed0=seed)
        want = torch.empty_like(x)
        got = torch.full_like(x, float("nan"))
        a = _fused_args(x, gw, buf, E, h, I, k, want, work, renorm=1)
        assert capi.call("wr_fused_moe", a, stream) == capi.WR_OK
        a = _fused_args(x, gw, buf, E, h, I, k, got, work, renorm=1)
        assert capi.call("wr_fused_moe_route", a, stream) == capi.WR_OK
        assert capi.call("wr_fused_moe_ffn", a, stream) == capi.WR_OK
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"seed {seed}"
        ref = oracle_token(x, gw, buf, E, h, I, k, True)
        assert_parity(got, None, None, ref, label=f"split {WNAME[wd]}")


def _fused_args(x, gw, buf, E, h, I, k, out, work, renorm=0):
    a = capi.WrMoeArgs()
    a.gate_w, a.weight_buf = gw.data_ptr(), buf.data_ptr()
    a.weight_bytes = buf.numel() * buf.element_size()
    a.weight_dtype = {F32: capi.WR_F32, F16: capi.WR_F16, BF16: capi.WR_BF16,
                      FP8: capi.WR_FP8_E4M3, MX4: capi.WR_MXFP4}[buf.dtype]
    a.act_dtype = capi.WR_F16 if x.dtype == torch.float16 else capi.WR_F32
    a.num_experts, a.hidden_dim, a.intermediate_dim, a.top_k = E, h, I, k
    a.renormalize, a.batch_size = renorm, 1
    a.x, a.out = x.data_ptr(), out.data_ptr()
    a.workspace, a.workspace_bytes = work.data_ptr(), work.numel()
    return a


@pytest.mark.parametrize("shape", [(16, 512, 256, 4, F16), (8, 4096, 14336, 2, F16),
                                   (64, 2048, 1408, 6, F16), (8, 192, 100, 3, F16),
                                   (8, 4096, 14336, 2, FP8), (16, 6144, 10752, 4, FP8),
                                   (8, 4096, 14336, 2, MX4), (16, 6144, 10752, 4, MX4)],
                         ids=["small", "mixtral", "deepseek", "ragged", "mixtral-fp8",
                              "dbrx-fp8", "mixtral-mxfp4", "dbrx-mxfp4"])
def test_fused_handoff_never_times_out(cuda, shape):
    """Single-token fused kernel: every gate/up block added its arrival to
    its arrival word (64 words of 64 bits, 256 bytes apart) and no down
    block's bounded wait expired (timeout word after them).  Gate/up blocks =
    act chunks k * ceil(ceil(I / rpw) / 4), rounded up to a multiple of
    8 * 32 / (4 rpw), with rpw = 4 rows per wave for fp16 rows of at most 2 KB
    (h <= 1024, 16-byte vectors) and for all 16-byte-vector fp8 rows, else 2.
    The workspace starts as junk: the router kernel must zero the control
    block on every call.  Word c holds {arrivals of the blocks b with b mod 64
    = c in bits 0-15, the sum of their XCD rotations r = (XCD - b) mod 8 in
    bits 16-31, the sum of r^2 in bits 32-63}.  Any rotations give correct
    results (more than one switches the down blocks to a full acquire)."""
    E, h, I, k, wd = shape
    x, gw, buf = make_layer(E, h, I, wd, router_std=h ** -0.5, seed=2, device=cuda,
                            gen_device=cuda)
    nws = capi.lib().wr_workspace_bytes(capi.WR_KIND_FUSED, E, h, I, k, 1)
    work = torch.full((nws,), 0xAB, dtype=torch.uint8, device=cuda)
    out = torch.empty_like(x)
    a = _fused_args(x, gw, buf, E, h, I, k, out, work)
    if wd == FP8:
        rpw = 4 if (h % 16 == 0 and I % 16 == 0) else 2
    elif wd == MX4:
        rpw = 4  # 16-byte aligned buffers
    else:
        rpw = 4 if (h % 8 == 0 and I % 8 == 0 and h * 2 <= 2048) else 2
    group = 8 * (32 // (4 * rpw))
    n1 = (k * (((I + rpw - 1) // rpw + 3) // 4) + group - 1) // group * group
    for _ in range(3):
        assert capi.call("wr_fused_moe", a, torch.cuda.current_stream().cuda_stream) == 0
        torch.cuda.synchronize()
        ctrl = work[:66 * 256].cpu()
        assert int(ctrl[64 * 256:64 * 256 + 4].view(torch.int32)[0]) == 0, \
            "a down block's wait expired"
        arr = [int(v) for v in ctrl[:64 * 256].view(torch.int64)[0::32]]
        counts = [a & 0xFFFF for a in arr]
        assert counts == [(n1 - c + 63) // 64 for c in range(64)]
        rots = set()
        for n, word in zip(counts, arr):
            sr, sq = (word >> 16) & 0xFFFF, word >> 32
            assert sr <= 7 * n and sq <= 49 * n and sr * sr <= n * sq, (n, sr, sq)
            if n and sr * sr == n * sq:
                rots.add(sr // n)  # one rotation among this word's arrivals
    print(f"[gpu] handoff {shape}: gate/up blocks {n1}, rotations {sorted(rots)}")
    ref = oracle_token(x, gw, buf, E, h, I, k, False)
    np.testing.assert_allclose(f64(out), ref["out"], rtol=1e-2, atol=1e-2)
    del buf
    torch.cuda.empty_cache()


def test_fused_workspace_reused_across_layers(cuda):
    """Two different layers called alternately through ONE workspace (the act
    lines sit at the same addresses every call) give, call after call, exactly
    the outputs each layer gives through a fresh workspace.  A down block that
    read act values left by the previous call would break the equality."""
    E, h, I, k = 8, 1024, 2048, 2
    layers = [make_layer(E, h, I, F16, router_std=h ** -0.5, seed=s, device=cuda,
                         gen_device=cuda) for s in (11, 12)]
    want = []
    for x, gw, buf in layers:
        fresh = torch.zeros(capi.lib().wr_workspace_bytes(capi.WR_KIND_FUSED, E, h, I, k, 1),
                            dtype=torch.uint8, device=cuda)
        o = torch.empty_like(x)
        assert capi.call("wr_fused_moe", _fused_args(x, gw, buf, E, h, I, k, o, fresh),
                         torch.cuda.current_stream().cuda_stream) == 0
        want.append(o)
    torch.cuda.synchronize()
    assert not torch.equal(want[0], want[1])
    shared = torch.empty_like(fresh)
    outs = [torch.empty_like(layers[0][0]) for _ in range(40)]
    stream = torch.cuda.current_stream().cuda_stream
    for i, o in enumerate(outs):
        x, gw, buf = layers[i % 2]
        assert capi.call("wr_fused_moe", _fused_args(x, gw, buf, E, h, I, k, o, shared),
                         stream) == 0
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert torch.equal(o, want[i % 2]), f"call {i}"


@pytest.mark.parametrize("wd", [F16, MX4], ids=["f16", "mxfp4"])
def test_fused_calls_on_two_streams(cuda, wd):
    """Single-token calls of two full-size Mixtral layers issued on two
    streams at once, 20 each, alternately, so that the two streams' kernels
    share the GPU and two hand-offs run at the same time, each on its own
    workspace.  Gate/up blocks never wait, and each kernel's gate/up blocks
    are dispatched before its down blocks, so neither kernel can hold slots
    the other one needs to finish.  Every output must equal its layer's
    output on one stream bit for bit (an expired wait would leave NaN
    rows)."""
    E, h, I, k = 8, 4096, 14336, 2
    layers = [make_layer(E, h, I, wd, router_std=h ** -0.5, seed=s, device=cuda,
                         gen_device=cuda) for s in (21, 22)]
    want = [F.fused_moe(x, gw, buf, E, h, I, k) for x, gw, buf in layers]
    torch.cuda.synchronize()
    assert not torch.equal(want[0], want[1])
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[], []]
    print(f"[gpu] fused calls on two streams, {WNAME[wd]}", flush=True)
    for _ in range(20):
        for i, st in enumerate(streams):
            with torch.cuda.stream(st):
                x, gw, buf = layers[i]
                outs[i].append(F.fused_moe(x, gw, buf, E, h, I, k))
    torch.cuda.synchronize()
    for i in range(2):
        for n, o in enumerate(outs[i]):
            assert torch.equal(o, want[i]), f"stream {i} call {n}"
    del layers
    torch.cuda.empty_cache()


def test_golden_toy_fixture(cuda):
    """The toy config (seed 0) against the committed fixture."""
    import json
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "toy_golden.json")
    gold = json.load(open(path))
    cfg = CONFIGS["toy"]
    x, gw, buf = make_config_layer(cfg, seed=0, device=cuda)
    ids = torch.empty(cfg.top_k, dtype=torch.int32, device=cuda)
    ws = torch.empty(cfg.top_k, dtype=torch.float32, device=cuda)
    for fn in (F.fused_moe, F.naive_moe):
        out = fn(x, gw, buf, cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k,
                 cfg.renormalize, ids, ws)
        torch.cuda.synchronize()
        assert ids.tolist() == gold["ids"]
        np.testing.assert_allclose(ws.cpu().numpy(), gold["weights"], rtol=1e-5)
        assert O.relative_error(f64(out), np.array(gold["out"])) < 1e-4


def test_moelayer(cuda):
    torch.manual_seed(0)
    layer = warp_route.MoELayer(8, 128, 96, top_k=2, renormalize=True,
                                weight_dtype=torch.float16).to(cuda)
    x = torch.randn(128, device=cuda)
    y1 = layer(x)
    yb = layer(torch.stack([x, -x]))
    assert_same_up_to_order(yb[0], y1, label="batched row vs single token")
    buf = layer._pack_weights()
    ref = oracle_token(x, layer.router.data, buf, 8, 128, 96, 2, True)
    np.testing.assert_allclose(f64(y1), ref["out"], rtol=1e-2, atol=1e-2)
    with torch.no_grad():
        layer.down_proj[int(ref["ids"][0])].mul_(2.0)
    assert layer._pack_weights() is not buf  # in-place change invalidates the pack
    y2 = layer(x)
    assert not torch.equal(y2, y1)


FULL = ["mixtral", "deepseek", "dbrx"]


@pytest.mark.parametrize("wd", [F16, FP8, BF16, MX4], ids=["f16", "fp8", "bf16", "mxfp4"])
@pytest.mark.parametrize("name", FULL)
@pytest.mark.parametrize("op", ["fused", "naive"])
def test_full_size_configs(cuda, name, op, wd):
    """BASELINE configs at full size (weights drawn on the GPU), parity on the
    selected experts; also with the same layers in bf16, fp8 and MXFP4."""
    cfg = CONFIGS[name].with_weights(wd)
    E, h, I, k = cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k
    for seed in range(20):
        x, gw, buf = make_config_layer(cfg, seed=seed, device=cuda, gen_device=cuda)
        if O.selection_is_robust(f64(gw), f64(x), k):
            break
        del buf
    print(f"[gpu] full {name} {op} {WNAME[wd]} seed={seed}", flush=True)
    ids = torch.empty(k, dtype=torch.int32, device=cuda)
    ws = torch.empty(k, dtype=torch.float32, device=cuda)
    fn = F.fused_moe if op == "fused" else F.naive_moe
    out = fn(x, gw, buf, E, h, I, k, cfg.renormalize, ids, ws)
    torch.cuda.synchronize()
    ref = oracle_token(x, gw, buf, E, h, I, k, cfg.renormalize)
    assert_parity(out, ids, ws, ref, label=f"{name} {op} {WNAME[wd]}")
    del buf
    torch.cuda.empty_cache()


TP = [("mixtral", F16, 2), ("mixtral", F16, 8), ("mixtral", FP8, 4), ("mixtral", MX4, 4),
      ("deepseek", F16, 2), ("dbrx", F16, 4)]


@pytest.mark.parametrize("name,wd,G", TP, ids=[f"{n}-{WNAME[w]}-tp{g}" for n, w, g in TP])
def test_tp_shards_sum_to_the_full_layer(cuda, name, wd, G):
    """A G-way tensor-parallel split over I on one GPU: each shard (the same
    kernels at I' = I/G) selects the full layer's experts and matches the
    oracle on its own weights, and the shards' outputs sum to the full
    layer's output up to fp32 summation order (the all-reduce a multi-GPU
    run would do)."""
    cfg = CONFIGS[name].with_weights(wd)
    E, h, I, k = cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k
    for seed in range(20):
        x, gw, buf = make_config_layer(cfg, seed=seed, device=cuda, gen_device=cuda)
        if O.selection_is_robust(f64(gw), f64(x), k):
            break
        del buf
    print(f"[gpu] tp {name} {WNAME[wd]} G={G} seed={seed}", flush=True)
    ids = torch.empty(k, dtype=torch.int32, device=cuda)
    full = F.fused_moe(x, gw, buf, E, h, I, k, cfg.renormalize, ids)
    total = torch.zeros_like(full)
    Is = I // G
    for s in range(G):
        part = F.shard_expert_weights(buf, E, h, I, G, s)
        sids = torch.empty(k, dtype=torch.int32, device=cuda)
        out = F.fused_moe(x, gw, part, E, h, Is, k, cfg.renormalize, sids)
        torch.cuda.synchronize()
        assert torch.equal(sids, ids), f"shard {s}: {sids.tolist()} != {ids.tolist()}"
        if s in (0, G - 1):
            ref = oracle_token(x, gw, part, E, h, Is, k, cfg.renormalize)
            assert_parity(out, sids, None, ref, label=f"{name} tp{G} shard {s}")
        total += out
        del part
    assert_same_up_to_order(total, full, label=f"{name} tp{G} sum of shards")
    del buf
    torch.cuda.empty_cache()
