"""GPU parity for batched decode and the layer stack at full Mixtral shape
for the grouped path's range scaling, and for the
single-token kernel's hand-off expiry report.

Every row of every batch is checked against the CPU oracle (ids bit-exact
under the margin guard, outputs within rtol = atol = 1e-2 and 1e-4 of
max|ref|); the stack is checked against an oracle chain
h_{l+1} = h_l + moe_l(h_l) computed in fp64 (warp_route/__init__.py:71-105
drives the reference's layers one call at a time; tests/test_batched.py:33-59
checks each batched row against the single-token result).
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests._helpers import (assert_parity, assert_same_up_to_order, f64, oracle_rows,
                            oracle_token)

from warp_route import capi
from warp_route import functional as F
from warp_route.synthetic import CONFIGS, clustered_batch, make_config_layer, make_layer

pytestmark = pytest.mark.gpu

F32, F16 = torch.float32, torch.float16
BF16, FP8, MX4 = torch.bfloat16, torch.float8_e4m3fn, torch.float4_e2m1fn_x2
WNAME = {F32: "f32", F16: "f16", BF16: "bf16", FP8: "fp8", MX4: "mxfp4"}
WTAG = {F32: capi.WR_F32, F16: capi.WR_F16, BF16: capi.WR_BF16, FP8: capi.WR_FP8_E4M3,
        MX4: capi.WR_MXFP4}


def check_rows(out, ids, ws, x, gw, buf, E, h, I, k, rn, label, rel_tol=1e-4,
               min_robust=None):
    """Every row of a batched result against the oracle (rows whose selection
    fails the margin guard are only counted), and against the single-token
    op: identical ids and weights, outputs equal up to summation order."""
    rows = oracle_rows(x, gw, buf, E, h, I, k, rn)
    robust = 0
    B = x.shape[0]
    for b in range(B):
        if rows[b]["robust"]:
            assert_parity(out[b], ids[b], ws[b] if ws is not None else None, rows[b],
                          rel_tol=rel_tol, label=f"{label} b={b}")
            robust += 1
        s_ids = torch.empty(k, dtype=torch.int32, device=x.device)
        single = F.fused_moe(x[b].contiguous(), gw, buf, E, h, I, k, rn, s_ids)
        torch.cuda.synchronize()
        assert torch.equal(s_ids, ids[b]), f"{label} row {b} selection"
        assert_same_up_to_order(out[b], single, label=f"{label} row {b} vs single-token op")
    need = max(1, (3 * B) // 4) if min_robust is None else min_robust
    assert robust >= need, f"{label}: only {robust} of {B} rows robust"
    return robust


@pytest.fixture(scope="module")
def mixtral_layer(cuda):
    cfg = CONFIGS["mixtral"]
    _, gw, buf = make_config_layer(cfg, seed=0, device=cuda, gen_device=cuda)
    yield cfg, gw, buf
    del buf
    torch.cuda.empty_cache()


@pytest.mark.parametrize("B", [1, 4, 16, 32, 64])
def test_full_size_batched_clustered_every_row(cuda, mixtral_layer, B):
    """batched_fused_moe at Mixtral shape, tokens clustered on one expert pair
    (the configs[4] recipe, alpha = 4): every row against the oracle and the
    single-token op."""
    cfg, gw, buf = mixtral_layer
    E, h, I, k = cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k
    x = clustered_batch(gw, B, pair=(3, 5), alpha=4.0, seed=1, device=cuda)
    print(f"[gpu] full batched mixtral B={B}, every row", flush=True)
    ids = torch.empty(B, k, dtype=torch.int32, device=cuda)
    ws = torch.empty(B, k, dtype=torch.float32, device=cuda)
    out = F.batched_fused_moe(x, gw, buf, E, h, I, k, True, ids, ws)
    torch.cuda.synchronize()
    pairs = {tuple(sorted(r)) for r in ids.cpu().tolist()}
    assert (3, 5) in pairs
    check_rows(out, ids, ws, x, gw, buf, E, h, I, k, True, f"mixtral B={B}")


TILE_CLASS = [("random", F16, F32), ("clustered", F16, F32), ("random", FP8, F32),
              ("clustered", FP8, F32), ("random", MX4, F32), ("clustered", MX4, F32),
              ("random", BF16, F32), ("clustered", BF16, F32), ("random", F16, F16)]


@pytest.mark.parametrize("routing,wd,x_dtype", TILE_CLASS,
                         ids=[f"{r}-{WNAME[w]}-x{WNAME[x]}" for r, w, x in TILE_CLASS])
def test_full_size_batched_tile_class_every_row(cuda, routing, wd, x_dtype):
    """Beyond 32 tokens a call runs every expert in 32-token tiles when no
    expert has more than 32 pairs, else in 64-token tiles (the device decides
    from the pair counts). B = 48 at Mixtral shape: random tokens (at most
    about 20 pairs per expert) take the 32-token launch, tokens clustered on
    one pair (most of the batch on each of its experts) the 64-token one. Every row
    against the oracle; fp16, fp8, MXFP4 and bf16 weights with fp32 x, and fp16
    x through the 32-token class."""
    cfg = CONFIGS["mixtral"].with_weights(wd)
    E, h, I, k = cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k
    B = 48
    x, gw, buf = make_config_layer(cfg, seed=5, batch=B, device=cuda, gen_device=cuda)
    if routing == "clustered":
        x = clustered_batch(gw, B, pair=(2, 7), alpha=4.0, seed=5, device=cuda)
    x = x.to(x_dtype)
    print(f"[gpu] full batched mixtral {WNAME[wd]} B={B} {routing} x {WNAME[x_dtype]}, "
          f"every row", flush=True)
    ids = torch.empty(B, k, dtype=torch.int32, device=cuda)
    ws = torch.empty(B, k, dtype=torch.float32, device=cuda)
    out = F.batched_fused_moe(x, gw, buf, E, h, I, k, cfg.renormalize, ids, ws)
    torch.cuda.synchronize()
    most = int(np.bincount(ids.cpu().numpy().reshape(-1), minlength=E).max())
    assert (most <= 32) == (routing == "random"), f"{routing}: {most} pairs on one expert"
    check_rows(out, ids, ws, x, gw, buf, E, h, I, k, cfg.renormalize,
               f"mixtral {WNAME[wd]} B={B} {routing} x {WNAME[x_dtype]}",
               rel_tol=2e-3 if x_dtype == F16 else 1e-4)
    del buf
    torch.cuda.empty_cache()


@pytest.mark.parametrize("B", [4, 24, 64])
def test_full_size_batched_fp32_weights_every_row(cuda, B):
    """fp32 weights (the reference's only format) at Mixtral shape through the
    grouped path (exact fp32 MFMA products), tokens clustered on one pair:
    every row against the oracle and the single-token op.  Each selected
    expert's weights stream once per call, not once per token."""
    cfg = CONFIGS["mixtral"].with_weights(F32)
    E, h, I, k = cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k
    _, gw, buf = make_config_layer(cfg, seed=0, device=cuda, gen_device=cuda)
    x = clustered_batch(gw, B, pair=(3, 5), alpha=4.0, seed=2, device=cuda)
    print(f"[gpu] full batched mixtral fp32 weights B={B}, every row", flush=True)
    ids = torch.empty(B, k, dtype=torch.int32, device=cuda)
    ws = torch.empty(B, k, dtype=torch.float32, device=cuda)
    out = F.batched_fused_moe(x, gw, buf, E, h, I, k, True, ids, ws)
    torch.cuda.synchronize()
    check_rows(out, ids, ws, x, gw, buf, E, h, I, k, True, f"mixtral fp32 B={B}")
    del buf
    torch.cuda.empty_cache()


@pytest.fixture(scope="module")
def mixtral_stack(cuda):
    """Four independent full-size Mixtral layers (11.3 GB of fp16 experts)."""
    cfg = CONFIGS["mixtral"]
    layers, x0 = [], None
    for s in range(4):
        x, gw, buf = make_config_layer(cfg, seed=100 + s, device=cuda, gen_device=cuda)
        layers.append((gw, buf))
        x0 = x if x0 is None else x0
    yield cfg, layers, x0
    del layers
    torch.cuda.empty_cache()


def oracle_chain(x, layers, cfg, residual=True):
    """fp64 h_{l+1} = h_l + moe_l(h_l) (or moe_l(h_l) without the residual)
    for every row of x ([h] or [B, h]); also whether every layer's selection
    of every row passed the margin guard."""
    E, h, I, k = cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k
    cur = f64(x).reshape(-1, h)
    robust = True
    for gw, buf in layers:
        rows = oracle_rows(torch.from_numpy(cur), gw, buf, E, h, I, k, cfg.renormalize)
        robust &= all(r["robust"] for r in rows)
        y = np.stack([r["out"] for r in rows])
        cur = cur + y if residual else y
    return cur.reshape(f64(x).shape), robust


@pytest.mark.parametrize("residual", [True, False], ids=["residual", "chained"])
@pytest.mark.parametrize("batch", [None, 4], ids=["token", "batch4"])
def test_stack_matches_oracle_chain(cuda, mixtral_stack, batch, residual):
    """A 4-layer full-size Mixtral stack, eager and replayed from one captured
    HIP graph, against the fp64 oracle chain; the graph is replayed several
    times with eager work and host synchronisations between replays, and
    every replay equals the eager step bit for bit.

    The synthetic layers have no normalisation between them, and a SwiGLU
    layer's output grows about with the square of its input, so the stream
    grows from layer to layer, with or without the residual adds (rows reach
    ~1e4-1e6 after four layers with the configs' N(0, 0.02) experts).  The
    rtol = atol = 1e-2 bar therefore applies to each row divided by its
    largest magnitude: an absolute tolerance of 1e-2 on an element of size 30
    in a row of size 6e5 is below fp32's resolution of that row."""
    from warp_route.stack import MoEStack
    cfg, layers, x0 = mixtral_stack
    E, h, I, k = cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k
    stack = MoEStack(layers, E, h, I, k, cfg.renormalize, residual=residual)
    for seed in range(9, 13):  # the first input whose chain routes robustly at every layer
        if batch is None:
            gen = torch.Generator(device="cpu").manual_seed(seed)
            x = x0 if seed == 9 else torch.randn(h, generator=gen).to(cuda)
        else:
            x = clustered_batch(layers[0][0], batch, pair=(2, 6), alpha=4.0, seed=seed,
                                device=cuda)
        want, robust = oracle_chain(x, layers, cfg, residual)
        if robust:
            break
    assert robust, "no input seed routes robustly through every layer"
    print(f"[gpu] stack of 4 mixtral layers, input {tuple(x.shape)}, residual={residual}, "
          f"seed {seed}", flush=True)
    eager = stack(x).clone()
    torch.cuda.synchronize()
    got = f64(eager)
    rows_got, rows_want = got.reshape(-1, h), want.reshape(-1, h)
    for b in range(rows_want.shape[0]):
        scale = np.abs(rows_want[b]).max()
        np.testing.assert_allclose(rows_got[b] / scale, rows_want[b] / scale, rtol=1e-2,
                                   atol=1e-2, err_msg=f"eager stack row {b}")
        err = O.relative_error(rows_got[b], rows_want[b])
        assert err < 1e-4, f"eager stack row {b}: relative error {err:.3e}"
    graphed = stack.capture(x)
    other = x.flip(0) if batch is not None else -x
    for rep in range(3):
        g = graphed(x).clone()
        torch.cuda.synchronize()
        assert torch.equal(g, eager), f"replay {rep} differs from the eager step"
        stack(other)  # eager work between replays
        torch.cuda.synchronize()
    print(f"[gpu] stack rel err {err:.2e}", flush=True)


# (name, x scale, router scale, expert std, x dtype): the grouped MFMA path
# splits x and act into two 16-bit terms; these cases take them far outside
# fp16's range (x 1e5: act ~1e11), below its normal range (x 1e-6; expert std
# 2e-4: act ~1e-5, whose low terms were fp16 subnormals before the power-of-
# two scaling), and fp16 x near the top of fp16's range (with small experts,
# so that the fp16 output stays finite).
RANGE = [("x1e5", 1e5, 1e-5, 0.05, F32), ("x1e-6", 1e-6, 1e6, 0.05, F32),
         ("std2e-4", 1.0, 1.0, 2e-4, F32), ("xf16-4096", 4096.0, 1.0 / 4096.0, 2e-4, F16)]


# (B, routing): 16-token tiles at B = 5, 32-token tiles at B = 24; at B = 40
# clustered tokens put more than 32 pairs on one expert (64-token tiles, act
# split ahead of the down kernel) and random tokens at most 32 on every
# expert (32-token tiles, whose down kernel splits act while staging it).
RANGE_BATCHES = [(5, "clustered"), (24, "clustered"), (40, "clustered"), (40, "random")]


@pytest.mark.parametrize("wd", [F16, FP8, BF16, MX4, F32], ids=["f16", "fp8", "bf16", "mxfp4", "f32"])
@pytest.mark.parametrize("B,routing", RANGE_BATCHES, ids=[f"B{b}-{r}" for b, r in RANGE_BATCHES])
@pytest.mark.parametrize("case", RANGE, ids=[c[0] for c in RANGE])
def test_grouped_batched_range(cuda, case, B, routing, wd):
    """The grouped path stays within the parity bar when x and act leave
    fp16's range: every row equals the single-token op (fp32 throughout) up
    to summation order, and every robust row the oracle."""
    name, xs, rs, es, x_dtype = case
    E, h, I, k, rn = 8, 512, 1024, 2, True
    _, gw, buf = make_layer(E, h, I, wd, router_std=h ** -0.5, expert_std=es, seed=3,
                            device=cuda)
    if routing == "clustered":
        x = clustered_batch(gw, B, pair=(1, E - 1), alpha=4.0, seed=B, device=cuda) * xs
    else:
        gen = torch.Generator(device="cpu").manual_seed(B)
        x = torch.randn(B, h, generator=gen).to(cuda) * xs
    x = x.to(x_dtype)
    gw = (gw * rs).contiguous()
    assert torch.isfinite(x).all()
    print(f"[gpu] grouped range {name} B={B} {routing} {WNAME[wd]}", flush=True)
    ids = torch.empty(B, k, dtype=torch.int32, device=cuda)
    ws = torch.empty(B, k, dtype=torch.float32, device=cuda)
    out = F.batched_fused_moe(x, gw, buf, E, h, I, k, rn, ids, ws)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all(), f"{name}: non-finite output"
    most = int(np.bincount(ids.cpu().numpy().reshape(-1), minlength=E).max())
    if B > 32:
        assert (most <= 32) == (routing == "random"), f"{routing}: {most} pairs on one expert"
    rows = oracle_rows(x, gw, buf, E, h, I, k, rn)
    checked = 0
    for b in range(B):
        s_ids = torch.empty(k, dtype=torch.int32, device=cuda)
        single = F.fused_moe(x[b].contiguous(), gw, buf, E, h, I, k, rn, s_ids)
        torch.cuda.synchronize()
        assert torch.equal(s_ids, ids[b]), f"row {b} selection"
        tol = 5e-5 if (wd in (BF16, MX4) and out.dtype == F32) else None
        assert_same_up_to_order(out[b], single, label=f"{name} row {b} vs single-token op",
                                tol=tol)
        if rows[b]["robust"]:
            # relative comparison only: outputs span 1e-13 to 1e11 here
            err = O.relative_error(f64(out[b]), rows[b]["out"])
            assert err < (2e-3 if x_dtype == F16 else 1e-4), f"{name} row {b}: {err:.3e}"
            np.testing.assert_array_equal(ids[b].cpu().numpy(), rows[b]["ids"])
            checked += 1
    assert checked >= 1


def _fused_args(x, gw, buf, E, h, I, k, out, work, renorm=0):
    a = capi.WrMoeArgs()
    a.gate_w, a.weight_buf = gw.data_ptr(), buf.data_ptr()
    a.weight_bytes = buf.numel() * buf.element_size()
    a.weight_dtype = WTAG[buf.dtype]
    a.act_dtype = capi.WR_F16 if x.dtype == torch.float16 else capi.WR_F32
    a.num_experts, a.hidden_dim, a.intermediate_dim, a.top_k = E, h, I, k
    a.renormalize, a.batch_size = renorm, 1
    a.x, a.out = x.data_ptr(), out.data_ptr()
    a.workspace, a.workspace_bytes = work.data_ptr(), work.numel()
    return a


@pytest.mark.parametrize("shape", [(8, 1024, 2048, 2, F16), (8, 4096, 14336, 2, F16),
                                   (64, 2048, 1408, 6, FP8)],
                         ids=["small", "mixtral", "deepseek-fp8"])
def test_fused_handoff_expiry_is_reported(cuda, shape):
    """Forced from the host: wait_extra = 1 raises every arrival target above
    what the gate/up blocks can reach, and spin_limit = 4 ends each down
    block's wait after 4 polls, so every kernel still exits normally.  Every
    down block must then write NaN to its rows, and wr_fused_moe_status must
    report WR_ETIMEOUT; the library's host-visible expiry word is set too
    (wr_fused_moe_expired, no synchronisation).  The next default call on the
    same workspace clears the timeout word and is correct again; the torch
    op's next call raises once for the earlier expiry (read from the
    host-visible word), the one after it does not, nor with the check
    switched on."""
    E, h, I, k, wd = shape
    x, gw, buf = make_layer(E, h, I, wd, router_std=h ** -0.5, seed=2, device=cuda,
                            gen_device=cuda)
    nws = capi.lib().wr_workspace_bytes(capi.WR_KIND_FUSED, E, h, I, k, 1)
    work = torch.empty(nws, dtype=torch.uint8, device=cuda)
    out = torch.zeros_like(x)
    stream = torch.cuda.current_stream().cuda_stream
    a = _fused_args(x, gw, buf, E, h, I, k, out, work)
    opts = capi.WrFusedOpts(spin_limit=4, wait_extra=1)
    print(f"[gpu] forced hand-off expiry {shape}", flush=True)
    st = capi.lib().wr_fused_moe_opts(ctypes.byref(a), ctypes.byref(opts),
                                      ctypes.c_void_p(stream))
    assert st == capi.WR_OK, capi.status_str(st)
    st = capi.lib().wr_fused_moe_status(ctypes.c_void_p(work.data_ptr()), nws,
                                        ctypes.c_void_p(stream))
    assert st == capi.WR_ETIMEOUT, capi.status_str(st)
    assert torch.isnan(out).all(), "a down block that gave up wrote a number"
    assert capi.lib().wr_fused_moe_expired(0) == 1  # set, and not cleared by reading
    assert capi.lib().wr_fused_moe_expired(0) == 1

    # default options again, same workspace: cleared and correct
    st = capi.lib().wr_fused_moe_opts(ctypes.byref(a), None, ctypes.c_void_p(stream))
    assert st == capi.WR_OK
    st = capi.lib().wr_fused_moe_status(ctypes.c_void_p(work.data_ptr()), nws,
                                        ctypes.c_void_p(stream))
    assert st == capi.WR_OK, capi.status_str(st)
    ref = oracle_token(x, gw, buf, E, h, I, k, False)
    np.testing.assert_allclose(f64(out), ref["out"], rtol=1e-2, atol=1e-2)
    with pytest.raises(RuntimeError, match="hand-off wait expired"):
        F.fused_moe(x, gw, buf, E, h, I, k)
    assert capi.lib().wr_fused_moe_expired(0) == 0  # reported once, then cleared
    want = F.fused_moe(x, gw, buf, E, h, I, k)
    torch.cuda.synchronize()
    assert torch.equal(out, want)

    F.set_handoff_check(True)
    try:
        again = F.fused_moe(x, gw, buf, E, h, I, k)
    finally:
        F.set_handoff_check(False)
    assert torch.equal(again, want)
    assert capi.lib().wr_fused_moe_expired(0) == 0
    del buf
    torch.cuda.empty_cache()


# Byte offset of the single-token workspace's 8 claim counters (one 256-byte
# line each): after 64 arrival words, the timeout word and one unused word.
CLAIM_OFFSET = (64 + 2) * 256


@pytest.mark.parametrize("shape,gu", [((8, 512, 8192, 2, F16), 64), ((8, 512, 8192, 2, F16), 992),
                                      ((8, 256, 2048, 2, F32), 32),
                                      ((8, 512, 8192, 2, BF16), 256),
                                      ((64, 2048, 1408, 6, F16), 0),
                                      ((64, 2048, 1408, 6, BF16), 0)],
                         ids=["f16-64", "f16-992", "f32-32", "bf16-256", "deepseek-f16",
                              "deepseek-bf16"])
def test_fused_claimed_gateup_slots(cuda, shape, gu):
    """Fewer gate/up blocks launched than the layer has chunk slots: the
    blocks claim the remaining slots as they finish (one claim counter per
    class of 8 blocks).  Forced with wr_fused_opts.gu_blocks at shapes that
    take the register path (1,024 slots over 64, 992 or 256 blocks, 256 over
    32), and the default at DeepSeek's shape (1,056 slots, one
    round of 1,024 resident blocks on a 256-CU GPU).  The output must be
    bit-identical to a call that launches every slot as a block (each act
    value is computed by one wave either way), match the oracle, and the
    claim counters must show n1 claims: every slot beyond the launched blocks
    once, plus one unsuccessful claim per block."""
    E, h, I, k, wd = shape
    x, gw, buf = make_layer(E, h, I, wd, router_std=h ** -0.5, seed=4, device=cuda,
                            gen_device=cuda)
    nws = capi.lib().wr_workspace_bytes(capi.WR_KIND_FUSED, E, h, I, k, 1)
    work = torch.empty(nws, dtype=torch.uint8, device=cuda)
    out = torch.zeros_like(x)
    stream = torch.cuda.current_stream().cuda_stream
    a = _fused_args(x, gw, buf, E, h, I, k, out, work)
    print(f"[gpu] claimed gate/up slots {shape} gu_blocks={gu}", flush=True)
    st = capi.lib().wr_fused_moe_opts(ctypes.byref(a), ctypes.byref(capi.WrFusedOpts(gu_blocks=gu)),
                                      ctypes.c_void_p(stream))
    assert st == capi.WR_OK, capi.status_str(st)
    st = capi.lib().wr_fused_moe_status(ctypes.c_void_p(work.data_ptr()), nws,
                                        ctypes.c_void_p(stream))
    assert st == capi.WR_OK, capi.status_str(st)
    claims = int(work[CLAIM_OFFSET:CLAIM_OFFSET + 8 * 256].view(torch.int32)[::64].sum())
    got = out.clone()

    # every slot launched as a block of its own (gu_blocks above the slot count)
    st = capi.lib().wr_fused_moe_opts(ctypes.byref(a),
                                      ctypes.byref(capi.WrFusedOpts(gu_blocks=1 << 20)),
                                      ctypes.c_void_p(stream))
    assert st == capi.WR_OK, capi.status_str(st)
    torch.cuda.synchronize()
    assert int(work[CLAIM_OFFSET:CLAIM_OFFSET + 8 * 256].view(torch.int32)[::64].sum()) == 0
    assert torch.equal(got, out), "claimed slots changed the output"
    ref = oracle_token(x, gw, buf, E, h, I, k, False)
    np.testing.assert_allclose(f64(got), ref["out"], rtol=1e-2, atol=1e-2)

    # n1: chunk slots, k * ceil(ceil(I / rpw) / 4) rounded up to 8 * 32 / (4 rpw)
    rpw = 2 if (h * buf.element_size() > 2048 and wd != FP8) else 4
    group = 8 * (32 // (4 * rpw))
    chunks = k * (-(-(-(-I // rpw)) // 4))
    n1 = -(-chunks // group) * group
    if gu > 0:
        assert claims == n1, (claims, n1)
    elif torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert claims == n1 == 1056, (claims, n1)
    del buf
    torch.cuda.empty_cache()
