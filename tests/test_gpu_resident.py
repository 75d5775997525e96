"""The single-token kernel's resident schedule (k_fused_res): every block of
the grid is resident at once, takes gate/up chunk slots from its XCD's queue,
then computes its own output rows from down weights it loaded into LDS.

Checked through the C-ABI (wr_fused_moe_opts: schedule 2 asks for it, 1 for
the split gate/up and down blocks of k_fused_ffn):

* outputs, ids and weights against the fp64 oracle at the parity bar, and
  against the split schedule (the same arithmetic per act value and per
  output row; only the order of the down sums across waves differs);
* the control block afterwards: every arrival counter at its count of slots,
  no expired wait, no slot taken across XCDs, and at least n1 claims;
* slots taken from other XCDs' queues: only XCD 0's blocks claim at first
  (claim_queues = 1) and every other block takes what is left after 2 polls;
  the output must be bit-identical to the default call (each act value and
  each output row is computed by the same code whichever block takes a
  slot), and the first rotation word must record the taking;
* the bounded wait's expiry, forced from the host: NaN rows and WR_ETIMEOUT.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests._helpers import assert_parity, f64, oracle_token
from warp_route import capi
from warp_route.synthetic import make_layer

pytestmark = pytest.mark.gpu

F32, F16, BF16 = torch.float32, torch.float16, torch.bfloat16
WTAG = {F32: capi.WR_F32, F16: capi.WR_F16, BF16: capi.WR_BF16}

# Word offsets (int32) in the control block: 64 arrival counters, the timeout
# word, one unused word, 64 rotation masks, 8 claim counters, 256 bytes apart.
TIMEOUT, ROT, CLAIM = 64 * 64, 66 * 64, 130 * 64

# (E, h, I, k, weights, x): DeepSeek's layer, Mixtral tensor-parallel shard
# shapes (I = 1792: the down weights fit LDS; I = 3584: the rest come from
# registers after the wait), a layer with 8 slots per block, small and odd
# ones, bf16, fp16 x.
SHAPES = [(64, 2048, 1408, 6, F16, F32), (64, 2048, 1408, 6, BF16, F32),
          (8, 4096, 1792, 2, F16, F32), (8, 4096, 3584, 2, F16, F16),
          (8, 256, 4096, 2, F16, F32), (16, 512, 256, 4, F16, F32),
          (8, 1024, 2048, 2, BF16, F16), (16, 520, 264, 3, F16, F32)]
IDS = ["deepseek", "deepseek-bf16", "tp8-shard", "tp4-shard-xf16", "claims", "small",
       "bf16-xf16", "odd"]


def _layer(E, h, I, k, wd, xd, device):
    """The first seed whose selection passes the margin guard."""
    for seed in range(40):
        x, gw, buf = make_layer(E, h, I, wd, router_std=h ** -0.5, seed=seed, device=device,
                                gen_device=device)
        if O.selection_is_robust(f64(gw), f64(x), k):
            return x.to(xd).contiguous(), gw, buf
    raise AssertionError("no robust seed")


def _args(x, gw, buf, E, h, I, k, out, ids, ws, work):
    a = capi.WrMoeArgs()
    a.gate_w, a.weight_buf = gw.data_ptr(), buf.data_ptr()
    a.weight_bytes = buf.numel() * buf.element_size()
    a.weight_dtype = WTAG[buf.dtype]
    a.act_dtype = capi.WR_F16 if x.dtype == torch.float16 else capi.WR_F32
    a.num_experts, a.hidden_dim, a.intermediate_dim, a.top_k = E, h, I, k
    a.renormalize, a.batch_size = 0, 1
    a.x, a.out = x.data_ptr(), out.data_ptr()
    a.topk_ids, a.topk_weights = ids.data_ptr(), ws.data_ptr()
    a.workspace, a.workspace_bytes = work.data_ptr(), work.numel()
    return a


def _run(a, **opts):
    st = capi.lib().wr_fused_moe_opts(ctypes.byref(a), ctypes.byref(capi.WrFusedOpts(**opts)),
                                      ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == capi.WR_OK, capi.status_str(st)


def _n1(h, I, k, wd):
    rpw = 4 if h * (4 if wd == F32 else 2) <= 2048 else 2
    group = 8 * (32 // (4 * rpw))
    return (k * (((I + rpw - 1) // rpw + 3) // 4) + group - 1) // group * group


@pytest.mark.parametrize("shape", SHAPES, ids=IDS)
def test_resident_schedule(cuda, shape):
    E, h, I, k, wd, xd = shape
    x, gw, buf = _layer(E, h, I, k, wd, xd, cuda)
    nws = capi.lib().wr_workspace_bytes(capi.WR_KIND_FUSED, E, h, I, k, 1)
    work = torch.full((nws,), 0xAB, dtype=torch.uint8, device=cuda)
    out, ids, ws = torch.empty_like(x), torch.empty(k, dtype=torch.int32, device=cuda), \
        torch.empty(k, dtype=torch.float32, device=cuda)
    a = _args(x, gw, buf, E, h, I, k, out, ids, ws, work)
    print(f"[gpu] resident schedule {shape}", flush=True)
    assert capi.lib().wr_fused_moe_schedule(ctypes.byref(a), ctypes.byref(
        capi.WrFusedOpts(schedule=2))) == 2
    _run(a, schedule=2)
    torch.cuda.synchronize()
    words = work[:138 * 256].view(torch.int32).cpu()
    n1 = _n1(h, I, k, wd)
    assert words[0:64 * 64:64].tolist() == [(n1 - c + 63) // 64 for c in range(64)]
    assert int(words[TIMEOUT]) == 0, "a wait expired"
    assert int(words[ROT]) == 0, "a slot was taken across XCDs in a normal call"
    assert int(words[CLAIM:CLAIM + 8 * 64:64].sum()) >= n1
    ref = oracle_token(x, gw, buf, E, h, I, k, False)
    # fp16 x gives fp16 outputs: their rounding (2^-11 relative) sets the bar
    tol = 2e-3 if xd == F16 else 1e-4
    assert_parity(out, ids, ws, ref, rel_tol=tol, label=f"resident {shape}")
    got = out.clone()

    # the split schedule: the same values up to the order of the down sums
    # (and, for fp16 outputs, one rounding step)
    _run(a, schedule=1)
    torch.cuda.synchronize()
    assert torch.equal(ids.cpu(), torch.from_numpy(ref["ids"]).to(torch.int32))
    scale = float(out.float().abs().max())
    near = 1e-3 if xd == F16 else 1e-5
    assert float((got.float() - out.float()).abs().max()) <= near * scale + 1e-30

    # again with the resident schedule: deterministic
    _run(a, schedule=2)
    torch.cuda.synchronize()
    assert torch.equal(out, got)
    del buf
    torch.cuda.empty_cache()


@pytest.mark.parametrize("shape", [SHAPES[0], SHAPES[2], SHAPES[4]],
                         ids=["deepseek", "tp8-shard", "claims"])
def test_resident_slots_taken_across_xcds(cuda, shape):
    E, h, I, k, wd, xd = shape
    x, gw, buf = _layer(E, h, I, k, wd, xd, cuda)
    nws = capi.lib().wr_workspace_bytes(capi.WR_KIND_FUSED, E, h, I, k, 1)
    work = torch.empty(nws, dtype=torch.uint8, device=cuda)
    out, ids, ws = torch.empty_like(x), torch.empty(k, dtype=torch.int32, device=cuda), \
        torch.empty(k, dtype=torch.float32, device=cuda)
    a = _args(x, gw, buf, E, h, I, k, out, ids, ws, work)
    print(f"[gpu] resident schedule, slots taken across XCDs {shape}", flush=True)
    _run(a, schedule=2)
    torch.cuda.synchronize()
    want = out.clone()
    for _ in range(2):
        out.zero_()
        _run(a, schedule=2, claim_queues=1, steal_after=2)
        torch.cuda.synchronize()
        words = work[:138 * 256].view(torch.int32).cpu()
        assert int(words[TIMEOUT]) == 0
        assert int(words[ROT]) != 0, "no slot of another XCD's queue was taken"
        assert torch.equal(out, want)
    del buf
    torch.cuda.empty_cache()


def test_resident_wait_expiry_is_reported(cuda):
    E, h, I, k, wd, xd = SHAPES[0]
    x, gw, buf = _layer(E, h, I, k, wd, xd, cuda)
    nws = capi.lib().wr_workspace_bytes(capi.WR_KIND_FUSED, E, h, I, k, 1)
    work = torch.empty(nws, dtype=torch.uint8, device=cuda)
    out, ids, ws = torch.empty_like(x), torch.empty(k, dtype=torch.int32, device=cuda), \
        torch.empty(k, dtype=torch.float32, device=cuda)
    a = _args(x, gw, buf, E, h, I, k, out, ids, ws, work)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    print("[gpu] resident schedule, forced wait expiry", flush=True)
    _run(a, schedule=2, spin_limit=4, wait_extra=1)
    assert capi.lib().wr_fused_moe_status(ctypes.c_void_p(work.data_ptr()), nws,
                                          stream) == capi.WR_ETIMEOUT
    assert torch.isnan(out).all()
    _run(a, schedule=2)
    assert capi.lib().wr_fused_moe_status(ctypes.c_void_p(work.data_ptr()), nws,
                                          stream) == capi.WR_OK
    ref = oracle_token(x, gw, buf, E, h, I, k, False)
    assert_parity(out, ids, ws, ref, label="resident after expiry")
    del buf
    torch.cuda.empty_cache()
