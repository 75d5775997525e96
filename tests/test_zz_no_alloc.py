"""The allocation-free single-token entry point (wr_fused_moe_noalloc): its
kernels use the library's fixed per-GPU scratch array instead of a caller
workspace.  Checked through the C-ABI against wr_fused_moe (same kernels,
caller workspace): bit-identical outputs, ids and weights, on two calls in a
row, the second with a smaller layer (the array keeps the first call's
contents), then once more with the first layer; the size limit is
rejected before any HIP call; and a call recorded into a HIP graph (after a
first eager call on the device) replays equal to the eager entry point."""
import ctypes

import numpy as np
import pytest
import torch

from tests._helpers import oracle_token, f64
from warp_route import capi
from warp_route.synthetic import make_layer

pytestmark = pytest.mark.gpu

WTAG = {torch.float16: capi.WR_F16, torch.float8_e4m3fn: capi.WR_FP8_E4M3,
        torch.float32: capi.WR_F32}


def _args(x, gw, buf, E, h, I, k, out, ids, ws, work=None):
    a = capi.WrMoeArgs()
    a.gate_w, a.weight_buf = gw.data_ptr(), buf.data_ptr()
    a.weight_bytes = buf.numel() * buf.element_size()
    a.weight_dtype = WTAG[buf.dtype]
    a.act_dtype = capi.WR_F16 if x.dtype == torch.float16 else capi.WR_F32
    a.num_experts, a.hidden_dim, a.intermediate_dim, a.top_k = E, h, I, k
    a.renormalize, a.batch_size = 1, 1
    a.x, a.out = x.data_ptr(), out.data_ptr()
    a.topk_ids, a.topk_weights = ids.data_ptr(), ws.data_ptr()
    if work is not None:
        a.workspace, a.workspace_bytes = work.data_ptr(), work.numel()
    return a


def _run_pair(cuda, shape, seed):
    """(noalloc out/ids/ws, reference out/ids/ws) for one layer."""
    E, h, I, k, wd = shape
    x, gw, buf = make_layer(E, h, I, wd, router_std=h ** -0.5, seed=seed, device=cuda,
                            gen_device=cuda)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    got = [torch.full_like(x, float("nan")), torch.full((k,), -1, dtype=torch.int32, device=cuda),
           torch.zeros(k, dtype=torch.float32, device=cuda)]
    a = _args(x, gw, buf, E, h, I, k, *got)  # no workspace
    st = capi.lib().wr_fused_moe_noalloc(ctypes.byref(a), stream)
    assert st == capi.WR_OK, capi.status_str(st)
    nws = capi.lib().wr_workspace_bytes(capi.WR_KIND_FUSED, E, h, I, k, 1)
    work = torch.empty(nws, dtype=torch.uint8, device=cuda)
    want = [torch.empty_like(x), torch.empty(k, dtype=torch.int32, device=cuda),
            torch.empty(k, dtype=torch.float32, device=cuda)]
    st = capi.lib().wr_fused_moe(ctypes.byref(_args(x, gw, buf, E, h, I, k, *want, work=work)),
                                 stream)
    assert st == capi.WR_OK, capi.status_str(st)
    torch.cuda.synchronize()
    return (x, gw, buf), got, want


def test_noalloc_matches_fused_on_two_calls(cuda):
    big = (8, 4096, 14336, 2, torch.float16)   # Mixtral: 148,480 bytes of the 1 MiB
    small = (16, 512, 256, 4, torch.float16)   # smaller layer, second call
    fp8 = (64, 2048, 1408, 6, torch.float8_e4m3fn)
    for i, shape in enumerate((big, small, fp8, big)):
        print(f"[gpu] noalloc call {i}: {shape}", flush=True)
        (x, gw, buf), got, want = _run_pair(cuda, shape, seed=30 + i)
        for g, w, what in zip(got, want, ("out", "ids", "weights")):
            assert torch.equal(g, w), f"call {i} {shape}: {what} differs from wr_fused_moe"
        E, h, I, k, _ = shape
        ref = oracle_token(x, gw, buf, E, h, I, k, True)
        np.testing.assert_allclose(f64(got[0]), ref["out"], rtol=1e-2, atol=1e-2)
        del buf
        torch.cuda.empty_cache()


def test_noalloc_rejects_problems_over_its_scratch(cuda):
    """k * roundup(I, 16) * 4 bytes of act plus the control block and logits
    must fit WR_NOALLOC_SCRATCH_BYTES; k = 6, I = 65536 needs 1.6 MB."""
    E, h, I, k = 8, 64, 65536, 6
    need = capi.lib().wr_workspace_bytes(capi.WR_KIND_FUSED, E, h, I, k, 1)
    assert need > capi.WR_NOALLOC_SCRATCH_BYTES
    t = torch.empty(16, device=cuda)
    a = _args(t, t, t, E, h, I, k, t, t.view(torch.int32), t)
    a.weight_bytes = 1 << 40  # pass the size check; the scratch check comes first anyway
    st = capi.lib().wr_fused_moe_noalloc(ctypes.byref(a), None)
    assert st == capi.WR_EINVAL_SCRATCH, capi.status_str(st)


def test_noalloc_call_captured_in_a_graph(cuda):
    """wr_fused_moe_noalloc recorded into a HIP graph (torch.cuda.graph on its
    capture stream) after a first eager call on the GPU (which looks up the
    scratch array's address; the captured call then makes no HIP call but the
    launch).  Each replay, with new x values copied into the captured input
    and eager calls of the same entry point between replays, equals
    wr_fused_moe on a caller workspace bit for bit."""
    E, h, I, k, wd = 64, 2048, 1408, 6, torch.float16
    x, gw, buf = make_layer(E, h, I, wd, router_std=h ** -0.5, seed=40, device=cuda,
                            gen_device=cuda)
    out = torch.empty_like(x)
    ids = torch.empty(k, dtype=torch.int32, device=cuda)
    ws = torch.empty(k, dtype=torch.float32, device=cuda)
    a = _args(x, gw, buf, E, h, I, k, out, ids, ws)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert capi.lib().wr_fused_moe_noalloc(ctypes.byref(a), stream) == capi.WR_OK
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cs = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        st = capi.lib().wr_fused_moe_noalloc(ctypes.byref(a), cs)
    assert st == capi.WR_OK, capi.status_str(st)
    nws = capi.lib().wr_workspace_bytes(capi.WR_KIND_FUSED, E, h, I, k, 1)
    work = torch.empty(nws, dtype=torch.uint8, device=cuda)
    gen = torch.Generator(device="cpu").manual_seed(41)
    for rep in range(4):
        print(f"[gpu] noalloc graph replay {rep}", flush=True)
        x.copy_(torch.randn(h, generator=gen).to(cuda))
        g.replay()
        torch.cuda.synchronize()
        got = (out.clone(), ids.clone(), ws.clone())
        want = (torch.empty_like(x), torch.empty_like(ids), torch.empty_like(ws))
        st = capi.lib().wr_fused_moe(
            ctypes.byref(_args(x, gw, buf, E, h, I, k, *want, work=work)), stream)
        assert st == capi.WR_OK, capi.status_str(st)
        # an eager call of the entry point between replays (other outputs)
        other = (torch.empty_like(x), torch.empty_like(ids), torch.empty_like(ws))
        xo = -x
        st = capi.lib().wr_fused_moe_noalloc(
            ctypes.byref(_args(xo, gw, buf, E, h, I, k, *other)), stream)
        assert st == capi.WR_OK, capi.status_str(st)
        torch.cuda.synchronize()
        for gv, wv, what in zip(got, want, ("out", "ids", "weights")):
            assert torch.equal(gv, wv), f"replay {rep}: {what} differs from wr_fused_moe"
    del g, buf
    torch.cuda.empty_cache()
