"""GPU parity at the reference's own test shapes and with its data recipe.

* tests/test_correctness.cu:46-48,74-87,160-166 sweeps E in {8, 16, 64},
  h in {4096, 8192}, I in {14336, 28672} and k in {1, 2}, with router
  N(0, 0.02), hidden N(0, 0.1) and experts N(0, 0.01), and compares the naive
  and fused ops.  Here, six points of that grid at full size with fp16
  weights (11.3 to 45.1 GB per layer, drawn on the GPU), each through the
  fused and naive ops against the fp64 oracle; one of them also through the
  batched op.
* tests/test_python.py:42-57,116-125 and tests/test_batched.py:9-24,72-79
  build fp32 layers from per-expert tensors packed with _pack_expert_weights:
  hidden x 0.1 and router x 0.02 from seed 42, experts x 0.01 from seed 43
  (seed 42 for everything in the batched test), at (8, 256, 512),
  (8, 512, 1024), (16, 256, 512) with k = 1 and 2, (8, 1024, 2048, 2) and
  (16, 512, 1024, 2).  Here the same shapes, scales and seeds through the
  fused, naive and batched ops against the oracle.  The draws come from a CPU
  torch.Generator, not the reference's CUDA generator, so the numbers differ
  from the reference's while following its recipe.

The bar is the parity bar of the other GPU tests: ids bit-exact (the margin
guard decides robustness on the CPU before anything runs), gate weights to
1e-5, outputs within rtol = atol = 1e-2 and within 1e-4 of max|ref|.  With
this recipe the outputs are small (about 1e-3), so the relative bound is the
one that binds.
"""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests._helpers import assert_parity, f64, oracle_rows, oracle_token

from warp_route import functional as F
from warp_route.synthetic import make_layer

pytestmark = pytest.mark.gpu

F32, F16 = torch.float32, torch.float16

# (E, h, I, k): points of the reference's sweep (tests/test_correctness.cu:160-166).
SWEEP = [(8, 8192, 28672, 1), (8, 8192, 28672, 2), (64, 8192, 14336, 1),
         (16, 4096, 28672, 2), (16, 8192, 14336, 2), (64, 4096, 28672, 2)]


def sweep_layer(E, h, I, k, device):
    """The sweep's recipe with fp16 weights, drawn on the GPU: the first seed
    whose selection passes the margin guard (decided from x and the router,
    which make_layer draws first, before the multi-GB experts are drawn)."""
    for seed in range(30):
        gen = torch.Generator(device=device).manual_seed(seed)
        x = torch.randn(h, generator=gen, device=device) * 0.1
        gw = torch.randn(E, h, generator=gen, device=device) * 0.02
        if O.selection_is_robust(f64(gw), f64(x), k):
            break
    else:
        raise AssertionError("no robust seed")
    x0, gw0, buf = make_layer(E, h, I, F16, router_std=0.02, expert_std=0.01, seed=seed,
                              device=device, gen_device=device)
    assert torch.equal(gw0, gw) and torch.equal(x0 * 0.1, x)
    return x.contiguous(), gw, buf, seed


@pytest.mark.parametrize("shape", SWEEP, ids=[f"E{e}-h{h}-I{i}-k{k}" for e, h, i, k in SWEEP])
def test_reference_sweep_shapes(cuda, shape):
    E, h, I, k = shape
    x, gw, buf, seed = sweep_layer(E, h, I, k, cuda)
    print(f"[gpu] sweep E={E} h={h} I={I} k={k} fp16 seed={seed}", flush=True)
    ref = oracle_token(x, gw, buf, E, h, I, k, False)
    for op, fn in (("fused", F.fused_moe), ("naive", F.naive_moe)):
        ids = torch.empty(k, dtype=torch.int32, device=cuda)
        ws = torch.empty(k, dtype=torch.float32, device=cuda)
        out = fn(x, gw, buf, E, h, I, k, False, ids, ws)
        torch.cuda.synchronize()
        assert_parity(out, ids, ws, ref, label=f"sweep {shape} {op}")
    if shape == (8, 8192, 28672, 2):
        # four tokens through the batched op: the sweep token and three more
        gen = torch.Generator(device="cpu").manual_seed(seed + 100)
        xs = torch.cat([x[None], 0.1 * torch.randn(3, h, generator=gen).to(cuda)]).contiguous()
        ids = torch.empty(4, k, dtype=torch.int32, device=cuda)
        ws = torch.empty(4, k, dtype=torch.float32, device=cuda)
        out = F.batched_fused_moe(xs, gw, buf, E, h, I, k, False, ids, ws)
        torch.cuda.synchronize()
        rows = oracle_rows(xs, gw, buf, E, h, I, k, False)
        assert rows[0]["robust"]
        for b in range(4):
            if rows[b]["robust"]:
                assert_parity(out[b], ids[b], ws[b], rows[b], label=f"sweep batched row {b}")
    del buf
    torch.cuda.empty_cache()


def reference_recipe_layer(E, h, I, B=None, seed=42, expert_seed=43, device="cpu"):
    """tests/test_python.py:42-57 (B None) or tests/test_batched.py:9-24 (B
    tokens, one seed for everything): hidden x 0.1 and router x 0.02 from
    `seed`; per-expert gate, up and down tensors x 0.01 from `expert_seed`
    (gate list, then up list, then down list); packed in fp32 with
    _pack_expert_weights (warp_route/functional.py:21-57)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(h if B is None else (B, h), generator=g) * 0.1
    gw = torch.randn(E, h, generator=g) * 0.02
    if expert_seed is not None:
        g = torch.Generator(device="cpu").manual_seed(expert_seed)
    gate = [torch.randn(I, h, generator=g) * 0.01 for _ in range(E)]
    up = [torch.randn(I, h, generator=g) * 0.01 for _ in range(E)]
    down = [torch.randn(h, I, generator=g) * 0.01 for _ in range(E)]
    buf = F._pack_expert_weights(gate, up, down, E, h, I)
    return x.to(device), gw.to(device), buf.to(device)


# tests/test_python.py:116-125 (E, h, I, k)
PY_CONFIGS = [(8, 256, 512, 1), (8, 256, 512, 2), (8, 512, 1024, 1), (8, 512, 1024, 2),
              (16, 256, 512, 1), (16, 256, 512, 2), (8, 1024, 2048, 2)]


@pytest.mark.parametrize("cfg", PY_CONFIGS, ids=[f"E{e}-h{h}-I{i}-k{k}" for e, h, i, k in PY_CONFIGS])
def test_reference_python_recipe(cuda, cfg):
    """fused, naive and (one token) batched against the oracle on the
    reference's own Python-test layers."""
    E, h, I, k = cfg
    x, gw, buf = reference_recipe_layer(E, h, I, device=cuda)
    ref = oracle_token(x, gw, buf, E, h, I, k, False)
    print(f"[gpu] reference python recipe {cfg} robust={ref['robust']}", flush=True)
    for op, fn in (("fused", F.fused_moe), ("naive", F.naive_moe)):
        ids = torch.empty(k, dtype=torch.int32, device=cuda)
        ws = torch.empty(k, dtype=torch.float32, device=cuda)
        out = fn(x, gw, buf, E, h, I, k, False, ids, ws)
        torch.cuda.synchronize()
        assert_parity(out, ids, ws, ref, label=f"python recipe {cfg} {op}")
    ids = torch.empty(1, k, dtype=torch.int32, device=cuda)
    ws = torch.empty(1, k, dtype=torch.float32, device=cuda)
    out = F.batched_fused_moe(x[None].contiguous(), gw, buf, E, h, I, k, False, ids, ws)
    torch.cuda.synchronize()
    assert_parity(out[0], ids[0], ws[0], ref, label=f"python recipe {cfg} batched")


# tests/test_batched.py:72-79: (E, h, I, k) at batch 1, 4, 16, 64
BATCHED_CONFIGS = [(8, 256, 512, 1), (8, 256, 512, 2), (16, 512, 1024, 2)]


@pytest.mark.parametrize("B", [1, 4, 16, 64])
@pytest.mark.parametrize("cfg", BATCHED_CONFIGS,
                         ids=[f"E{e}-h{h}-I{i}-k{k}" for e, h, i, k in BATCHED_CONFIGS])
def test_reference_batched_recipe(cuda, cfg, B):
    """The reference's batched test (every row against a loop of single-token
    fused calls) on its own recipe, plus every robust row against the oracle."""
    E, h, I, k = cfg
    x, gw, buf = reference_recipe_layer(E, h, I, B=B, seed=42, expert_seed=None, device=cuda)
    print(f"[gpu] reference batched recipe {cfg} B={B}", flush=True)
    ids = torch.empty(B, k, dtype=torch.int32, device=cuda)
    ws = torch.empty(B, k, dtype=torch.float32, device=cuda)
    out = F.batched_fused_moe(x, gw, buf, E, h, I, k, False, ids, ws)
    torch.cuda.synchronize()
    rows = oracle_rows(x, gw, buf, E, h, I, k, False)
    robust = 0
    for b in range(B):
        single = F.fused_moe(x[b].contiguous(), gw, buf, E, h, I, k)
        torch.cuda.synchronize()
        # tests/test_batched.py:49-56: cosine > 0.999 and mean abs error < 1e-2 of max|ref|
        a, c = f64(single), f64(out[b])
        cos = float(a @ c / (np.linalg.norm(a) * np.linalg.norm(c)))
        assert cos > 0.999 and np.abs(a - c).mean() < 1e-2 * np.abs(a).max(), (b, cos)
        if rows[b]["robust"]:
            assert_parity(out[b], ids[b], ws[b], rows[b], label=f"batched recipe {cfg} row {b}")
            robust += 1
    assert robust >= max(1, (3 * B) // 4), f"only {robust} of {B} rows robust"
