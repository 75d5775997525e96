"""Checkpoint converter (warp_route.convert): synthetic Hugging Face-style
checkpoints in bf16, written here with safetensors, converted to the expert
layout and checked two ways:

* the packed buffer holds each expert's matrices, bit for bit (the oracle's
  expert views of the flat layout, src/expert_layout.cuh:50-71);
* the oracle's layer on the converted buffers equals each architecture's own
  MoE block, restated below in fp64 straight from the checkpoint tensors
  (softmax router, top-k, optional renormalisation, SwiGLU experts: the
  Mixtral / DeepSeek / Qwen2-MoE / DBRX module definitions).  A planted
  mistake (gate and up swapped, DBRX's down not transposed) must fail it.
"""
import json
import os

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from oracle import moe_oracle as O

from warp_route import convert as C

from ._helpers import assert_parity, oracle_token


def _names(arch, l, e):
    if arch == "mixtral":
        b = f"model.layers.{l}.block_sparse_moe."
        return b + "gate.weight", [b + f"experts.{e}.{w}.weight" for w in ("w1", "w3", "w2")]
    b = f"model.layers.{l}.mlp."
    return b + "gate.weight", [b + f"experts.{e}.{w}_proj.weight" for w in ("gate", "up", "down")]


def make_checkpoint(root, arch, E, h, I, k, n_layers, seed=0, shards=1, **cfg_extra):
    """Write config.json and bf16 tensors; return {name: tensor}."""
    g = torch.Generator().manual_seed(seed)

    def rnd(*shape, std=0.05):
        return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)

    t = {}
    for l in range(n_layers):
        if arch == "dbrx":
            b = f"transformer.blocks.{l}.ffn."
            t[b + "router.layer.weight"] = rnd(E, h, std=h ** -0.5)
            for w in ("w1", "v1", "w2"):
                t[b + "experts.mlp." + w] = rnd(E * I, h)
            continue
        rname, _ = _names(arch, l, 0)
        t[rname] = rnd(E, h, std=h ** -0.5)
        for e in range(E):
            _, (gn, un, dn) = _names(arch, l, e)
            t[gn], t[un], t[dn] = rnd(I, h), rnd(I, h), rnd(h, I)
    if arch == "mixtral":
        cfg = {"model_type": "mixtral", "num_local_experts": E, "hidden_size": h,
               "intermediate_size": I, "num_experts_per_tok": k, "num_hidden_layers": n_layers}
    elif arch == "deepseek":
        cfg = {"model_type": "deepseek", "n_routed_experts": E, "hidden_size": h,
               "moe_intermediate_size": I, "num_experts_per_tok": k,
               "num_hidden_layers": n_layers, "norm_topk_prob": False}
    elif arch == "qwen2_moe":
        cfg = {"model_type": "qwen2_moe", "num_experts": E, "hidden_size": h,
               "moe_intermediate_size": I, "num_experts_per_tok": k,
               "num_hidden_layers": n_layers}
    else:
        cfg = {"model_type": "dbrx", "d_model": h, "n_layers": n_layers,
               "ffn_config": {"ffn_hidden_size": I, "moe_num_experts": E, "moe_top_k": k,
                              "moe_normalize_expert_weights": 1}}
    cfg.update(cfg_extra)
    os.makedirs(root, exist_ok=True)
    with open(os.path.join(root, "config.json"), "w") as f:
        json.dump(cfg, f)
    names = sorted(t)
    if shards == 1:
        save_file(t, os.path.join(root, "model.safetensors"))
    else:
        wm = {}
        for s in range(shards):
            fn = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
            part = {n: t[n] for n in names[s::shards]}
            save_file(part, os.path.join(root, fn))
            wm.update({n: fn for n in part})
        with open(os.path.join(root, "model.safetensors.index.json"), "w") as f:
            json.dump({"metadata": {}, "weight_map": wm}, f)
    return t


def module_forward(arch, t, l, x, E, I, k, renorm):
    """The architecture's MoE block in fp64, from the raw checkpoint tensors.

    Mixtral / DeepSeek / Qwen2-MoE experts: down @ (silu(gate @ x) * (up @ x))
    with (w1, w3, w2) or (gate_proj, up_proj, down_proj).  DBRX experts:
    (silu(x @ w1_e^T) * (x @ v1_e^T)) @ w2_e with w1, v1, w2 viewed as
    [E, I, h].  Routing: softmax over all experts, top-k, and for Mixtral,
    DBRX (p = 1) and norm_topk_prob the weights divided by their sum."""
    d = lambda a: a.to(torch.float64)
    xs = d(x)
    if arch == "dbrx":
        b = f"transformer.blocks.{l}.ffn."
        router = d(t[b + "router.layer.weight"])
        w1, v1, w2 = (d(t[b + "experts.mlp." + w]).view(E, I, -1) for w in ("w1", "v1", "w2"))
    else:
        rname, _ = _names(arch, l, 0)
        router = d(t[rname])
    p = torch.softmax(router @ xs, dim=0)
    w, ids = torch.topk(p, k)
    if renorm:
        w = w / w.sum()
    out = torch.zeros_like(xs)
    for kk in range(k):
        e = int(ids[kk])
        if arch == "dbrx":
            a = torch.nn.functional.silu(xs @ w1[e].T) * (xs @ v1[e].T)
            out += w[kk] * (a @ w2[e])
        else:
            _, (gn, un, dn) = _names(arch, l, e)
            a = torch.nn.functional.silu(d(t[gn]) @ xs) * (d(t[un]) @ xs)
            out += w[kk] * (d(t[dn]) @ a)
    return out.numpy(), ids.numpy()


SHAPES = {"mixtral": (8, 96, 160, 2), "deepseek": (16, 64, 48, 6), "qwen2_moe": (12, 64, 80, 4),
          "dbrx": (16, 96, 96, 4)}


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
@pytest.mark.parametrize("arch", list(SHAPES))
def test_converted_layer_equals_module(tmp_path, arch, dtype):
    E, h, I, k = SHAPES[arch]
    t = make_checkpoint(str(tmp_path), arch, E, h, I, k, n_layers=2, seed=3,
                        shards=2 if arch == "mixtral" else 1,
                        **({"norm_topk_prob": True} if arch == "qwen2_moe" else {}))
    spec = C.read_spec(str(tmp_path))
    assert (spec.arch, spec.num_experts, spec.hidden_dim, spec.intermediate_dim,
            spec.top_k) == (arch, E, h, I, k)
    assert spec.renormalize == (arch != "deepseek")
    layers = C.load_layers(str(tmp_path), dtype=dtype)
    assert len(layers) == 2
    g = torch.Generator().manual_seed(11)
    for l, (gw, buf) in enumerate(layers):
        assert gw.dtype == torch.float32 and buf.dtype == dtype
        bnp = buf.numpy()
        for e in range(E):
            gm, um, dm = O.expert_views(bnp, e, E, h, I)
            if arch == "dbrx":
                b = f"transformer.blocks.{l}.ffn.experts.mlp."
                want = [t[b + w][e * I:(e + 1) * I] for w in ("w1", "v1")]
                want.append(t[b + "w2"][e * I:(e + 1) * I].T)
            else:
                want = [t[n] for n in _names(arch, l, e)[1]]
            for got, w in zip((gm, um, dm), want):
                np.testing.assert_array_equal(got, w.to(dtype).numpy())
        checked = 0
        for _ in range(4):
            x = torch.randn(h, generator=g)
            ref, ids = module_forward(arch, t, l, x, E, I, k, spec.renormalize)
            r = O.moe_forward(x.numpy(), gw.numpy(), bnp, E, h, I, k, spec.renormalize)
            if not O.selection_is_robust(gw.numpy().astype(np.float64), x.numpy(), k):
                continue
            np.testing.assert_array_equal(r["ids"], ids)
            tol = 1e-9 if dtype == torch.float32 else 1e-6  # fp16 subnormal weights round
            assert np.abs(r["out"] - ref).max() <= tol * np.abs(ref).max()
            checked += 1
        assert checked >= 2


def test_planted_mistakes_are_caught(tmp_path):
    """Packing gate and up swapped, or DBRX's down untransposed, changes the
    layer by far more than the tolerance above."""
    E, h, I, k = SHAPES["dbrx"]
    t = make_checkpoint(str(tmp_path), "dbrx", E, h, I, k, n_layers=1, seed=4)
    b = "transformer.blocks.0.ffn.experts.mlp."
    f32 = {w: t[b + w].float().view(E, I, h) for w in ("w1", "v1", "w2")}
    gw = t["transformer.blocks.0.ffn.router.layer.weight"].float().numpy()
    right = O.pack_expert_weights([f32["w1"][e].numpy() for e in range(E)],
                                  [f32["v1"][e].numpy() for e in range(E)],
                                  [f32["w2"][e].T.numpy() for e in range(E)], E, h, I)
    swapped = O.pack_expert_weights([f32["v1"][e].numpy() for e in range(E)],
                                    [f32["w1"][e].numpy() for e in range(E)],
                                    [f32["w2"][e].T.numpy() for e in range(E)], E, h, I)
    untransposed = O.pack_expert_weights([f32["w1"][e].numpy() for e in range(E)],
                                         [f32["v1"][e].numpy() for e in range(E)],
                                         [f32["w2"][e].numpy() for e in range(E)], E, h, I)
    x = torch.randn(h, generator=torch.Generator().manual_seed(5))
    ref, _ = module_forward("dbrx", t, 0, x, E, I, k, True)
    scale = np.abs(ref).max()
    assert np.abs(O.moe_forward(x.numpy(), gw, right, E, h, I, k, True)["out"] - ref).max() \
        <= 1e-9 * scale
    for bad in (swapped, untransposed):
        assert np.abs(O.moe_forward(x.numpy(), gw, bad, E, h, I, k, True)["out"] - ref).max() \
            > 1e-2 * scale


def test_moe_layer_selection(tmp_path):
    ds = tmp_path / "ds"
    make_checkpoint(str(ds), "deepseek", 16, 32, 24, 2, n_layers=3, first_k_dense_replace=1)
    spec = C.read_spec(str(ds))
    assert spec.moe_layers == (1, 2)
    with pytest.raises(ValueError, match="not an MoE layer"):
        C.load_layer(str(ds), 0, spec)
    qw = tmp_path / "qw"
    make_checkpoint(str(qw), "qwen2_moe", 8, 32, 24, 2, n_layers=4, decoder_sparse_step=2,
                    mlp_only_layers=[3])
    assert C.read_spec(str(qw)).moe_layers == (1,)


def test_warp_route_state_dict(tmp_path):
    """A MoELayer state dict saved with safetensors converts to the same
    buffer as MoELayer's own packing."""
    from warp_route import MoELayer
    from warp_route.functional import _pack_expert_weights

    torch.manual_seed(0)
    m = MoELayer(4, 32, 48, 2)
    sd = {"moe." + n: p.detach().clone() for n, p in m.state_dict().items()}
    fn = str(tmp_path / "layer.safetensors")
    save_file(sd, fn)
    spec = C.MoESpec("warp_route", 4, 32, 48, 2, False, (0,), prefix="moe.")
    for dtype in (torch.float32, torch.float16):
        gw, buf = C.load_layer(fn, 0, spec, dtype=dtype)
        want = _pack_expert_weights(list(m.gate_proj), list(m.up_proj), list(m.down_proj), 4, 32,
                                    48, dtype=dtype)
        assert torch.equal(buf, want.detach())
        assert torch.equal(gw, m.router.detach())


def test_packed_file_round_trip(tmp_path):
    make_checkpoint(str(tmp_path / "ck"), "mixtral", 8, 32, 40, 2, n_layers=3)
    spec = C.read_spec(str(tmp_path / "ck"))
    layers = C.load_layers(str(tmp_path / "ck"), [0, 2])
    out = str(tmp_path / "packed.safetensors")
    C.save_packed(out, spec, [0, 2], layers)
    spec2, nums, back = C.load_packed(out)
    assert spec2 == spec and nums == [0, 2]
    for (a, b), (c, d) in zip(layers, back):
        assert torch.equal(a, c) and torch.equal(b, d) and d.dtype == torch.float16


def test_conversion_errors(tmp_path):
    root = str(tmp_path / "ck")
    t = make_checkpoint(root, "mixtral", 8, 32, 40, 2, n_layers=1)
    with pytest.raises(ValueError, match="unsupported model_type"):
        C.read_spec(root, arch="llama")
    with pytest.raises(ValueError, match="top_k"):
        C.load_layer(root, 0, C.MoESpec("mixtral", 8, 32, 40, 7, True, (0,)))
    with pytest.raises(ValueError, match="expected"):
        C.load_layer(root, 0, C.MoESpec("mixtral", 8, 32, 20, 2, True, (0,)))
    with pytest.raises(ValueError, match="dtype"):
        C.load_layer(root, 0, dtype=torch.int8)
    # a value beyond fp16's range
    big = dict(t)
    big["model.layers.0.block_sparse_moe.experts.3.w3.weight"] = torch.full(
        (40, 32), 1e6, dtype=torch.bfloat16)
    save_file(big, os.path.join(root, "model.safetensors"))
    with pytest.raises(ValueError, match="not finite"):
        C.load_layer(root, 0)
    C.load_layer(root, 0, dtype=torch.float32)  # fits fp32
    del big["model.layers.0.block_sparse_moe.experts.5.w2.weight"]
    save_file(big, os.path.join(root, "model.safetensors"))
    with pytest.raises(KeyError, match="experts.5.w2"):
        C.load_layer(root, 0, dtype=torch.float32)
    with pytest.raises(ValueError, match="not a warp_route"):
        C.load_packed(os.path.join(root, "model.safetensors"))


@pytest.mark.gpu
@pytest.mark.parametrize("arch", list(SHAPES))
def test_converted_layer_on_gpu(cuda, tmp_path, arch):
    """Converted fp16 layers of every architecture the converter reads
    (Mixtral, DeepSeek-MoE, Qwen2-MoE, DBRX) through the fused and batched
    ops, against the oracle on the converted weights."""
    from warp_route.functional import batched_fused_moe, fused_moe

    E, h, I, k = SHAPES[arch]
    make_checkpoint(str(tmp_path), arch, E, h, I, k, n_layers=1, seed=8)
    spec = C.read_spec(str(tmp_path))
    gw, buf = C.load_layer(str(tmp_path), 0, spec, dtype=torch.float16, device=cuda)
    g = torch.Generator().manual_seed(9)
    xs = torch.randn(4, h, generator=g).to(cuda)
    args = (gw, buf, E, h, I, k, spec.renormalize)
    yb = batched_fused_moe(xs, *args)
    robust = 0
    for b in range(4):
        ref = oracle_token(xs[b], gw, buf, E, h, I, k, spec.renormalize)
        if not ref["robust"]:
            continue
        robust += 1
        ids = torch.empty(k, dtype=torch.int32, device=cuda)
        ws = torch.empty(k, dtype=torch.float32, device=cuda)
        y = fused_moe(xs[b], *args, topk_ids=ids, topk_weights=ws)
        assert_parity(y, ids, ws, ref, label=f"{arch} token {b}")
        assert_parity(yb[b], None, None, ref, label=f"{arch} batched row {b}")
    assert robust >= 3, f"{arch}: only {robust} of 4 tokens route robustly"
