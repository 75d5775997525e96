"""Checkpoint -> expert_layout converter for local safetensors checkpoints.

The reference's only weight producer is ``_pack_expert_weights``
(warp_route/functional.py:21-57), fed from ``MoELayer``'s parameters
(warp_route/__init__.py:34-60, packed at :81).  This module reads the MoE
layers of a checkpoint on disk into the same packed buffers, one layer at a
time, without holding more than one expert matrix on the host at once:

    spec = read_spec("/models/Mixtral-8x7B")          # config.json
    gate_w, buf = load_layer("/models/Mixtral-8x7B", 0, spec, device="cuda")
    y = fused_moe(x, gate_w, buf, spec.num_experts, spec.hidden_dim,
                  spec.intermediate_dim, spec.top_k, spec.renormalize)

Supported layouts (tensor names as the Hugging Face checkpoints store them):

  mixtral    model.layers.{l}.block_sparse_moe.gate.weight       [E, h]
             ...experts.{e}.w1.weight (gate) / w3.weight (up)    [I, h]
             ...experts.{e}.w2.weight (down)                     [h, I]
  deepseek   model.layers.{l}.mlp.gate.weight                    [E, h]
  qwen2_moe  ...mlp.experts.{e}.gate_proj / up_proj .weight      [I, h]
             ...mlp.experts.{e}.down_proj.weight                 [h, I]
  dbrx       transformer.blocks.{l}.ffn.router.layer.weight      [E, h]
             ...ffn.experts.mlp.w1 (gate) / v1 (up)              [E*I, h]
             ...ffn.experts.mlp.w2, expert e's rows e*I..(e+1)*I [E*I, h]
             hold down_e transposed (the module computes act @ w2_e)
  warp_route a state dict of warp_route.MoELayer (router, gate_proj.{e},
             up_proj.{e}, down_proj.{e}), optionally under a name prefix

Only the routed experts and the router are converted.  Shared experts
(DeepSeek-MoE, Qwen2-MoE) are a dense FFN the caller adds to the layer output;
dense layers (DeepSeek's first layer) have no MoE block and are not listed in
``spec.moe_layers``.  Paths are local; nothing is fetched.
"""
from __future__ import annotations

import dataclasses
import json
import os
from typing import Dict, Iterator, List, Optional, Sequence, Tuple

import torch

from .functional import MAX_EXPERTS, MAX_TOPK, expert_layout

__all__ = ["MoESpec", "read_spec", "tensor_index", "load_layer", "load_layers", "save_packed",
           "load_packed", "ARCHS"]

ARCHS = ("mixtral", "deepseek", "qwen2_moe", "dbrx", "warp_route")
PACKED_FORMAT = "warp_route.expert_layout.v1"


@dataclasses.dataclass(frozen=True)
class MoESpec:
    """Shape and routing of a checkpoint's MoE layers."""
    arch: str
    num_experts: int
    hidden_dim: int
    intermediate_dim: int
    top_k: int
    renormalize: bool
    moe_layers: Tuple[int, ...]
    prefix: str = ""  # warp_route state dicts only: name prefix of the layer

    def to_json(self) -> str:
        d = dataclasses.asdict(self)
        d["moe_layers"] = list(self.moe_layers)
        return json.dumps(d, sort_keys=True)

    @staticmethod
    def from_json(s: str) -> "MoESpec":
        d = json.loads(s)
        d["moe_layers"] = tuple(d["moe_layers"])
        return MoESpec(**d)


def _check_spec(spec: MoESpec) -> MoESpec:
    if spec.arch not in ARCHS:
        raise ValueError(f"unknown arch {spec.arch!r}; expected one of {ARCHS}")
    if min(spec.num_experts, spec.hidden_dim, spec.intermediate_dim) < 1:
        raise ValueError(f"non-positive MoE dimensions in {spec}")
    if spec.num_experts > MAX_EXPERTS:
        raise ValueError(f"{spec.num_experts} experts exceed the router limit of {MAX_EXPERTS}")
    if not 1 <= spec.top_k <= min(MAX_TOPK, spec.num_experts):
        raise ValueError(f"top_k={spec.top_k} outside [1, min({MAX_TOPK}, {spec.num_experts})]")
    return spec


def read_spec(path: str, arch: Optional[str] = None) -> MoESpec:
    """MoESpec from the ``config.json`` in directory ``path`` (or the file
    ``path`` itself).  ``arch`` overrides the detection from ``model_type``."""
    cfg_path = path if os.path.isfile(path) else os.path.join(path, "config.json")
    with open(cfg_path, "r", encoding="utf-8") as f:
        cfg = json.load(f)
    mt = arch or cfg.get("model_type", "")
    if mt == "mixtral":
        n = int(cfg["num_hidden_layers"])
        spec = MoESpec("mixtral", int(cfg["num_local_experts"]), int(cfg["hidden_size"]),
                       int(cfg["intermediate_size"]), int(cfg["num_experts_per_tok"]),
                       True, tuple(range(n)))
    elif mt in ("deepseek", "qwen2_moe"):
        n = int(cfg["num_hidden_layers"])
        if mt == "deepseek":
            ne = int(cfg["n_routed_experts"])
            if cfg.get("scoring_func", "softmax") != "softmax":
                raise ValueError(f"scoring_func {cfg['scoring_func']!r}: only softmax routing")
            first = int(cfg.get("first_k_dense_replace", 0))
            freq = int(cfg.get("moe_layer_freq", 1))
            layers = tuple(l for l in range(n) if l >= first and l % freq == 0)
        else:
            ne = int(cfg["num_experts"])
            dense = set(cfg.get("mlp_only_layers", []))
            step = int(cfg.get("decoder_sparse_step", 1))
            layers = tuple(l for l in range(n) if l not in dense and (l + 1) % step == 0)
        spec = MoESpec(mt, ne, int(cfg["hidden_size"]), int(cfg["moe_intermediate_size"]),
                       int(cfg["num_experts_per_tok"]), bool(cfg.get("norm_topk_prob", False)),
                       layers)
    elif mt == "dbrx":
        ffn = cfg["ffn_config"]
        p = ffn.get("moe_normalize_expert_weights", 1)
        if p not in (None, 1, 1.0):
            raise ValueError(f"moe_normalize_expert_weights={p}: only the sum (p=1) or none")
        spec = MoESpec("dbrx", int(ffn["moe_num_experts"]), int(cfg["d_model"]),
                       int(ffn["ffn_hidden_size"]), int(ffn["moe_top_k"]), p is not None,
                       tuple(range(int(cfg["n_layers"]))))
    else:
        raise ValueError(f"unsupported model_type {mt!r}; pass arch= one of {ARCHS}")
    return _check_spec(spec)


def tensor_index(path: str) -> Dict[str, str]:
    """Tensor name -> safetensors file, from ``model.safetensors.index.json``
    when present, else from the headers of every ``*.safetensors`` file in
    ``path`` (or of the file ``path``)."""
    from safetensors import safe_open

    if os.path.isfile(path):
        files = [path]
        root = os.path.dirname(path)
    else:
        root = path
        idx = os.path.join(path, "model.safetensors.index.json")
        if os.path.isfile(idx):
            with open(idx, "r", encoding="utf-8") as f:
                wm = json.load(f)["weight_map"]
            return {k: os.path.join(root, v) for k, v in wm.items()}
        files = sorted(os.path.join(path, f) for f in os.listdir(path)
                       if f.endswith(".safetensors"))
    if not files:
        raise FileNotFoundError(f"no .safetensors files under {path}")
    out: Dict[str, str] = {}
    for fn in files:
        with safe_open(fn, framework="pt") as f:
            for k in f.keys():
                out[k] = fn
    return out


class _Reader:
    """Opens each safetensors file once and reads tensors by name."""

    def __init__(self, index: Dict[str, str]) -> None:
        self.index = index
        self._open: Dict[str, object] = {}

    def _file(self, name: str):
        from safetensors import safe_open

        fn = self.index.get(name)
        if fn is None:
            raise KeyError(f"tensor {name!r} not in the checkpoint")
        f = self._open.get(fn)
        if f is None:
            f = safe_open(fn, framework="pt")
            self._open[fn] = f
        return f

    def get(self, name: str) -> torch.Tensor:
        return self._file(name).get_tensor(name)

    def shape(self, name: str) -> Tuple[int, ...]:
        return tuple(self._file(name).get_slice(name).get_shape())

    def rows(self, name: str, r0: int, r1: int) -> torch.Tensor:
        """Rows [r0, r1) of a 2-D tensor, reading only those bytes."""
        return self._file(name).get_slice(name)[r0:r1]


def _names(spec: MoESpec, layer: int) -> Dict[str, str]:
    if spec.arch == "mixtral":
        b = f"model.layers.{layer}.block_sparse_moe."
        return {"router": b + "gate.weight", "gate": b + "experts.{e}.w1.weight",
                "up": b + "experts.{e}.w3.weight", "down": b + "experts.{e}.w2.weight"}
    if spec.arch in ("deepseek", "qwen2_moe"):
        b = f"model.layers.{layer}.mlp."
        return {"router": b + "gate.weight", "gate": b + "experts.{e}.gate_proj.weight",
                "up": b + "experts.{e}.up_proj.weight", "down": b + "experts.{e}.down_proj.weight"}
    if spec.arch == "dbrx":
        b = f"transformer.blocks.{layer}.ffn."
        return {"router": b + "router.layer.weight", "gate": b + "experts.mlp.w1",
                "up": b + "experts.mlp.v1", "down": b + "experts.mlp.w2"}
    p = spec.prefix
    return {"router": p + "router", "gate": p + "gate_proj.{e}", "up": p + "up_proj.{e}",
            "down": p + "down_proj.{e}"}


def _expert_mats(rd: _Reader, spec: MoESpec, names: Dict[str, str],
                 e: int) -> Iterator[Tuple[str, torch.Tensor]]:
    """(which, matrix) for expert e: gate [I, h], up [I, h], down [h, I]."""
    E, h, I = spec.num_experts, spec.hidden_dim, spec.intermediate_dim
    if spec.arch == "dbrx":
        for which in ("gate", "up", "down"):
            shp = rd.shape(names[which])
            if shp != (E * I, h):
                raise ValueError(f"{names[which]}: expected [{E * I}, {h}], got {list(shp)}")
            m = rd.rows(names[which], e * I, (e + 1) * I)
            yield which, (m.t() if which == "down" else m)
        return
    want = {"gate": (I, h), "up": (I, h), "down": (h, I)}
    for which in ("gate", "up", "down"):
        name = names[which].format(e=e)
        t = rd.get(name)
        if tuple(t.shape) != want[which]:
            raise ValueError(f"{name}: expected {list(want[which])}, got {list(t.shape)}")
        yield which, t


def _pack_layer(rd: _Reader, spec: MoESpec, layer: int, dtype: torch.dtype,
                device) -> Tuple[torch.Tensor, torch.Tensor]:
    if dtype not in (torch.float32, torch.float16):
        raise ValueError(f"dtype must be torch.float32 or torch.float16, got {dtype}")
    E, h, I = spec.num_experts, spec.hidden_dim, spec.intermediate_dim
    names = _names(spec, layer)
    router = rd.get(names["router"])
    if tuple(router.shape) != (E, h):
        raise ValueError(f"{names['router']}: expected [{E}, {h}], got {list(router.shape)}")
    gate_w = router.to(device=device, dtype=torch.float32).contiguous()
    es = torch.empty((), dtype=dtype).element_size()
    off = expert_layout(E, h, I, es)
    stride = off["expert_stride"] // es
    start = {"gate": off["gate_proj_offset"] // es, "up": off["up_proj_offset"] // es,
             "down": off["down_proj_offset"] // es}
    buf = torch.zeros(E * stride, dtype=dtype, device=device)
    n = I * h
    for e in range(E):
        for which, m in _expert_mats(rd, spec, names, e):
            src = m.to(device=device).to(dtype)
            if not bool(torch.isfinite(src).all()):
                raise ValueError(f"layer {layer} expert {e} {which}: values not finite in {dtype}")
            base = e * stride + start[which]
            buf[base:base + n].view(m.shape[0], m.shape[1]).copy_(src)
    return gate_w, buf


def load_layer(path: str, layer: int, spec: Optional[MoESpec] = None,
               dtype: torch.dtype = torch.float16, device="cpu",
               index: Optional[Dict[str, str]] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """(gate_w [E, h] fp32, packed expert buffer) of MoE layer ``layer``.

    Expert matrices are cast to ``dtype`` (float16 or float32) and packed in
    the expert layout: per expert [gate I x h][up I x h][down h x I], the
    expert stride rounded up to 128 bytes, padding zero.  Raises ValueError
    for a tensor of the wrong shape or a value that does not fit ``dtype``
    (an fp16 overflow), KeyError for a missing tensor."""
    spec = _check_spec(spec or read_spec(path))
    if layer not in spec.moe_layers:
        raise ValueError(f"layer {layer} is not an MoE layer of this checkpoint "
                         f"(MoE layers: {list(spec.moe_layers)})")
    rd = _Reader(index or tensor_index(path))
    return _pack_layer(rd, spec, layer, dtype, device)


def load_layers(path: str, layers: Optional[Sequence[int]] = None,
                spec: Optional[MoESpec] = None, dtype: torch.dtype = torch.float16,
                device="cpu") -> List[Tuple[torch.Tensor, torch.Tensor]]:
    """``load_layer`` for each of ``layers`` (default: every MoE layer), in
    order; the result feeds ``warp_route.stack.MoEStack``."""
    spec = _check_spec(spec or read_spec(path))
    idx = tensor_index(path)
    rd = _Reader(idx)
    out = []
    for l in (spec.moe_layers if layers is None else layers):
        if l not in spec.moe_layers:
            raise ValueError(f"layer {l} is not an MoE layer of this checkpoint")
        out.append(_pack_layer(rd, spec, l, dtype, device))
    return out


def save_packed(out_file: str, spec: MoESpec, layers: Sequence[int],
                packed: Sequence[Tuple[torch.Tensor, torch.Tensor]]) -> None:
    """Write converted layers to one safetensors file: ``layer.{l}.gate_w``
    and ``layer.{l}.weight_buf`` per layer, the spec and layout in the
    header's metadata."""
    from safetensors.torch import save_file

    if len(layers) != len(packed):
        raise ValueError("one (gate_w, weight_buf) pair per layer")
    tensors = {}
    dtypes = set()
    for l, (gw, buf) in zip(layers, packed):
        tensors[f"layer.{l}.gate_w"] = gw.detach().to("cpu").contiguous()
        tensors[f"layer.{l}.weight_buf"] = buf.detach().to("cpu").contiguous()
        dtypes.add(str(buf.dtype))
    if len(dtypes) > 1:
        raise ValueError(f"mixed weight dtypes {sorted(dtypes)}")
    meta = {"format": PACKED_FORMAT, "spec": spec.to_json(),
            "layers": json.dumps(list(layers)), "weight_dtype": dtypes.pop()}
    save_file(tensors, out_file, metadata=meta)


def load_packed(in_file: str, device="cpu"
                ) -> Tuple[MoESpec, List[int], List[Tuple[torch.Tensor, torch.Tensor]]]:
    """Read a file written by ``save_packed``: (spec, layer numbers, layers)."""
    from safetensors import safe_open

    with safe_open(in_file, framework="pt") as f:
        meta = f.metadata() or {}
        if meta.get("format") != PACKED_FORMAT:
            raise ValueError(f"{in_file}: not a {PACKED_FORMAT} file")
        spec = _check_spec(MoESpec.from_json(meta["spec"]))
        layers = [int(l) for l in json.loads(meta["layers"])]
        out = []
        for l in layers:
            gw = f.get_tensor(f"layer.{l}.gate_w").to(device)
            buf = f.get_tensor(f"layer.{l}.weight_buf").to(device)
            es = buf.element_size()
            need = spec.num_experts * expert_layout(spec.num_experts, spec.hidden_dim,
                                                    spec.intermediate_dim, es)["expert_stride"]
            if buf.numel() * es != need or tuple(gw.shape) != (spec.num_experts, spec.hidden_dim):
                raise ValueError(f"{in_file}: layer {l} does not match its spec")
            out.append((gw, buf))
    return spec, layers, out
