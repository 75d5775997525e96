"""Writes tests/golden/toy_golden.json: the BASELINE toy config (h=256,
I=512, E=8, k=2, fp32, seed 0, reference routing without renormalisation)
run through the CPU oracle.

The reference ships no golden vectors (its tests are differential only), so
this fixture records the oracle's own answer on the generator's inputs; the
oracle itself is pinned by tests/test_oracle.py.  Weights are not stored:
they are regenerated from the seed, and the fixture keeps their SHA-256 so
that a change of random generator is detected rather than silently absorbed.

Usage: python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "warp-route_amd")]

import numpy as np  # noqa: E402

from oracle import moe_oracle as O  # noqa: E402
from warp_route.synthetic import CONFIGS, make_config_layer  # noqa: E402


def sha256(t) -> str:
    return hashlib.sha256(t.contiguous().cpu().numpy().tobytes()).hexdigest()


def compute():
    cfg = CONFIGS["toy"]
    x, gw, buf = make_config_layer(cfg, seed=0)
    r = O.moe_forward(x.numpy(), gw.numpy(), buf.numpy(), cfg.num_experts, cfg.hidden_dim,
                      cfg.intermediate_dim, cfg.top_k, cfg.renormalize)
    return {
        "config": {"num_experts": cfg.num_experts, "hidden_dim": cfg.hidden_dim,
                   "intermediate_dim": cfg.intermediate_dim, "top_k": cfg.top_k,
                   "renormalize": cfg.renormalize, "weight_dtype": "float32", "seed": 0},
        "sha256": {"x": sha256(x), "gate_w": sha256(gw), "weight_buf": sha256(buf)},
        "logits": [float(v) for v in r["logits64"]],
        "probs": [float(v) for v in r["probs"]],
        "ids": [int(v) for v in r["ids"]],
        "weights": [float(v) for v in r["weights"]],
        "out": [float(v) for v in r["out"]],
    }


if __name__ == "__main__":
    with open(os.path.join(HERE, "toy_golden.json"), "w") as f:
        json.dump(compute(), f, indent=1)
    print("wrote toy_golden.json")
