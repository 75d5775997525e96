"""Pins the CPU oracle (oracle/moe_oracle.py) with checks that do not retype
its formulas: hand-computed byte tables, exactly rounded sums (math.fsum),
scipy's softmax, brute-force sorting, constructed ties, pure-Python loops on
tiny shapes, identity / linearity / zero special cases, and torch's library
routines in the reference's own test formula (tests/test_python.py:15-37).
A planted-mistake test shows each check would catch a plausible error.
"""
import math

import numpy as np
import pytest
import scipy.special
import torch

from oracle import moe_oracle as O


# ---------------------------------------------------------------------------
# Layout (src/expert_layout.cuh:34-47, 74-77; warp_route/functional.py:21-57)
# ---------------------------------------------------------------------------
# (E, h, I, elem_bytes) -> (up_off, down_off, stride, total), computed by hand.
LAYOUT_TABLE = [
    ((8, 4096, 14336, 2), (117_440_512, 234_881_024, 352_321_536, 2_818_572_288)),
    ((64, 2048, 1408, 2), (5_767_168, 11_534_336, 17_301_504, 1_107_296_256)),
    ((16, 6144, 10752, 2), (132_120_576, 264_241_152, 396_361_728, 6_341_787_648)),
    ((8, 256, 512, 4), (524_288, 1_048_576, 1_572_864, 12_582_912)),
    # Padding cases: 3*5*4*3 = 180 bytes -> 256; 3*5*2*3 = 90 -> 128.
    ((2, 3, 5, 4), (60, 120, 256, 512)),
    ((2, 3, 5, 2), (30, 60, 128, 256)),
    ((1, 1, 1, 2), (2, 4, 128, 128)),
]


@pytest.mark.parametrize("args,want", LAYOUT_TABLE)
def test_layout_table(args, want):
    off = O.layout_offsets(*args)
    assert off["gate_proj_offset"] == 0
    assert (off["up_proj_offset"], off["down_proj_offset"], off["expert_stride"]) == want[:3]
    assert O.total_weight_bytes(*args) == want[3]


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_pack_round_trip_and_zero_padding(dtype):
    rng = np.random.default_rng(1)
    E, h, I = 3, 5, 7   # 3*35*elem bytes is not a multiple of 128: padding present
    g = [rng.standard_normal((I, h)).astype(dtype) for _ in range(E)]
    u = [rng.standard_normal((I, h)).astype(dtype) for _ in range(E)]
    d = [rng.standard_normal((h, I)).astype(dtype) for _ in range(E)]
    buf = O.pack_expert_weights(g, u, d, E, h, I, dtype)
    es = np.dtype(dtype).itemsize
    assert buf.nbytes == O.total_weight_bytes(E, h, I, es)
    for e in range(E):
        ge, ue, de = O.expert_views(buf, e, E, h, I)
        np.testing.assert_array_equal(ge, g[e])
        np.testing.assert_array_equal(ue, u[e])
        np.testing.assert_array_equal(de, d[e])
    stride_el = O.layout_offsets(E, h, I, es)["expert_stride"] // es
    for e in range(E):
        pad = buf[e * stride_el + 3 * I * h:(e + 1) * stride_el]
        assert pad.size > 0 and np.all(pad == 0)


# ---------------------------------------------------------------------------
# Router logits (src/fused_moe.cu:100-112)
# ---------------------------------------------------------------------------
def test_logits_match_exactly_rounded_sums():
    rng = np.random.default_rng(2)
    E, h = 5, 37
    w = rng.standard_normal((E, h))
    x = rng.standard_normal(h)
    got = O.router_logits(w, x)
    for e in range(E):
        exact = math.fsum(float(w[e, i]) * float(x[i]) for i in range(h))
        assert abs(got[e] - exact) <= 1e-12 * max(1.0, abs(exact))


def test_logit_error_bound_holds_for_fp32_sums():
    rng = np.random.default_rng(3)
    E, h = 8, 4096
    w = (rng.standard_normal((E, h)) / 64).astype(np.float32)
    x = rng.standard_normal(h).astype(np.float32)
    bound = O.logit_error_bound(w, x)
    exact = O.router_logits(w, x)
    # Two fp32 summation orders: sequential, and pairwise (numpy).
    for e in range(E):
        acc = np.float32(0)
        for i in range(h):
            acc = np.float32(acc + np.float32(w[e, i] * x[i]))
        assert abs(float(acc) - exact[e]) <= bound[e]
        pw = float(np.dot(w[e], x))
        assert abs(pw - exact[e]) <= bound[e]


# ---------------------------------------------------------------------------
# Softmax + top-K (src/naive_moe.cu:152-175)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("E,k", [(8, 1), (8, 2), (16, 4), (64, 6), (3, 3)])
def test_softmax_topk_against_scipy_and_brute_force(E, k):
    rng = np.random.default_rng(E * 10 + k)
    for _ in range(20):
        l = rng.standard_normal(E).astype(np.float32)
        probs, ids, ws = O.softmax_topk(l, k)
        np.testing.assert_allclose(probs, scipy.special.softmax(l.astype(np.float64)),
                                   rtol=2e-6, atol=1e-9)
        assert abs(float(np.sum(probs, dtype=np.float64)) - 1.0) < 1e-5
        brute = sorted(range(E), key=lambda e: (-float(probs[e]), e))[:k]
        assert list(ids) == brute
        np.testing.assert_array_equal(ws, probs[ids])
        _, ids_r, ws_r = O.softmax_topk(l, k, renormalize=True)
        assert list(ids_r) == brute
        np.testing.assert_allclose(ws_r, probs[ids] / np.sum(probs[ids]), rtol=1e-6)


def test_topk_order_matches_torch_topk_on_distinct_values():
    g = torch.Generator().manual_seed(5)
    for _ in range(20):
        l = torch.randn(16, generator=g)
        probs, ids, ws = O.softmax_topk(l.numpy(), 4)
        tw, ti = torch.topk(torch.softmax(l.double(), 0), 4)
        assert list(ids) == ti.tolist()
        np.testing.assert_allclose(ws, tw.numpy(), rtol=1e-6)


def test_all_equal_logits_give_uniform_probs_and_lowest_ids():
    for E in (4, 8, 16, 64):
        probs, ids, ws = O.softmax_topk(np.full(E, 0.75, np.float32), min(6, E))
        assert np.all(probs == np.float32(1.0 / E))   # exact for a power of two
        assert list(ids) == list(range(min(6, E)))


def test_duplicate_top_logits_pick_lower_index_first():
    l = np.array([0.1, 2.0, -1.0, 0.5, 2.0, 0.3], np.float32)
    _, ids, ws = O.softmax_topk(l, 3)
    assert list(ids) == [1, 4, 3]
    assert ws[0] == ws[1]


def test_nan_probability_is_never_selected():
    l = np.array([0.0, np.nan, 1.0, 0.5], np.float32)
    _, ids, _ = O.softmax_topk(l, 2)
    # max ignores NaN; the NaN expert's prob is NaN and fails the strict '>'.
    assert 1 not in list(ids)


def test_margin_guard():
    w = np.eye(4, dtype=np.float32)
    assert O.selection_is_robust(w, np.array([4.0, 3.0, 2.0, 1.0], np.float32), 2)
    assert not O.selection_is_robust(w, np.array([4.0, 3.0, 3.0, 1.0], np.float32), 2)
    assert O.topk_margin(np.array([4.0, 3.0, 1.0]), 2) == 2.0


# ---------------------------------------------------------------------------
# Expert FFN (tests/test_python.py:32-35)
# ---------------------------------------------------------------------------
def _ffn_loops(x, g, u, d):
    """Pure-Python restatement on tiny shapes, written independently."""
    I, h = len(g), len(x)
    act = []
    for r in range(I):
        gs = sum(g[r][i] * x[i] for i in range(h))
        us = sum(u[r][i] * x[i] for i in range(h))
        act.append(gs / (1.0 + math.exp(-gs)) * us)
    return [sum(d[o][j] * act[j] for j in range(I)) for o in range(h)]


def _tiny(seed, h=4, I=3):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(h), rng.standard_normal((I, h)), rng.standard_normal((I, h)),
            rng.standard_normal((h, I)))


def test_ffn_matches_pure_python_loops():
    for seed in range(5):
        x, g, u, d = _tiny(seed)
        want = _ffn_loops(x.tolist(), g.tolist(), u.tolist(), d.tolist())
        np.testing.assert_allclose(O.expert_ffn(x, g, u, d), want, rtol=1e-12, atol=1e-12)


def test_planted_mistakes_are_caught_by_the_loop_check():
    x, g, u, d = _tiny(11, h=4, I=4)
    want = np.array(_ffn_loops(x.tolist(), g.tolist(), u.tolist(), d.tolist()))
    wrong = [
        O.expert_ffn(x, u, g, d),                      # gate and up swapped
        O.expert_ffn(x, g, u, d.T),                    # down transposed
        d @ ((g @ x) * (u @ x)),                       # silu dropped
        O.expert_ffn(x, g, u, d) - d[:, 0] * 0.0 + 1e-3 * d[:, -1],  # extra term
    ]
    for w in wrong:
        assert not np.allclose(w, want, rtol=1e-6, atol=1e-9)


def test_ffn_identity_linearity_and_zero():
    rng = np.random.default_rng(7)
    n = 6
    x = rng.standard_normal(n)
    g = rng.standard_normal((n, n))
    u = rng.standard_normal((n, n))
    gv, uv = g @ x, u @ x
    want = gv / (1 + np.exp(-gv)) * uv
    np.testing.assert_allclose(O.expert_ffn(x, g, u, np.eye(n)), want, rtol=1e-13)
    d = rng.standard_normal((n, n))
    np.testing.assert_allclose(O.expert_ffn(x, g, u, 2.5 * d), 2.5 * O.expert_ffn(x, g, u, d),
                               rtol=1e-12)
    assert np.all(O.expert_ffn(np.zeros(n), g, u, d) == 0)


# ---------------------------------------------------------------------------
# Whole layer
# ---------------------------------------------------------------------------
def _toy_layer(seed=43, E=8, h=64, I=96):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(h, generator=g)
    gw = torch.randn(E, h, generator=g) * 0.3
    gp = [torch.randn(I, h, generator=g) * 0.05 for _ in range(E)]
    up = [torch.randn(I, h, generator=g) * 0.05 for _ in range(E)]
    dp = [torch.randn(h, I, generator=g) * 0.05 for _ in range(E)]
    buf = O.pack_expert_weights([t.numpy() for t in gp], [t.numpy() for t in up],
                                [t.numpy() for t in dp], E, h, I, np.float32)
    return x, gw, gp, up, dp, buf


@pytest.mark.parametrize("k,renorm", [(1, False), (2, False), (2, True), (6, False), (6, True)])
def test_layer_matches_reference_test_formula_in_torch(k, renorm):
    x, gw, gp, up, dp, buf = _toy_layer()
    E, h, I = gw.shape[0], x.shape[0], gp[0].shape[0]
    r = O.moe_forward(x.numpy(), gw.numpy(), buf, E, h, I, k, renorm)
    out, ids, ws = O.torch_moe_reference_cpu(x, gw, gp, up, dp, k, renorm)
    assert list(r["ids"]) == ids.tolist()
    np.testing.assert_allclose(r["weights"], ws.numpy(), rtol=1e-5)
    assert O.relative_error(out.numpy(), r["out"]) < 1e-5


def test_layer_k1_renorm_is_a_single_expert_ffn():
    x, gw, gp, up, dp, buf = _toy_layer(seed=9)
    E, h, I = gw.shape[0], x.shape[0], gp[0].shape[0]
    r = O.moe_forward(x.numpy(), gw.numpy(), buf, E, h, I, 1, True)
    e = int(np.argmax(gw.double().numpy() @ x.double().numpy()))
    assert int(r["ids"][0]) == e and float(r["weights"][0]) == 1.0
    np.testing.assert_allclose(r["out"], O.expert_ffn(x.numpy(), gp[e].numpy(), up[e].numpy(),
                                                      dp[e].numpy()), rtol=1e-12)


def test_layer_zero_hidden_gives_zero_output_and_first_k_ids():
    x, gw, gp, up, dp, buf = _toy_layer(seed=3)
    E, h, I = gw.shape[0], x.shape[0], gp[0].shape[0]
    r = O.moe_forward(np.zeros(h, np.float32), gw.numpy(), buf, E, h, I, 3, False)
    assert list(r["ids"]) == [0, 1, 2]
    np.testing.assert_array_equal(r["weights"], np.full(3, np.float32(1.0 / 8)))
    assert np.all(r["out"] == 0)


def test_batch_rows_equal_single_token_results():
    x, gw, gp, up, dp, buf = _toy_layer(seed=4)
    E, h, I = gw.shape[0], x.shape[0], gp[0].shape[0]
    xb = np.stack([x.numpy(), -x.numpy(), 0.5 * x.numpy()])
    rb = O.moe_forward_batch(xb, gw.numpy(), buf, E, h, I, 2, True)
    for b in range(3):
        r = O.moe_forward(xb[b], gw.numpy(), buf, E, h, I, 2, True)
        np.testing.assert_array_equal(rb["out"][b], r["out"])
        np.testing.assert_array_equal(rb["ids"][b], r["ids"])


# ----------------------------------------------------------------------------
# Reduced-precision weight formats
# ----------------------------------------------------------------------------
def test_decode_e4m3_matches_torch_for_every_code():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    got = O.decode_e4m3(codes)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_array_equal(got[~np.isnan(got)], want[~np.isnan(want)])
    # hand-checked codes: 1.0, -1.0, 448 (largest), 2^-9 (smallest subnormal), NaN
    assert O.decode_e4m3(np.array([0x38, 0xB8, 0x7E, 0x01], np.uint8)).tolist() == [
        1.0, -1.0, 448.0, 2.0 ** -9]
    assert np.isnan(O.decode_e4m3(np.array([0x7F, 0xFF], np.uint8))).all()


def test_decode_bf16_matches_torch_for_every_code():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(torch.float64).numpy()
    got = O.decode_bf16(bits)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(got)
    np.testing.assert_array_equal(got[ok], want[ok])


def _raw_block(layout, codes, scales=None):
    raw = np.zeros(layout["expert_stride"], np.uint8)
    raw[:len(codes)] = codes
    if scales is not None:
        sc = np.asarray(scales, np.float32).view(np.uint8)
        raw[layout["scale_offset"]:layout["scale_offset"] + len(sc)] = sc
    return raw


def test_fp8_expert_matrices_hand_computed():
    """E=1, h=2, I=2: gate codes 1, -1 / 2, 0.5; up 1.5, 2^-6 / 0, -2; down
    1, 2 / -1, 0.5.  Row scales: gate (2, 3), up (0.25, 4), down (10, 100)."""
    lo = O.weight_layout(1, 2, 2, "fp8")
    assert (lo["up_proj_offset"], lo["down_proj_offset"], lo["scale_offset"],
            lo["expert_stride"]) == (4, 8, 16, 128)
    codes = [0x38, 0xB8, 0x40, 0x30,   # gate
             0x3C, 0x08, 0x00, 0xC0,   # up
             0x38, 0x40, 0xB8, 0x30]   # down
    raw = _raw_block(lo, codes, [2, 3, 0.25, 4, 10, 100])
    g, u, d = O.expert_matrices(raw, 0, 1, 2, 2, "fp8")
    np.testing.assert_array_equal(g, [[2.0, -2.0], [6.0, 1.5]])
    np.testing.assert_array_equal(u, [[0.375, 0.25 * 2.0 ** -6], [0.0, -8.0]])
    np.testing.assert_array_equal(d, [[10.0, 20.0], [-100.0, 50.0]])


def test_bf16_expert_matrices_hand_computed():
    """bf16 0x3F80 = 1.0, 0xC000 = -2.0, 0x3F00 = 0.5, 0x4040 = 3.0."""
    lo = O.weight_layout(1, 1, 2, "bf16")
    vals = np.array([0x3F80, 0xC000, 0x3F00, 0x4040, 0x3F80, 0x3F00], np.uint16)
    raw = _raw_block(lo, vals.view(np.uint8))
    g, u, d = O.expert_matrices(raw, 0, 1, 1, 2, "bf16")
    np.testing.assert_array_equal(g, [[1.0], [-2.0]])
    np.testing.assert_array_equal(u, [[0.5], [3.0]])
    np.testing.assert_array_equal(d, [[1.0, 0.5]])


@pytest.mark.parametrize("fmt,np_dt", [("f32", np.float32), ("f16", np.float16)])
def test_expert_matrices_agree_with_expert_views(fmt, np_dt):
    rng = np.random.default_rng(0)
    E, h, I = 3, 5, 7
    mats = [[rng.standard_normal(s).astype(np_dt) for s in ((I, h), (I, h), (h, I))]
            for _ in range(E)]
    buf = O.pack_expert_weights([m[0] for m in mats], [m[1] for m in mats],
                                [m[2] for m in mats], E, h, I, dtype=np_dt)
    for e in range(E):
        a = O.expert_matrices(buf.view(np.uint8), e, E, h, I, fmt)
        b = O.expert_views(buf, e, E, h, I)
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y.astype(np.float64))


def test_decode_e2m1_table():
    """The OCP FP4 E2M1 value table, written out: codes 0-7 are 0, 0.5, 1,
    1.5, 2, 3, 4, 6 and codes 8-15 their negatives."""
    want = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
    got = O.decode_e2m1(np.arange(16))
    np.testing.assert_array_equal(got, want)
    assert np.signbit(got[8])


def test_decode_e8m0_matches_torch_for_every_code():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e8m0fnu).to(torch.float64).numpy()
    got = O.decode_e8m0(codes)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(got)
    np.testing.assert_array_equal(got[ok], want[ok])
    assert O.decode_e8m0(np.array([127, 0, 254], np.uint8)).tolist() == [1.0, 2.0 ** -127, 2.0 ** 127]


def test_mxfp4_expert_matrices_hand_computed():
    """E=1, h=32, I=32 (one block per row).  Gate row 0: codes 1 (0.5) and 15
    (-6) in its first byte (element 0 in the low nibble), scale byte 129 (x4);
    down row 31: element 31 code 7 (6), scale 120 (2^-7).  Everything else is
    code 0 with scale 127."""
    lo = O.weight_layout(1, 32, 32, "mxfp4")
    assert (lo["up_proj_offset"], lo["down_proj_offset"], lo["scale_offset"],
            lo["expert_stride"]) == (512, 1024, 1536, 1664)
    raw = np.zeros(lo["expert_stride"], np.uint8)
    raw[lo["scale_offset"]:lo["scale_offset"] + 96] = 127
    raw[0] = 0xF1                                    # gate[0][0] = 0.5, gate[0][1] = -6
    raw[lo["scale_offset"] + 0] = 129               # gate row 0 scale 4
    raw[lo["down_proj_offset"] + 31 * 16 + 15] = 0x70  # down[31][31] = 6 (high nibble)
    raw[lo["scale_offset"] + 64 + 31] = 120         # down row 31 scale 2^-7
    g, u, d = O.expert_matrices(raw, 0, 1, 32, 32, "mxfp4")
    want_g = np.zeros((32, 32))
    want_g[0, 0], want_g[0, 1] = 2.0, -24.0
    want_d = np.zeros((32, 32))
    want_d[31, 31] = 6.0 * 2.0 ** -7
    np.testing.assert_array_equal(g, want_g)
    np.testing.assert_array_equal(u, np.zeros((32, 32)))
    np.testing.assert_array_equal(d, want_d)
