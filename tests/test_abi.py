"""C-ABI checks that need no GPU: the library loads, exports every entry point
include/warp_route.h declares, and rejects invalid arguments with the right
status before any HIP call (each case below has at least one invalid
argument, so no kernel is ever launched from this file)."""
import ctypes
import os
import re

import pytest

from warp_route import capi
from warp_route import functional as F

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "warp_route.h")


def declared_symbols():
    text = open(HEADER).read()
    return re.findall(r"WR_API\s+[\w\s\*]+?\b(wr_\w+)\s*\(", text)


def test_header_declares_the_expected_entry_points():
    assert sorted(declared_symbols()) == sorted([
        "wr_status_str", "wr_layout", "wr_total_weight_bytes", "wr_layout_dtype",
        "wr_weight_bytes", "wr_workspace_bytes", "wr_gate_topk", "wr_fused_moe",
        "wr_fused_moe_route", "wr_fused_moe_ffn", "wr_batched_fused_moe", "wr_naive_moe",
        "wr_fused_moe_opts", "wr_fused_moe_status", "wr_fused_moe_noalloc",
        "wr_fused_moe_expired"])


def test_expiry_query_needs_no_gpu():
    """wr_fused_moe_expired is a host read of a word that only a
    single-token call allocates: before any such call it reports 0, with or
    without clearing, and makes no HIP call (none succeeds without a GPU)."""
    assert capi.lib().wr_fused_moe_expired(0) == 0
    assert capi.lib().wr_fused_moe_expired(1) == 0


def test_library_exports_every_declared_symbol():
    lib = capi.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_header_constants_match_binding():
    text = open(HEADER).read()
    for name in ("WR_MAX_EXPERTS", "WR_MAX_TOPK", "WR_EXPERT_ALIGN"):
        m = re.search(rf"#define {name} (\d+)", text)
        assert int(m.group(1)) == getattr(capi, name)
    for name in ("WR_OK", "WR_EINVAL_NULL", "WR_EINVAL_SHAPE", "WR_EINVAL_TOPK",
                 "WR_EINVAL_EXPERTS", "WR_EINVAL_DTYPE", "WR_EINVAL_WEIGHT_SIZE",
                 "WR_EINVAL_WORKSPACE", "WR_EINVAL_BATCH", "WR_EINVAL_KIND", "WR_EHIP",
                 "WR_F32", "WR_F16", "WR_BF16", "WR_FP8_E4M3", "WR_MXFP4", "WR_EINVAL_BLOCK",
                 "WR_ETIMEOUT", "WR_EINVAL_SCRATCH",
                 "WR_KIND_FUSED",
                 "WR_KIND_BATCHED", "WR_KIND_NAIVE"):
        m = re.search(rf"\b{name} = (\d+)", text)
        assert m and int(m.group(1)) == getattr(capi, name), name


def test_struct_layout_matches_header_order():
    # 3 pointer-sized fields, 8 int32, 6 pointer-sized: 104 bytes, no padding.
    assert ctypes.sizeof(capi.WrMoeArgs) == 104
    assert capi.WrMoeArgs.x.offset == 56
    assert ctypes.sizeof(capi.WrOffsets) == 32
    assert ctypes.sizeof(capi.WrLayoutInfo) == 48
    # spin_limit, wait_extra, gu_blocks
    assert ctypes.sizeof(capi.WrFusedOpts) == 12
    assert capi.WrFusedOpts.gu_blocks.offset == 8


FMT = {capi.WR_F32: "f32", capi.WR_F16: "f16", capi.WR_BF16: "bf16", capi.WR_FP8_E4M3: "fp8",
       capi.WR_MXFP4: "mxfp4"}
TDT = {capi.WR_F32: "float32", capi.WR_F16: "float16", capi.WR_BF16: "bfloat16",
       capi.WR_FP8_E4M3: "float8_e4m3fn", capi.WR_MXFP4: "float4_e2m1fn_x2"}


@pytest.mark.parametrize("wdt", sorted(FMT))
@pytest.mark.parametrize("E,h,I", [(8, 4096, 14336), (64, 2048, 1408), (2, 3, 5), (3, 7, 1),
                                   (3, 96, 32)])
def test_layout_dtype_agrees_with_python_and_oracle(E, h, I, wdt):
    if wdt == capi.WR_MXFP4 and (h % 32 or I % 32):
        info = capi.WrLayoutInfo()
        st = capi.lib().wr_layout_dtype(E, h, I, wdt, ctypes.byref(info))
        assert st == capi.WR_EINVAL_BLOCK
        assert capi.lib().wr_weight_bytes(E, h, I, wdt) == -1
        return
    import torch
    from oracle import moe_oracle as O
    got = capi.layout_dtype(E, h, I, wdt)
    want = O.weight_layout(E, h, I, FMT[wdt])
    assert {k: got[k] for k in want} == want and got["weight_dtype"] == wdt
    assert F.weight_layout(E, h, I, getattr(torch, TDT[wdt])) == want
    assert capi.lib().wr_weight_bytes(E, h, I, wdt) == E * want["expert_stride"]


def test_fp8_layout_byte_table():
    """Hand-computed: E=8, h=4096, I=14336 (Mixtral): codes 3 I h =
    176,160,768 bytes (a multiple of 16), then 4 (2 I + h) = 131,072 bytes of
    row scales; 176,291,840 is a multiple of 128.  h=3, I=5: codes 45 bytes,
    scales at 48, 52 bytes of them, stride 128."""
    assert capi.layout_dtype(8, 4096, 14336, capi.WR_FP8_E4M3) == {
        "gate_proj_offset": 0, "up_proj_offset": 58720256, "down_proj_offset": 117440512,
        "scale_offset": 176160768, "expert_stride": 176291840, "elem_bytes": 1,
        "weight_dtype": capi.WR_FP8_E4M3}
    # MXFP4, Mixtral: codes 3 I h / 2 = 88,080,384 bytes, then 3 I h / 32 =
    # 5,505,024 bytes of E8M0 scales; 93,585,408 is a multiple of 128.
    assert capi.layout_dtype(8, 4096, 14336, capi.WR_MXFP4) == {
        "gate_proj_offset": 0, "up_proj_offset": 29360128, "down_proj_offset": 58720256,
        "scale_offset": 88080384, "expert_stride": 93585408, "elem_bytes": 0,
        "weight_dtype": capi.WR_MXFP4}
    lo = capi.layout_dtype(2, 3, 5, capi.WR_FP8_E4M3)
    assert (lo["up_proj_offset"], lo["down_proj_offset"], lo["scale_offset"],
            lo["expert_stride"]) == (15, 30, 48, 128)
    assert capi.layout_dtype(2, 3, 5, capi.WR_BF16)["scale_offset"] == -1


@pytest.mark.parametrize("E,h,I,es", [(8, 4096, 14336, 2), (64, 2048, 1408, 2),
                                      (16, 6144, 10752, 2), (8, 256, 512, 4), (2, 3, 5, 4),
                                      (2, 3, 5, 2)])
def test_layout_agrees_with_python_and_oracle(E, h, I, es):
    from oracle import moe_oracle as O
    assert capi.layout(E, h, I, es) == O.layout_offsets(E, h, I, es)
    assert F.expert_layout(E, h, I, es) == O.layout_offsets(E, h, I, es)
    assert capi.lib().wr_total_weight_bytes(E, h, I, es) == O.total_weight_bytes(E, h, I, es)


def test_layout_rejects_bad_arguments():
    o = capi.WrOffsets()
    lib = capi.lib()
    assert lib.wr_layout(0, 4, 4, 2, ctypes.byref(o)) == capi.WR_EINVAL_SHAPE
    assert lib.wr_layout(1, 4, 4, 3, ctypes.byref(o)) == capi.WR_EINVAL_DTYPE
    assert lib.wr_layout(1, 4, 4, 2, None) == capi.WR_EINVAL_NULL
    assert lib.wr_total_weight_bytes(1, 0, 4, 2) == -1
    info = capi.WrLayoutInfo()
    assert lib.wr_layout_dtype(1, 4, 4, 5, ctypes.byref(info)) == capi.WR_EINVAL_DTYPE
    assert lib.wr_layout_dtype(1, 4, 0, 1, ctypes.byref(info)) == capi.WR_EINVAL_SHAPE
    assert lib.wr_layout_dtype(1, 4, 4, 1, None) == capi.WR_EINVAL_NULL
    assert lib.wr_weight_bytes(1, 4, 4, -1) == -1


def test_workspace_bytes():
    lib = capi.lib()
    # fused: control block (64 arrival words, a timeout flag, an unused word
    # and 8 gate/up claim counters, one 256-byte line each, then 16 copies of
    # the router slots of a kernel with the router inside, 1152 bytes each)
    # + 64 fp32 logits per token (E padded to 64) + act: single
    # token k rows of I rounded up to 16 columns, B > 1 B*k*I; fp32, rounded up
    # to 256 bytes.
    ctrl = 74 * 256 + 16 * 1152
    assert lib.wr_workspace_bytes(capi.WR_KIND_FUSED, 8, 4096, 14336, 2, 1) == (
        ctrl + 256 + 2 * 14336 * 4)
    assert lib.wr_workspace_bytes(capi.WR_KIND_FUSED, 8, 64, 100, 3, 1) == (
        ctrl + 256 + 1536)  # 3 * 112 * 4 = 1344 -> 1536
    # batched, B > 1: the larger of the per-token layout above and the
    # grouped MFMA layout: logits, x as two fp16 terms and its per-token
    # exponents, one act-maximum word per pair on its own 256-byte line, five
    # [P] pair arrays, expert offsets / active list / count, act [P][I] and
    # four K-slice partials [4][P][h] (P = B * k), each region rounded up to
    # 256 bytes.
    def up(n):
        return (n + 255) // 256 * 256
    B, E, h, I, k = 4, 8, 4096, 14336, 2
    P = B * k
    per_token = ctrl + B * 256 + P * I * 4
    grouped = (up(B * 256) + 2 * up(B * h * 2) + up(B * 4) + P * 256 + 5 * up(P * 4)
               + up((E + 1) * 4) + up(E * 4) + up(4) + up(P * I * 4) + up(4 * P * h * 4))
    assert grouped == 1051648 + 256 + 8 * 256
    assert lib.wr_workspace_bytes(capi.WR_KIND_BATCHED, E, h, I, k, B) == max(per_token, grouped)
    assert lib.wr_workspace_bytes(capi.WR_KIND_NAIVE, 8, 100, 10, 1, 1) == 256 + 3 * 256 + 2 * 512
    assert lib.wr_workspace_bytes(7, 8, 64, 64, 2, 1) == 0
    assert lib.wr_workspace_bytes(capi.WR_KIND_FUSED, 65, 64, 64, 2, 1) == 0
    assert lib.wr_workspace_bytes(capi.WR_KIND_FUSED, 8, 64, 64, 0, 1) == 0
    assert lib.wr_workspace_bytes(capi.WR_KIND_BATCHED, 8, 64, 64, 2, -1) == 0


def test_status_strings():
    for s in range(0, 14):
        assert capi.status_str(s)
    assert capi.status_str(capi.WR_EHIP) == "HIP runtime error"


FAKE = 0x1000  # never dereferenced: every case below fails validation first


def valid_args(B=1):
    E, h, I, k = 8, 64, 32, 2
    a = capi.WrMoeArgs()
    a.gate_w = FAKE
    a.weight_buf = FAKE
    a.weight_bytes = capi.lib().wr_total_weight_bytes(E, h, I, 2)
    a.weight_dtype = capi.WR_F16
    a.num_experts, a.hidden_dim, a.intermediate_dim, a.top_k = E, h, I, k
    a.renormalize = 0
    a.batch_size = B
    a.act_dtype = capi.WR_F32
    a.x = FAKE
    a.out = FAKE
    a.topk_ids = FAKE
    a.topk_weights = FAKE
    a.workspace = FAKE
    a.workspace_bytes = 1 << 30
    return a


CASES = [
    ("num_experts", 0, capi.WR_EINVAL_SHAPE),
    ("hidden_dim", 0, capi.WR_EINVAL_SHAPE),
    ("intermediate_dim", -3, capi.WR_EINVAL_SHAPE),
    ("num_experts", 65, capi.WR_EINVAL_EXPERTS),
    ("top_k", 0, capi.WR_EINVAL_TOPK),
    ("top_k", 7, capi.WR_EINVAL_TOPK),
    ("weight_dtype", 5, capi.WR_EINVAL_DTYPE),
    ("act_dtype", -1, capi.WR_EINVAL_DTYPE),
    ("act_dtype", capi.WR_BF16, capi.WR_EINVAL_DTYPE),
    ("gate_w", None, capi.WR_EINVAL_NULL),
    ("x", None, capi.WR_EINVAL_NULL),
    ("out", None, capi.WR_EINVAL_NULL),
    ("weight_buf", None, capi.WR_EINVAL_NULL),
    ("weight_bytes", 1000, capi.WR_EINVAL_WEIGHT_SIZE),
    ("workspace", None, capi.WR_EINVAL_WORKSPACE),
    ("workspace_bytes", 16, capi.WR_EINVAL_WORKSPACE),
]


@pytest.mark.parametrize("entry", ["wr_fused_moe", "wr_fused_moe_route", "wr_fused_moe_ffn",
                                   "wr_batched_fused_moe", "wr_naive_moe"])
@pytest.mark.parametrize("field,value,want", CASES)
def test_validation_codes(entry, field, value, want):
    a = valid_args()
    setattr(a, field, value)
    assert capi.call(entry, a) == want


def test_fused_opts_entry_point_validates_like_wr_fused_moe():
    """wr_fused_moe_opts runs the same argument checks before any HIP call,
    with or without options."""
    opts = capi.WrFusedOpts(spin_limit=4, wait_extra=1)
    for field, value, want in CASES:
        a = valid_args()
        setattr(a, field, value)
        assert capi.lib().wr_fused_moe_opts(ctypes.byref(a), ctypes.byref(opts), None) == want
        assert capi.lib().wr_fused_moe_opts(ctypes.byref(a), None, None) == want
    a = valid_args(B=2)
    assert capi.lib().wr_fused_moe_opts(ctypes.byref(a), None, None) == capi.WR_EINVAL_BATCH


def test_noalloc_validates_before_hip():
    """wr_fused_moe_noalloc ignores the workspace fields, runs the other
    checks of wr_fused_moe, and rejects a problem whose workspace exceeds its
    fixed scratch before any HIP call."""
    lib = capi.lib()
    assert lib.wr_fused_moe_noalloc(None, None) == capi.WR_EINVAL_NULL
    for field, value, want in CASES:
        if field.startswith("workspace"):
            continue
        a = valid_args()
        setattr(a, field, value)
        assert lib.wr_fused_moe_noalloc(ctypes.byref(a), None) == want, field
    a = valid_args()
    a.intermediate_dim, a.top_k = 65536, 2
    a.weight_bytes = 1 << 40
    assert (lib.wr_workspace_bytes(capi.WR_KIND_FUSED, 8, 64, 65536, 2, 1)
            <= capi.WR_NOALLOC_SCRATCH_BYTES)
    a.top_k = 6
    assert lib.wr_fused_moe_noalloc(ctypes.byref(a), None) == capi.WR_EINVAL_SCRATCH
    a = valid_args(B=2)
    assert lib.wr_fused_moe_noalloc(ctypes.byref(a), None) == capi.WR_EINVAL_BATCH
    text = open(HEADER).read()
    import re
    m = re.search(r"#define WR_NOALLOC_SCRATCH_BYTES \(1u << (\d+)\)", text)
    assert m and (1 << int(m.group(1))) == capi.WR_NOALLOC_SCRATCH_BYTES


def test_fused_status_checks_its_workspace_before_hip():
    lib = capi.lib()
    assert lib.wr_fused_moe_status(None, 1 << 20, None) == capi.WR_EINVAL_NULL
    # smaller than the control block (74 lines of 256 bytes)
    assert lib.wr_fused_moe_status(FAKE, 74 * 256 - 1, None) == capi.WR_EINVAL_WORKSPACE
    assert "NaN" in capi.status_str(capi.WR_ETIMEOUT)


def test_mxfp4_needs_blocks_of_32():
    a = valid_args()  # h = 64, I = 32
    a.weight_dtype = capi.WR_MXFP4
    a.intermediate_dim = 48
    assert capi.call("wr_fused_moe", a) == capi.WR_EINVAL_BLOCK
    assert capi.status_str(capi.WR_EINVAL_BLOCK).startswith("MXFP4")


@pytest.mark.parametrize("wdt", [capi.WR_BF16, capi.WR_FP8_E4M3, capi.WR_MXFP4])
def test_weight_size_is_checked_per_format(wdt):
    """One byte short of wr_weight_bytes is rejected for every format (the
    fp8 layout is smaller than fp16's, and holds its scales)."""
    a = valid_args()
    a.weight_dtype = wdt
    need = capi.lib().wr_weight_bytes(a.num_experts, a.hidden_dim, a.intermediate_dim, wdt)
    a.weight_bytes = need - 1
    a.workspace = None  # so that a passing size check still stops before HIP
    assert capi.call("wr_fused_moe", a) == capi.WR_EINVAL_WEIGHT_SIZE
    a.weight_bytes = need
    assert capi.call("wr_fused_moe", a) == capi.WR_EINVAL_WORKSPACE


def test_top_k_above_num_experts_is_rejected():
    a = valid_args()
    a.num_experts, a.top_k = 2, 3
    a.weight_bytes = 1 << 40
    assert capi.call("wr_fused_moe", a) == capi.WR_EINVAL_TOPK


def test_batch_rules():
    a = valid_args(B=2)
    a.weight_bytes = 10  # would fail later; batch is checked first
    assert capi.call("wr_fused_moe", a) == capi.WR_EINVAL_BATCH
    assert capi.call("wr_fused_moe_route", a) == capi.WR_EINVAL_BATCH
    assert capi.call("wr_fused_moe_ffn", a) == capi.WR_EINVAL_BATCH
    assert capi.call("wr_naive_moe", a) == capi.WR_EINVAL_BATCH
    a.batch_size = -1
    assert capi.call("wr_batched_fused_moe", a) == capi.WR_EINVAL_BATCH
    # B == 0 is a no-op, as in src/fused_moe_batched.cu:201 (returns before HIP)
    a.batch_size = 0
    assert capi.call("wr_batched_fused_moe", a) == capi.WR_OK
    assert capi.call("wr_gate_topk", a) == capi.WR_OK


def test_gate_topk_requires_outputs():
    a = valid_args()
    a.topk_ids = None
    assert capi.call("wr_gate_topk", a) == capi.WR_EINVAL_NULL
    a = valid_args()
    a.topk_weights = None
    assert capi.call("wr_gate_topk", a) == capi.WR_EINVAL_NULL
    assert capi.lib().wr_fused_moe(None, None) == capi.WR_EINVAL_NULL


def test_timeline_hook_is_exported_and_off_by_default():
    """include/wr_timeline.h: both functions are exported; a default build
    (no WR_TIMELINE) records nothing and says so before any HIP call."""
    import re as _re
    text = open(os.path.join(ROOT, "include", "wr_timeline.h")).read()
    names = _re.findall(r"WR_TL_API\s+[\w\s\*]+?\b(wr_\w+)\s*\(", text)
    assert sorted(names) == ["wr_timeline_clock_khz", "wr_timeline_read"]
    lib = capi.lib()
    for name in names:
        assert hasattr(lib, name), name
    buf = (ctypes.c_uint64 * 8)()
    assert lib.wr_timeline_read(buf, 1, None) == -1
