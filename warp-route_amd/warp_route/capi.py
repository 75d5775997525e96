"""ctypes binding of the C-ABI in include/warp_route.h (libwarp_route_hip.so).

This is the binding a caller without the torch extension uses: plain device
pointers, sizes and a hipStream_t passed as an integer.  It mirrors the header
field for field; ``tests/test_abi.py`` checks that every declared entry point
is exported.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libwarp_route_hip.so")

WR_MAX_EXPERTS = 64
WR_MAX_TOPK = 6
WR_EXPERT_ALIGN = 128

WR_OK = 0
WR_EINVAL_NULL = 1
WR_EINVAL_SHAPE = 2
WR_EINVAL_TOPK = 3
WR_EINVAL_EXPERTS = 4
WR_EINVAL_DTYPE = 5
WR_EINVAL_WEIGHT_SIZE = 6
WR_EINVAL_WORKSPACE = 7
WR_EINVAL_BATCH = 8
WR_EINVAL_KIND = 9
WR_EINVAL_BLOCK = 10
WR_ETIMEOUT = 11
WR_EINVAL_SCRATCH = 12
WR_NOALLOC_SCRATCH_BYTES = 1 << 20
WR_EHIP = 100

WR_F32 = 0
WR_F16 = 1
WR_BF16 = 2
WR_FP8_E4M3 = 3
WR_MXFP4 = 4

WR_KIND_FUSED = 0
WR_KIND_BATCHED = 1
WR_KIND_NAIVE = 2


class WrOffsets(ctypes.Structure):
    _fields_ = [("gate_proj_offset", ctypes.c_int64), ("up_proj_offset", ctypes.c_int64),
                ("down_proj_offset", ctypes.c_int64), ("expert_stride", ctypes.c_int64)]


class WrLayoutInfo(ctypes.Structure):
    _fields_ = [("gate_proj_offset", ctypes.c_int64), ("up_proj_offset", ctypes.c_int64),
                ("down_proj_offset", ctypes.c_int64), ("scale_offset", ctypes.c_int64),
                ("expert_stride", ctypes.c_int64), ("elem_bytes", ctypes.c_int32),
                ("weight_dtype", ctypes.c_int32)]


class WrFusedOpts(ctypes.Structure):
    _fields_ = [("spin_limit", ctypes.c_uint32), ("wait_extra", ctypes.c_uint32),
                ("gu_blocks", ctypes.c_uint32)]


class WrMoeArgs(ctypes.Structure):
    _fields_ = [
        ("gate_w", ctypes.c_void_p),
        ("weight_buf", ctypes.c_void_p),
        ("weight_bytes", ctypes.c_int64),
        ("weight_dtype", ctypes.c_int32),
        ("num_experts", ctypes.c_int32),
        ("hidden_dim", ctypes.c_int32),
        ("intermediate_dim", ctypes.c_int32),
        ("top_k", ctypes.c_int32),
        ("renormalize", ctypes.c_int32),
        ("batch_size", ctypes.c_int32),
        ("act_dtype", ctypes.c_int32),
        ("x", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("topk_ids", ctypes.c_void_p),
        ("topk_weights", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
    ]


_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """Load libwarp_route_hip.so and declare its prototypes."""
    global _lib
    if _lib is None:
        l = ctypes.CDLL(LIB_PATH)
        l.wr_status_str.argtypes = [ctypes.c_int]
        l.wr_status_str.restype = ctypes.c_char_p
        l.wr_layout.argtypes = [ctypes.c_int] * 4 + [ctypes.POINTER(WrOffsets)]
        l.wr_layout.restype = ctypes.c_int
        l.wr_total_weight_bytes.argtypes = [ctypes.c_int] * 4
        l.wr_total_weight_bytes.restype = ctypes.c_int64
        l.wr_layout_dtype.argtypes = [ctypes.c_int] * 4 + [ctypes.POINTER(WrLayoutInfo)]
        l.wr_layout_dtype.restype = ctypes.c_int
        l.wr_weight_bytes.argtypes = [ctypes.c_int] * 4
        l.wr_weight_bytes.restype = ctypes.c_int64
        l.wr_workspace_bytes.argtypes = [ctypes.c_int] * 6
        l.wr_workspace_bytes.restype = ctypes.c_size_t
        for name in ("wr_gate_topk", "wr_fused_moe", "wr_fused_moe_route", "wr_fused_moe_ffn",
                     "wr_batched_fused_moe", "wr_naive_moe", "wr_fused_moe_noalloc"):
            f = getattr(l, name)
            f.argtypes = [ctypes.POINTER(WrMoeArgs), ctypes.c_void_p]
            f.restype = ctypes.c_int
        l.wr_fused_moe_opts.argtypes = [ctypes.POINTER(WrMoeArgs), ctypes.POINTER(WrFusedOpts),
                                        ctypes.c_void_p]
        l.wr_fused_moe_opts.restype = ctypes.c_int
        l.wr_fused_moe_status.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        l.wr_fused_moe_status.restype = ctypes.c_int
        l.wr_fused_moe_expired.argtypes = [ctypes.c_int]
        l.wr_fused_moe_expired.restype = ctypes.c_int
        # include/wr_timeline.h (measurement hook)
        l.wr_timeline_read.argtypes = [ctypes.POINTER(ctypes.c_uint64), ctypes.c_int64,
                                       ctypes.c_void_p]
        l.wr_timeline_read.restype = ctypes.c_int64
        l.wr_timeline_clock_khz.argtypes = []
        l.wr_timeline_clock_khz.restype = ctypes.c_int64
        _lib = l
    return _lib


def status_str(status: int) -> str:
    return lib().wr_status_str(status).decode()


def layout(E: int, h: int, I: int, elem_bytes: int) -> dict:
    o = WrOffsets()
    st = lib().wr_layout(E, h, I, elem_bytes, ctypes.byref(o))
    if st != WR_OK:
        raise ValueError(status_str(st))
    return {f: getattr(o, f) for f, _ in WrOffsets._fields_}


def layout_dtype(E: int, h: int, I: int, weight_dtype: int) -> dict:
    o = WrLayoutInfo()
    st = lib().wr_layout_dtype(E, h, I, weight_dtype, ctypes.byref(o))
    if st != WR_OK:
        raise ValueError(status_str(st))
    return {f: getattr(o, f) for f, _ in WrLayoutInfo._fields_}


def call(name: str, args: WrMoeArgs, stream: int = 0) -> int:
    """Invoke wr_gate_topk / wr_fused_moe / wr_batched_fused_moe / wr_naive_moe."""
    return getattr(lib(), name)(ctypes.byref(args), ctypes.c_void_p(stream))
