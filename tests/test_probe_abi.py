"""libwr_probe.so (include/wr_probe.h), the measurement utility bench.py
uses beside the MoE library: it loads, exports every entry point the header
declares, and rejects invalid arguments before any HIP call (every case
here is invalid, so no kernel is launched and no GPU is needed)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "wr_probe.h")
LIB = os.path.join(ROOT, "warp-route_amd", "warp_route", "libwr_probe.so")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(LIB)
    lib.wr_probe_read.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_int64),
                                  ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                  ctypes.c_void_p]
    lib.wr_probe_gateup.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int,
                                    ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_void_p, ctypes.c_void_p]
    lib.wr_probe_down.argtypes = lib.wr_probe_gateup.argtypes
    return lib


def test_exports_every_declared_entry_point(lib):
    names = re.findall(r"WR_PROBE_API\s+[\w\s\*]+?\b(wr_probe_\w+)\s*\(", open(HEADER).read())
    assert sorted(names) == ["wr_probe_down", "wr_probe_gateup", "wr_probe_read"]
    for n in names:
        assert hasattr(lib, n), n


FAKE = 4096  # a 16-byte aligned stand-in address, never dereferenced


@pytest.mark.parametrize("n_experts,row_bytes,I,pattern,blocks", [
    (0, 8192, 14336, 0, 1), (9, 8192, 14336, 0, 1),       # expert count
    (2, 2048, 14336, 0, 1), (2, 12288, 14336, 0, 1),      # row length
    (2, 8192, 12, 0, 1), (2, 8192, 0, 0, 1),              # I not a positive multiple of 8
    (2, 8192, 14336, 2, 1), (2, 8192, 14336, 0, 0),       # pattern, grid
])
def test_gateup_rejects_invalid_arguments(lib, n_experts, row_bytes, I, pattern, blocks):
    ptrs = (ctypes.c_void_p * 9)(*([FAKE] * 9))
    assert lib.wr_probe_gateup(ptrs, n_experts, row_bytes, I, pattern, blocks,
                               ctypes.c_void_p(FAKE), None) == -1


def test_gateup_rejects_null_and_unaligned_pointers(lib):
    ok = (ctypes.c_void_p * 2)(FAKE, FAKE)
    assert lib.wr_probe_gateup(None, 2, 8192, 14336, 0, 1, ctypes.c_void_p(FAKE), None) == -1
    assert lib.wr_probe_gateup(ok, 2, 8192, 14336, 0, 1, None, None) == -1
    for bad in ((FAKE, 0), (FAKE, FAKE + 8)):
        p = (ctypes.c_void_p * 2)(*bad)
        assert lib.wr_probe_gateup(p, 2, 8192, 14336, 0, 1, ctypes.c_void_p(FAKE), None) == -1


@pytest.mark.parametrize("n_experts,row_bytes,h,pattern,blocks", [
    (0, 28672, 4096, 0, 1), (9, 28672, 4096, 0, 1),       # expert count
    (2, 8, 4096, 0, 1), (2, 28670, 4096, 0, 1),           # row length: >= 16, whole 16 B
    (2, 65552, 4096, 0, 1),                               # row length: at most 64 KB
    (2, 28672, 4094, 0, 1), (2, 28672, 0, 0, 1),          # h not a positive multiple of 4
    (2, 28672, 4096, 2, 1), (2, 28672, 4096, 0, 0),       # pattern, grid
])
def test_down_rejects_invalid_arguments(lib, n_experts, row_bytes, h, pattern, blocks):
    ptrs = (ctypes.c_void_p * 9)(*([FAKE] * 9))
    assert lib.wr_probe_down(ptrs, n_experts, row_bytes, h, pattern, blocks,
                             ctypes.c_void_p(FAKE), None) == -1


def test_read_rejects_invalid_arguments(lib):
    p = (ctypes.c_void_p * 1)(FAKE)
    n = (ctypes.c_int64 * 1)(1024)
    sink = ctypes.c_void_p(FAKE)
    assert lib.wr_probe_read(p, n, 0, 1, 1, sink, None) == -1          # no range
    assert lib.wr_probe_read(p, n, 1, 0, 1, sink, None) == -1          # blocks per CU
    assert lib.wr_probe_read(p, n, 1, 1, 3, sink, None) == -1          # unroll
    n_bad = (ctypes.c_int64 * 1)(1000)                                   # not whole 16 B
    assert lib.wr_probe_read(p, n_bad, 1, 1, 1, sink, None) == -1


@pytest.mark.gpu
def test_probe_patterns_run_on_small_experts(cuda, lib):
    """Every pattern of wr_probe_gateup and wr_probe_down, and wr_probe_read,
    over two small packed experts (h = 2048 and 4096 fp16 rows, I = 64):
    each returns 0, and none writes the sink (random bytes never fold to the
    value that would)."""
    import torch
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for h in (2048, 4096):
        I, row = 64, 2 * h
        expert = 3 * I * row  # gate, up [I][h] and down [h][I], fp16
        buf = torch.randint(0, 255, (2 * expert,), dtype=torch.uint8, device=cuda)
        sink = torch.zeros(4, dtype=torch.int32, device=cuda)
        gu = (ctypes.c_void_p * 2)(buf.data_ptr(), buf.data_ptr() + expert)
        dn = (ctypes.c_void_p * 2)(buf.data_ptr() + 2 * I * row,
                                   buf.data_ptr() + expert + 2 * I * row)
        print(f"[gpu] probe patterns h={h}", flush=True)
        for pattern in (0, 1):
            for blocks in (1, 7, 64):
                assert lib.wr_probe_gateup(gu, 2, row, I, pattern, blocks,
                                           ctypes.c_void_p(sink.data_ptr()), stream) == 0
                assert lib.wr_probe_down(dn, 2, 2 * I, h, pattern, blocks,
                                         ctypes.c_void_p(sink.data_ptr()), stream) == 0
        n = (ctypes.c_int64 * 1)(2 * expert)
        p = (ctypes.c_void_p * 1)(buf.data_ptr())
        assert lib.wr_probe_read(p, n, 1, 2, 4, ctypes.c_void_p(sink.data_ptr()), stream) == 0
        torch.cuda.synchronize()
        assert int(sink.abs().sum()) == 0
