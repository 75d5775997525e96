"""Resource checks on the gfx950 code object built here (no GPU needed).

The kernels' speed rests on properties the source does not show:
- no kernel may keep an array in scratch memory (a scratch load's wait also
  waits for every weight load issued before it, since vmcnt counts in order)
  or spill;
- the register-path kernels may not hold a per-thread array in LDS;
- the fp16 / bf16 / MXFP4 single-token kernels must fit 128 VGPRs (4 waves
  per SIMD), as the kernel descriptor allocates them: the metadata's
  vgpr_count can be lower than the allocation, which is rounded up from the
  accumulation-register offset (124 listed and 136 allocated has happened);
- in the batched kernels' K loops, a K step's weight loads must still be in
  flight when the previous step's MFMAs run.  The load counter is in order,
  so any use of a value loaded after the weights (a conversion of the act or
  x tile, a mask of an MXFP4 scale byte) placed before the MFMAs waits for
  the weights too; that has happened three times, invisible in the source.
The compiler has broken the first two silently, by folding a select chain
over the TopK arrays back into a runtime-indexed array (in scratch memory in
the x-in-LDS kernels, in LDS in the others).  These tests read the kernel
descriptors' metadata (the AMDGPU note in the code object of
libwarp_route_hip.so) with the ROCm LLVM tools.
"""
import os
import re
import struct
import subprocess

import pytest

from warp_route import capi

LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"


def _descriptor_vgprs(elf_path, readelf):
    """{kernel symbol: VGPRs the kernel descriptor allocates} of one code
    object: (GRANULATED_WORKITEM_VGPR_COUNT + 1) * 8 from COMPUTE_PGM_RSRC1
    (bytes 48-51 of the 64-byte descriptor at symbol <kernel>.kd)."""
    b = open(elf_path, "rb").read()
    shoff, = struct.unpack_from("<Q", b, 0x28)
    shentsize, shnum = struct.unpack_from("<HH", b, 0x3a)
    secs = [struct.unpack_from("<IIQQQQ", b, shoff + i * shentsize) for i in range(shnum)]
    syms = subprocess.run([readelf, "-s", elf_path], check=True, capture_output=True,
                          text=True).stdout
    out = {}
    for line in syms.splitlines():
        f = line.split()
        if len(f) < 8 or not f[-1].endswith(".kd"):
            continue
        addr = int(f[1], 16)
        for _, typ, _, sa, so, size in secs:
            if typ != 8 and sa <= addr < sa + size:  # not NOBITS
                rsrc1, = struct.unpack_from("<I", b, so + addr - sa + 48)
                out[f[-1][:-3]] = ((rsrc1 & 0x3F) + 1) * 8
                break
    return out


def _branch_target(addr, op, args):
    if not (op == "s_branch" or op.startswith("s_cbranch")):
        return None
    imm = int(args.split()[0])
    return addr + 4 + 4 * (imm - 65536 if imm > 32767 else imm)


def _walk(insns, idx, i):
    """Instruction indices executed after instruction i: fall-through at
    conditional branches, unconditional branches followed."""
    j, n = i + 1, 0
    while j < len(insns) and n < 4000:
        n += 1
        yield j
        addr, op, args = insns[j]
        if op == "s_endpgm":
            return
        if op == "s_branch":
            t = _branch_target(addr, op, args)
            if t not in idx:
                return
            j = idx[t]
        else:
            j += 1


def _waits_before_mfma(insns):
    """Weight loads (global_load_dwordx4 ... nt) inside a loop whose forward
    path reaches a wait that needs them before any MFMA: [(load, wait)]."""
    idx = {a: i for i, (a, _, _) in enumerate(insns)}
    bad = []
    for i, (addr, op, args) in enumerate(insns):
        if not (op.startswith("global_load_dwordx4") and args.endswith(" nt")):
            continue
        path = list(_walk(insns, idx, i))
        if i not in path:  # not in a loop: a prologue load, awaited before the first step
            continue
        after = 0  # vector-memory instructions issued after this load
        for j in path:
            a, opj, argj = insns[j]
            if opj.startswith("v_mfma") or j == i:
                break
            if re.match(r"(global|buffer)_(load|store|atomic)", opj):
                after += 1
            m = re.search(r"vmcnt\((\d+)\)", argj) if opj == "s_waitcnt" else None
            if m and int(m.group(1)) <= after:
                bad.append((hex(addr), hex(a)))
                break
    return bad


def _tool(name):
    path = os.path.join(LLVM, name)
    if not os.access(path, os.X_OK):
        pytest.skip(f"{path} not available")
    return path


@pytest.fixture(scope="module")
def kernels(tmp_path_factory):
    """{kernel symbol: {metadata key: int}} of every kernel in the library."""
    if not os.path.exists(capi.LIB_PATH):
        pytest.fail(f"{capi.LIB_PATH} is not built (run __graft_entry__.build())")
    d = tmp_path_factory.mktemp("codeobj")
    fat = d / "fat.bin"
    subprocess.run([_tool("llvm-objcopy"), f"--dump-section=.hip_fatbin={fat}", capi.LIB_PATH,
                    str(d / "host.so")], check=True, capture_output=True)
    # One offload bundle per translation unit with device code, back to back.
    blob = fat.read_bytes()
    starts = [m.start() for m in re.finditer(rb"__CLANG_OFFLOAD_BUNDLE__", blob)]
    assert starts and starts[0] == 0, "no offload bundle in .hip_fatbin"
    out = {}
    for i, s in enumerate(starts):
        part, co = d / f"bundle{i}.bin", d / f"gfx950_{i}.elf"
        part.write_bytes(blob[s:starts[i + 1] if i + 1 < len(starts) else len(blob)])
        subprocess.run([_tool("clang-offload-bundler"), "--unbundle", "--type=o",
                        f"--input={part}", f"--targets={TARGET}", f"--output={co}"],
                       check=True, capture_output=True)
        notes = subprocess.run([_tool("llvm-readelf"), "--notes", str(co)], check=True,
                               capture_output=True, text=True).stdout
        # Each kernel is one item of the amdhsa.kernels list, its keys in
        # alphabetical order (.group_segment_fixed_size comes before .name).
        m = re.search(r"^(\s*)amdhsa\.kernels:\s*$", notes, re.M)
        if not m:  # a translation unit with device variables but no kernels
            continue
        alloc = _descriptor_vgprs(str(co), _tool("llvm-readelf"))
        item = re.compile(rf"^{m.group(1)}  - \.")
        rec = None
        for line in notes[m.end():].splitlines():
            if item.match(line):
                rec = {}
            kv = re.match(rf"^{m.group(1)}  (?:- |  )\.(\w+):\s+(\S+)\s*$", line)
            if rec is None or not kv:
                continue
            key, val = kv.groups()
            if key == "name":
                out[val] = rec
                rec["vgpr_alloc"] = alloc.get(val, 0)
            elif re.fullmatch(r"-?\d+", val):
                rec.setdefault(key, int(val))
    assert any("k_fused_ffn" in k for k in out) and any("k_gu_mfma" in k for k in out), \
        f"expected kernels missing from the code object ({len(out)} found)"
    return out


@pytest.fixture(scope="module")
def batched_isa(kernels, tmp_path_factory):
    """{kernel symbol: [(address, mnemonic, operands)]} of the batched MFMA
    kernels, disassembled from the code objects the kernels fixture unpacked."""
    d = tmp_path_factory.getbasetemp()
    out = {}
    for co in sorted(d.glob("codeobj*/gfx950_*.elf")):
        text = subprocess.run([_tool("llvm-objdump"), "-d", "--no-show-raw-insn", str(co)],
                              check=True, capture_output=True, text=True).stdout
        name = None
        for line in text.splitlines():
            m = re.match(r"^[0-9a-f]+ <(\S+)>:$", line)
            if m:
                name = m.group(1) if re.search(r"k_(gu|dn)_(mfma|f32)", m.group(1)) else None
                if name:
                    out[name] = []
                continue
            m = re.match(r"^\s+(\S+)\s*(.*?)\s*//\s*([0-9A-F]+):", line)
            if name and m:
                out[name].append((int(m.group(3), 16), m.group(1), m.group(2)))
    return out


def test_batched_k_loops_keep_weight_loads_in_flight_over_mfmas(batched_isa):
    assert len(batched_isa) >= 30, sorted(batched_isa)
    looped = 0
    bad = {}
    for name, insns in batched_isa.items():
        idx = {a: i for i, (a, _, _) in enumerate(insns)}
        looped += any(op.startswith("global_load_dwordx4") and args.endswith(" nt")
                      and i in _walk(insns, idx, i) for i, (_, op, args) in enumerate(insns))
        b = _waits_before_mfma(insns)
        if b:
            bad[name] = b[:3]
    assert looped == len(batched_isa), "a kernel's K loop was not found"
    assert not bad, f"K-loop weight loads awaited before the MFMAs: {bad}"


def test_no_kernel_uses_scratch_memory_or_spills(kernels):
    bad = {k: (v.get("private_segment_fixed_size"), v.get("vgpr_spill_count"))
           for k, v in kernels.items()
           if v.get("private_segment_fixed_size", 0) != 0 or v.get("vgpr_spill_count", 0) != 0}
    assert not bad, f"kernels with scratch memory or VGPR spills: {bad}"


def test_single_token_kernels_keep_four_waves_per_simd(kernels):
    # k_fused_ffn<WT, XT, VEC, ...> with 16-byte vectors: f16 / bf16 (VEC 8)
    # and MXFP4 (VEC 32).  fp8 keeps 3 waves by design (16 fp32 x values
    # per chunk and lane on the register path), and so do the MXFP4 kernels
    # with whole rows in flight (U1 = 2, below).
    fused = {k: v["vgpr_alloc"] for k, v in kernels.items() if re.search(
        r"k_fused_ffnI(DF16_|NS_5bf16wE)(DF16_|f)Li8E|k_fused_ffnINS_5fp4x2E(DF16_|f)Li32E", k)
        and not re.search(WHOLE_ROWS, k)}
    # 3 weight types x 2 x types x 2 RPW x 2 x paths, plus the MXFP4 kernels
    # with staged block scales (x in LDS, 4 rows per wave) for the 2 x types,
    # plus the claiming register-path variants of f16 and bf16 (2 x 2 x 2),
    # plus the register-path variants with the router inside (3 x 2 x 2),
    # plus the all-resident x-in-LDS variants of f16 and bf16 (2 x 2 x 2)
    assert len(fused) == 54, sorted(fused)
    assert all(n > 0 for n in fused.values()), "kernel descriptors not found"
    over = {k: n for k, n in fused.items() if n > 128}
    assert not over, f"single-token kernels allocating more than 128 VGPRs: {over}"


# f16 / bf16 single-token kernels with x in LDS and half the column chunks in
# flight (2 per down tile): the variant taken when every gate/up and down
# block of the layer can be resident at once.
ALL_RESIDENT = r"k_fused_ffnI(DF16_|NS_5bf16wE)(DF16_|f)Li8ELi[24]ELi[12]ELi4ELi2ELb1ELb0ELb0ELb0EEEv"


def test_all_resident_kernels_fit_six_blocks_per_cu(kernels):
    # x-in-LDS f16 / bf16 layers have h <= 4096 (at most 1024 down blocks of
    # 4 rows) and at most 2 gate/up blocks per CU: on 256 CUs all of them are
    # resident at once when 6 blocks of 4 waves fit a CU (512 VGPRs per SIMD
    # lane, 160 KB of LDS).
    ar = {k: (v["vgpr_alloc"], v.get("group_segment_fixed_size", 0))
          for k, v in kernels.items() if re.search(ALL_RESIDENT, k)}
    assert len(ar) == 8, sorted(ar)
    assert all(n > 0 for n, _ in ar.values()), "kernel descriptors not found"
    over = {k: (n, lds) for k, (n, lds) in ar.items() if 6 * n > 512 or 6 * lds > 160 * 1024}
    assert not over, f"all-resident kernels fitting fewer than 6 blocks per CU: {over}"


# MXFP4 single-token kernels with both column chunks of a row in flight
# (VEC 32, 4 rows per wave, U1 = 2), x in LDS with and without staged scales.
WHOLE_ROWS = r"k_fused_ffnINS_5fp4x2E(DF16_|f)Li32ELi4ELi2E"


def test_whole_row_mxfp4_kernels_keep_two_waves_per_simd(kernels):
    # They run only where every gate/up block of the layer is resident at once
    # at their own occupancy (queried at launch), which needs at least 2
    # blocks of 4 waves per CU.
    whole = {k: v["vgpr_alloc"] for k, v in kernels.items() if re.search(WHOLE_ROWS, k)}
    assert len(whole) == 4, sorted(whole)
    assert all(re.search(r"ELb1ELb[01]ELb0ELb0EEEv", k) for k in whole), "x-in-LDS variants only"
    over = {k: n for k, n in whole.items() if n > 256}
    assert not over, f"whole-row MXFP4 kernels allocating more than 256 VGPRs: {over}"


def test_register_path_kernels_hold_no_per_thread_arrays_in_lds(kernels):
    # Without x staged in LDS (k_fused_ffn<..., false>, k_gateup, k_down) a
    # kernel's LDS is its few block-shared words (partial sums, fp8 down
    # scales, the logits of E > 16) plus, in the fused kernel with 16-byte
    # weight vectors (f16 / bf16 VEC 8, fp8 VEC 16, f32 VEC 4), the down
    # blocks' 32 KB prefetch buffer.  A per-thread array promoted to LDS adds 256 copies
    # of itself (the TopK selection, 48 bytes, once took 12 KB there, and
    # every read of it waited between weight loads).
    def limit(k):
        pre = re.search(r"k_fused_ffnI(DF16_|NS_5bf16wE)(DF16_|f)Li8E|"
                        r"k_fused_ffnINS_4fp8wE(DF16_|f)Li16E|k_fused_ffnIf(DF16_|f)Li4E", k)
        return 1024 + (32768 if pre else 0)

    reg = {k: v.get("group_segment_fixed_size", 0) for k, v in kernels.items()
           if ("k_fused_ffn" in k and re.search(r"ELb0ELb0ELb[01]ELb[01]EEEv", k)) or "k_gateup" in k
           or "k_down" in k}
    assert len(reg) >= 16, sorted(reg)
    big = {k: n for k, n in reg.items() if n > limit(k)}
    assert not big, f"register-path kernels with more LDS than their buffers: {big}"


def test_x_in_lds_kernels_fit_four_blocks_per_cu(kernels):
    # The x-in-LDS single-token kernels (k_fused_ffn<..., true, STG, ...>) size their
    # buffer for 4 blocks of 4 waves per CU: at most 40 KB of the CU's 160 KB
    # each.  The MXFP4 staged-scale kernels fill that budget (their down
    # blocks stage one more weight chunk per wave in the x copy's bytes).
    xl = {k: v.get("group_segment_fixed_size", 0) for k, v in kernels.items()
          if "k_fused_ffn" in k and re.search(r"ELb1ELb[01]ELb0ELb0EEEv", k)}
    assert len(xl) >= 8, sorted(xl)
    assert all(n > 0 for n in xl.values()), xl
    big = {k: n for k, n in xl.items() if n > 40 * 1024}
    assert not big, f"x-in-LDS kernels over 40 KB of LDS: {big}"
    stg = [n for k, n in xl.items() if re.search(r"ELb1ELb1ELb0ELb0EEEv", k)]
    assert stg and min(stg) > 36 * 1024, f"staged-scale kernels without their chunk buffer: {stg}"


def test_bounded_gateup_tiles_fit_their_blocks_per_cu(kernels):
    # k_gu_mfma<WT, LO, TOK, ROUTE, KC> with a minimum-blocks launch bound:
    # 64-token tiles of fp8 and MXFP4 weights at 3 blocks of 4 waves per CU
    # (168 VGPRs, 3 x LDS <= 160 KB), 32-token tiles of fp8 weights with the lo
    # term of x at 4 (128 VGPRs, 4 x LDS <= 160 KB), 16-token tiles of fp8
    # weights in 256-column steps at 3 (their weight tiles swizzled, not
    # padded, to fit the LDS).
    # (The template arguments end with the token and the weight K step; MXFP4's
    # 64-token kernel with 256-column weight steps holds 2 blocks, unbounded.)
    want = {r"k_gu_mfmaINS_4fp8wELb[01]ELi64ELb0ELi128ELi128E": 3,
            r"k_gu_mfmaINS_5fp4x2ELb1ELi64ELb0ELi128ELi128E": 3,
            r"k_gu_mfmaINS_4fp8wELb1ELi32ELb0ELi128ELi128E": 4,
            r"k_gu_mfmaINS_4fp8wELb[01]ELi16ELb1ELi256ELi256E": 3}
    for pat, blocks in want.items():
        ks = {k: v for k, v in kernels.items() if re.search(pat, k)}
        assert ks, pat
        for k, v in ks.items():
            assert 0 < v["vgpr_alloc"] <= 512 // blocks // 8 * 8, (k, v["vgpr_alloc"])
            assert blocks * v.get("group_segment_fixed_size", 0) <= 160 * 1024, (k, v)
