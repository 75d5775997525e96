"""In-tree build of the gfx950 MoE library and its torch extension.

  libwarp_route_hip.so  hipcc --offload-arch=gfx950, from csrc/*.hip; exports
                        exactly the C-ABI of include/warp_route.h
  _C.<ext-suffix>.so    the pybind11/torch module warp_route._C, compiled
                        from csrc/bindings.cpp with the host compiler and
                        linked against libwarp_route_hip.so (rpath $ORIGIN)
  libwr_probe.so        the read-only HBM streaming probe bench.py uses for
                        the achievable-bandwidth ceiling (include/wr_probe.h);
                        a measurement utility, not part of the MoE library

Both land in warp_route/ so that the package directory is self-contained and
travels with the source tree.  Run ``python warp-route_amd/build.py``.

WR_HIPCC_FLAGS in the environment adds hipcc options to every HIP compile:
the kernels' tuning macros (#ifndef WR_... in csrc/) are set that way, e.g.
``WR_HIPCC_FLAGS=-DWR_POLL_ONE=0 python warp-route_amd/build.py`` builds the
single-token kernel's down blocks polling all 64 arrival words from the start.
Tests assume the defaults.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shlex
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
CSRC = HERE / "csrc"
PKG = HERE / "warp_route"
INCLUDE = REPO / "include"
BUILD = HERE / "_build"
LIB_NAME = "libwarp_route_hip.so"

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = shutil.which("hipcc") or f"{ROCM}/bin/hipcc"

# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    *shlex.split(os.environ.get("WR_HIPCC_FLAGS", "")),
]
HIP_SOURCES = ["wr_api.hip", "wr_kernels.hip", "wr_batched.hip", "wr_naive.hip"]
PROBE_SOURCE = "wr_probe.hip"
PROBE_NAME = "libwr_probe.so"


def _run(cmd, **kw):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, **kw)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(map(str, cmd))}\n{out}")
    return out


def build_lib(verbose: bool = False) -> Path:
    """Compile csrc/*.hip for gfx950 and link libwarp_route_hip.so."""
    BUILD.mkdir(exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = BUILD / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(CSRC / src),
                     "-o", str(obj)])
    with cf.ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        for out in ex.map(_run, cmds):
            if verbose and out.strip():
                print(out)
    lib = PKG / LIB_NAME
    tmp = BUILD / LIB_NAME
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, lib)
    return lib


def build_probe(verbose: bool = False) -> Path:
    """Compile csrc/wr_probe.hip into libwr_probe.so."""
    BUILD.mkdir(exist_ok=True)
    tmp = BUILD / PROBE_NAME
    out = _run([HIPCC, *HIP_FLAGS, "-shared", f"-I{INCLUDE}", str(CSRC / PROBE_SOURCE),
                "-o", str(tmp)])
    if verbose and out.strip():
        print(out)
    lib = PKG / PROBE_NAME
    os.replace(tmp, lib)
    return lib


def _ext_suffix() -> str:
    return sysconfig.get_config_var("EXT_SUFFIX") or ".so"


def build_ext(verbose: bool = False) -> Path:
    """Compile csrc/bindings.cpp into warp_route/_C<ext-suffix>."""
    import torch
    from torch.utils import cpp_extension as ce

    BUILD.mkdir(exist_ok=True)
    incs = list(ce.include_paths(device_type="cuda")) + [sysconfig.get_paths()["include"],
                                                          str(INCLUDE)]
    libdirs = list(ce.library_paths(device_type="cuda"))
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    out = PKG / ("_C" + _ext_suffix())
    tmp = BUILD / out.name
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
           "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           *[f"-I{d}" for d in incs], str(CSRC / "bindings.cpp"), "-o", str(tmp),
           *[f"-L{d}" for d in libdirs], f"-L{PKG}",
           "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip", "-ltorch_hip",
           "-lamdhip64", "-lwarp_route_hip", "-Wl,-rpath,$ORIGIN"]
    o = _run(cmd)
    if verbose and o.strip():
        print(o)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> None:
    with cf.ThreadPoolExecutor(max_workers=2) as ex:
        probe = ex.submit(build_probe, verbose)
        lib = build_lib(verbose)
        probe = probe.result()
    ext = build_ext(verbose)
    if verbose:
        print(f"built {lib}\nbuilt {ext}\nbuilt {probe}")


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
