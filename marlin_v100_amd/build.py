"""In-tree build of the gfx950 kernel library and the torch op bindings.

Products (next to this file):
  libmarlin_mi355x.so  -- HIP kernels + the C ABI declared in include/marlin_mi355x.h
  _C.so, _moe_C.so     -- TORCH_LIBRARY bindings registering the reference op schemas,
                          linked against libmarlin_mi355x.so (rpath $ORIGIN)

Usage: python -m marlin_v100_amd.build [--jobs N] [--only-lib]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
ROOT = os.path.dirname(HERE)
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # keep the compiler from forming packed-fp32 VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]

# (the GEMM instance files take longest: they go to the compile pool first)
HIP_SOURCES = [f"gemm_{fmt}_{at}.hip" for fmt in ("u4", "u4b8", "u8", "u8b128", "fp8", "mxfp4",
                                                  "nvfp4", "u4z", "u8z") for at in ("bf16", "f16")] + [
    "capi.hip",
    "repack.hip",
    "aux_kernels.hip",
    "router_kernels.hip",
]

LIB_NAME = "libmarlin_mi355x.so"


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")


def _stale(src: str, obj: str) -> bool:
    """Object older than its source or any header in csrc/ or include/."""
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    deps = [os.path.join(CSRC, src)]
    deps += [os.path.join(CSRC, h) for h in os.listdir(CSRC) if h.endswith(".h")]
    inc = os.path.join(ROOT, "include")
    deps += [os.path.join(inc, h) for h in os.listdir(inc) if h.endswith(".h")]
    return any(os.path.getmtime(d) > t for d in deps)


def _compile_hip(src: str, incremental: bool = False) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    if incremental and not _stale(src, obj):
        return obj
    _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def build_library(jobs: int, incremental: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda src: _compile_hip(src, incremental), HIP_SOURCES))
    out = os.path.join(HERE, LIB_NAME)
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, out)
    return out


def _torch_paths() -> tuple[list[str], str, bool]:
    import torch
    from torch.utils import cpp_extension

    incs = cpp_extension.include_paths()
    libdir = os.path.join(os.path.dirname(torch.__file__), "lib")
    return incs, libdir, bool(torch._C._GLIBCXX_USE_CXX11_ABI)


def _build_binding(ext: str, define: str, incs: list[str], libdir: str, abi: bool) -> str:
    out = os.path.join(HERE, f"{ext}.so")
    tmp = out + ".tmp"
    cxx = os.environ.get("CXX", "g++")
    cmd = [
        cxx, "-O2", "-std=c++17", "-fPIC", "-shared",
        f"-D_GLIBCXX_USE_CXX11_ABI={int(abi)}",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        f"-DMMI_EXT_NAME={ext}", f"-D{define}",
        f"-I{ROCM}/include",
        f"-I{sysconfig.get_paths()['include']}",
        *[f"-I{p}" for p in incs],
        os.path.join(CSRC, "torch_ops.cpp"),
        "-o", tmp,
        f"-L{HERE}", "-lmarlin_mi355x",
        f"-L{libdir}", "-ltorch", "-ltorch_cpu", "-lc10", "-lc10_hip",
        f"-L{ROCM}/lib", "-lamdhip64",
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}",
    ]
    _run(cmd)
    os.replace(tmp, out)
    return out


def build_bindings() -> list[str]:
    incs, libdir, abi = _torch_paths()
    with cf.ThreadPoolExecutor(max_workers=2) as ex:
        futs = [
            ex.submit(_build_binding, "_C", "MMI_BUILD_C", incs, libdir, abi),
            ex.submit(_build_binding, "_moe_C", "MMI_BUILD_MOE_C", incs, libdir, abi),
        ]
        return [f.result() for f in futs]


def build(jobs: int | None = None, only_lib: bool = False, incremental: bool = False) -> list[str]:
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    jobs = jobs or min(8, os.cpu_count() or 4)
    outs = [build_library(jobs, incremental)]
    if not only_lib:
        outs += build_bindings()
    return outs


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--only-lib", action="store_true")
    ap.add_argument("--incremental", action="store_true",
                    help="recompile only sources older than their object (development)")
    args = ap.parse_args()
    for p in build(args.jobs, args.only_lib, args.incremental):
        print("built", os.path.relpath(p, ROOT))
    return 0


if __name__ == "__main__":
    sys.exit(main())
