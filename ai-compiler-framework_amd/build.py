"""Builds the gfx950 backend in-tree.

Outputs (next to the Python package that loads them):
  python/aicf_cuda/libaicf_hip.so   C-ABI library: registry, kernels, graph runtime
  python/aicf_cuda/_C<ext>.so       pybind module calling only the C-ABI

Device code is compiled by hipcc for gfx950 only; host-only C++ by g++.
Run:  python ai-compiler-framework_amd/build.py  [--jobs N]
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "python" / "aicf_cuda"
OBJ_DIR = PKG / "_build"
INCLUDE = REPO / "include"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")

HIP_SOURCES = ["kernels/optim.hip", "kernels/eltwise.hip", "kernels/reduce.hip", "kernels/gemm.hip",
               "kernels/norm.hip", "kernels/diag.hip", "kernels/smallstep.hip"]
CXX_SOURCES = ["registry/registry.cpp", "registry/register_all.cpp", "runtime/graph.cpp"]

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # packed-fp32 instructions stay off (hipcc's host pass warns about the
    # unknown feature; that is expected)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-D__HIP_PLATFORM_AMD__",
             f"-I{INCLUDE}", f"-I{ROCM / 'include'}"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops" not in l and "is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def _obj(src: str) -> Path:
    return OBJ_DIR / (src.replace("/", "_") + ".o")


def build_library(jobs: int) -> Path:
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    OUT_DIR.mkdir(parents=True, exist_ok=True)
    cmds = []
    for s in HIP_SOURCES:
        cmds.append([HIPCC, *HIP_FLAGS, "-c", str(CSRC / s), "-o", str(_obj(s))])
    for s in CXX_SOURCES:
        cmds.append(["g++", *CXX_FLAGS, "-c", str(CSRC / s), "-o", str(_obj(s))])
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    lib = OUT_DIR / "libaicf_hip.so"
    tmp = lib.with_suffix(".so.tmp")
    objs = [str(_obj(s)) for s in HIP_SOURCES + CXX_SOURCES]
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *objs,
          f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}",
          "-Wl,-soname,libaicf_hip.so"])
    os.replace(tmp, lib)
    return lib


def _torch_flags() -> tuple[list[str], list[str]]:
    import torch
    from torch.utils import cpp_extension

    inc = cpp_extension.include_paths()
    tlib = Path(torch.__file__).resolve().parent / "lib"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cflags = [f"-I{p}" for p in inc] + [f"-I{sysconfig.get_paths()['include']}",
                                        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DUSE_ROCM",
                                        "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H"]
    getf = getattr(cpp_extension, "_get_pybind11_abi_build_flags", None)
    if getf is not None:
        cflags += list(getf())
    ldflags = [f"-L{tlib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
               f"-Wl,-rpath,{tlib}"]
    return cflags, ldflags


def build_bindings() -> Path:
    cflags, ldflags = _torch_flags()
    ext = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = OUT_DIR / f"_C{ext}"
    tmp = out.with_suffix(".tmp")
    _run(["g++", *CXX_FLAGS, "-w", *cflags, "-shared", str(CSRC / "bindings" / "bindings.cpp"),
          "-o", str(tmp), f"-L{OUT_DIR}", "-laicf_hip", "-Wl,-rpath,$ORIGIN", *ldflags])
    os.replace(tmp, out)
    return out


def build_all(jobs: int | None = None, bindings: bool = True) -> None:
    jobs = jobs or min(8, os.cpu_count() or 4)
    lib = build_library(jobs)
    print(f"[build] {lib.relative_to(REPO)}")
    if bindings:
        b = build_bindings()
        print(f"[build] {b.relative_to(REPO)}")


def clean() -> None:
    shutil.rmtree(OBJ_DIR, ignore_errors=True)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--no-bindings", action="store_true")
    ap.add_argument("--clean", action="store_true")
    a = ap.parse_args()
    if a.clean:
        clean()
    build_all(a.jobs, bindings=not a.no_bindings)
    sys.exit(0)
