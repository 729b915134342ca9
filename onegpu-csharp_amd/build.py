"""Builds the MI355X int8 path in-tree:

  lib/libonegpu_hip.so            the C-ABI HIP library (include/onegpu_hip.h), gfx950 only
  onegpu_hip/_onegpu_host*.so     the host layer (host/onegpu.hpp, the reference's Int8Gemm / DynamicQuantizeKernels /
                                  DequantizeKernels API in C++) with its Python binding

Run directly (python onegpu-csharp_amd/build.py) or through __graft_entry__.build(). Always recompiles.
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
INCLUDE = os.path.join(ROOT, "include")
CSRC = os.path.join(HERE, "csrc")
HOST = os.path.join(HERE, "host")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "lib", "libonegpu_hip.so")
PKG = os.path.join(HERE, "onegpu_hip")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Exact arithmetic flags: no fused multiply-add, IEEE division, denormals kept. Packed FP32 instructions are kept off.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", f"-I{INCLUDE}", f"-I{CSRC}",
    "-ffp-contract=off", "-fno-fast-math", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed: {' '.join(cmd)}\n{out}")
    if out.strip() and os.environ.get("OG_BUILD_VERBOSE"):
        print(out)


def build_hip() -> str:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    objs = [os.path.join(OBJ, os.path.basename(s)[:-4] + ".o") for s in srcs]
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(lambda so: _run([HIPCC, *HIP_FLAGS, "-c", so[0], "-o", so[1]]), zip(srcs, objs)))
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    return LIB


def build_host() -> str:
    import pybind11

    os.makedirs(PKG, exist_ok=True)
    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(PKG, "_onegpu_host" + suffix)
    srcs = [os.path.join(HOST, "onegpu.cpp"), os.path.join(HOST, "pymodule.cpp")]
    py_inc = sysconfig.get_paths()["include"]
    tmp = out + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", f"-I{INCLUDE}", f"-I{HOST}",
          f"-I{pybind11.get_include()}", f"-I{py_inc}", *srcs, "-o", tmp,
          f"-L{os.path.dirname(LIB)}", "-lonegpu_hip", "-Wl,-rpath,$ORIGIN/../lib"])
    os.replace(tmp, out)
    return out


def build_oracle() -> None:
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)


def build_all() -> None:
    build_hip()
    build_host()
    build_oracle()


if __name__ == "__main__":
    build_all()
    print("built", LIB)
    sys.exit(0)
