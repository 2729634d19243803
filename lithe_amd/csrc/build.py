"""Build liblithe_amd.so (gfx950) from the HIP sources next to this file.

    python -m lithe_amd.csrc.build         # or lithe_amd.csrc.build.build()

Every call recompiles. Packed-fp32 VALU forms are disabled for all device code.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, "include")
OBJ_DIR = os.path.join(HERE, "_obj")
LIB_PATH = os.path.join(PKG, "_lib", "liblithe_amd.so")

SOURCES = ["decode.hip", "lora.hip", "lora_shrink_bf16.hip", "lora_shrink_f32.hip", "lora_expand_bf16_bf16.hip",
           "lora_expand_bf16_f32.hip", "lora_expand_f32_bf16.hip", "lora_expand_f32_f32.hip", "ingest.hip",
           "encode.hip", "host.cpp"]
ARCH = os.environ.get("LITHE_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; install ROCm or set HIPCC")


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), "-c", "-fPIC", "-O3", "-std=c++17", "-Wall", "-Wno-unused-function",
           f"--offload-arch={ARCH}", "-I", INCLUDE, "-I", HERE,
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           os.path.join(HERE, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd = [hipcc(), "-c", "-fPIC", "-O3", "-std=c++17", "-Wall", "-I", INCLUDE,
               os.path.join(HERE, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compiling {src} failed:\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(os.path.dirname(LIB_PATH), exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp, "-lpthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"linking liblithe_amd.so failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
