"""Build recipe for the gfx950 library and its Node-API addon.

    python web-xpu-ops_amd/build.py          # or __graft_entry__.build()

Produces, in-tree (git-ignored, shipped with the tree to the GPU box):
  web-xpu-ops_amd/lib/libwxo_q8.so    HIP kernels + C ABI (include/wxo_q8.h)
  web-xpu-ops_amd/lib/wxo_q8.node     Node-API addon over the C ABI

hipcc cross-compiles for gfx950 without a GPU.  Every HIP file is built with
packed-FP32 instructions disabled (v_pk_fma_f32 and friends are not emitted).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
NAPI = os.path.join(PKG, "napi")
LIB_DIR = os.path.join(PKG, "lib")
OBJ_DIR = os.path.join(PKG, "lib", "obj")
LIB = os.path.join(LIB_DIR, "libwxo_q8.so")
ADDON = os.path.join(LIB_DIR, "wxo_q8.node")
INCLUDE = os.path.join(ROOT, "include")

HIP_SOURCES = ["matvec_q8.hip", "quantize_q8.hip", "matmul_q8.hip", "dequant_q8.hip", "roofline.hip", "wxo_api.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    # gfx950 firmware loads the first kernel arguments (up to 16 SGPRs) into
    # SGPRs at wave launch, so a wave's first buffer loads do not wait on a
    # kernarg fetch from memory.  Only scalar (non-struct) arguments qualify.
    # The code object keeps a prologue that loads them itself for firmware
    # without the feature.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]
# quantize must round x * inverse before comparing its fraction (JS semantics):
# no multiply-add contraction in that file.
PER_FILE_FLAGS = {"quantize_q8.hip": ["-ffp-contract=off"]}
NODE_INCLUDE = "/usr/include/node"


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"  # host pass only
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build_library(verbose: bool = False) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    build_id = time.strftime("%Y%m%d-%H%M%S")
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = os.path.join(OBJ_DIR, src.replace(".hip", ".o"))
        objs.append(obj)
        extra = PER_FILE_FLAGS.get(src, [])
        cmds.append([HIPCC, *HIP_FLAGS, *extra, f"-DWXO_BUILD_ID=\"{build_id}\"", "-I", INCLUDE, "-I", CSRC,
                     "-c", os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB)
    return LIB


def build_addon(verbose: bool = False) -> str | None:
    """Node-API addon (plain C against node_api.h), linked to libwxo_q8.so with
    an $ORIGIN rpath so it loads from lib/ wherever the tree is."""
    if not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")):
        print("build: node_api.h not found; skipping the Node-API addon", file=sys.stderr)
        return None
    cc = shutil.which("gcc") or "cc"
    tmp = ADDON + ".tmp"
    _run([cc, "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-Wextra", "-DNAPI_VERSION=8", "-DNODE_GYP_MODULE_NAME=wxo_q8",
          "-I", NODE_INCLUDE, "-I", INCLUDE, os.path.join(NAPI, "wxo_napi.c"),
          "-o", tmp, "-L", LIB_DIR, "-lwxo_q8", "-Wl,-rpath,$ORIGIN"], verbose)
    os.replace(tmp, ADDON)
    return ADDON


def build(verbose: bool = False) -> None:
    build_library(verbose)
    if os.path.exists(os.path.join(NAPI, "wxo_napi.c")):
        build_addon(verbose)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(LIB)
