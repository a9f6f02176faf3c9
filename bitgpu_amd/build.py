"""Build the gfx950 HIP library ``bitgpu_amd/lib/libbitgpu_attn.so`` in-tree with hipcc.

Usage: ``python -m bitgpu_amd.build [--incremental]`` (also called by ``__graft_entry__.build()``,
which always compiles everything).
Every .hip file under csrc/ is compiled for gfx950 and linked into one shared library that
exports the C ABI of include/bitgpu_attn.h.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "lib", "libbitgpu_attn.so")
NODE_SRC = os.path.join(HERE, "node", "bitgpu_attn_napi.c")
NODE_OUT = os.path.join(HERE, "node", "bitgpu_attn.node")
NODE_INC = "/usr/include/node"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # packed FP32 instructions stay off (hipcc's host pass warns it does not know the feature)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", "-Wno-unused-variable",
]


def _headers_mtime() -> float:
    hs = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    hs.append(os.path.join(HERE, "..", "include", "bitgpu_attn.h"))
    return max(os.path.getmtime(h) for h in hs if os.path.exists(h))


def _compile(src: str, incremental: bool = False) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    if incremental and os.path.exists(obj) and os.path.getmtime(obj) > max(os.path.getmtime(src), _headers_mtime()):
        return obj
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = True, incremental: bool = False) -> str:
    """Compile every csrc/*.hip for gfx950 and link the library (``incremental`` skips sources
    whose object is newer than the source and every header: a development shortcut)."""
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda f: _compile(f, incremental), srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    build_node_addon(verbose)
    return LIB


def build_node_addon(verbose: bool = True) -> str | None:
    """The N-API addon for a JS/TypeScript host (needs the Node headers; skipped without them)."""
    if not os.path.isdir(NODE_INC):
        if verbose:
            print("node headers not found; N-API addon not built")
        return None
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-std=c11", "-Wall", f"-I{NODE_INC}", "-DNODE_GYP_MODULE_NAME=bitgpu_attn",
           NODE_SRC, "-o", NODE_OUT + ".tmp", f"-L{os.path.dirname(LIB)}", "-lbitgpu_attn",
           "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN/../lib", "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"N-API addon build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(NODE_OUT + ".tmp", NODE_OUT)
    if verbose:
        print(f"built {NODE_OUT}")
    return NODE_OUT


if __name__ == "__main__":
    try:
        build(incremental="--incremental" in sys.argv)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
