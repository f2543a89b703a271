"""Build libqattn.so (gfx950) in-tree with hipcc.

    python -m qattention_amd.build

The library is a plain C-ABI shared object: it links only the HIP runtime.
When loaded into a process that has already imported torch, the dynamic
linker resolves libamdhip64.so.7 to torch's copy, so torch's streams and
allocations are valid handles for it.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_PATH = os.path.join(PKG_DIR, "libqattn.so")
SOURCES = ["tree_attn.hip", "subtree_stream.hip", "prefix_attn.hip"]
HEADERS = ["qattn_common.h", "qattn_device.h", "tree_walk.h"]
ARCH = os.environ.get("QATTN_ARCH", "gfx950")


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def compile_flags() -> list:
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        # packed fp32 VALU ops stay off (correctness issue on this platform)
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # one-lane counter atomics stay single instructions: the atomic
        # optimizer would turn each into a wave reduction that waits for the
        # answer at once, where the subtree kernel overlaps it with its loads
        "-Xarch_device", "-mllvm=-amdgpu-atomic-optimizer-strategy=None",
        "-Wall", "-Wno-unused-function",
    ]


def build(verbose: bool = True) -> str:
    """Compile every HIP source into qattention_amd/libqattn.so (always rebuilds)."""
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), *compile_flags(), "-shared", "-o", tmp, *srcs]
    if verbose:
        print("[qattention_amd.build]", " ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def is_stale() -> bool:
    if not os.path.exists(LIB_PATH):
        return True
    t = os.path.getmtime(LIB_PATH)
    deps = [os.path.join(CSRC, f) for f in SOURCES + HEADERS]
    deps.append(os.path.join(PKG_DIR, "..", "include", "qattn.h"))
    return any(os.path.getmtime(d) > t for d in deps if os.path.exists(d))


if __name__ == "__main__":
    print(build())
