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
OBJ_DIR = os.path.join(PKG_DIR, "_build")
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
        # inline assembly must not clobber registers the compiler reserves
        # (M0, EXEC, VCC): such an asm statement is undefined behaviour
        "-Werror=inline-asm",
    ]


def _run(cmd, verbose):
    if verbose:
        print("[qattention_amd.build]", " ".join(cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)


def _finish(proc, verbose):
    _, stderr = proc.communicate()
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = True) -> str:
    """Compile every HIP source into qattention_amd/libqattn.so (always rebuilds).

    Each source is compiled to an object in its own hipcc process (they run
    in parallel), then the objects are linked into the shared library."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    objs, procs = [], []
    for s in SOURCES:
        obj = os.path.join(OBJ_DIR, os.path.splitext(s)[0] + ".o")
        objs.append(obj)
        procs.append(_run([_hipcc(), *compile_flags(), "-c", "-o", obj, os.path.join(CSRC, s)], verbose))
    for proc in procs:
        _finish(proc, verbose)
    tmp = LIB_PATH + ".tmp"
    _finish(_run([_hipcc(), f"--offload-arch={ARCH}", "-shared", "-o", tmp, *objs], verbose), verbose)
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
