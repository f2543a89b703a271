"""ctypes binding of libqattn.so (the C ABI declared in include/qattn.h).

The library must be built in-tree (python -m qattention_amd.build).  There is
no fallback: if it is missing, every call raises.
"""
from __future__ import annotations

import contextlib
import ctypes as C
import os

import torch  # must be loaded first so libqattn.so binds torch's HIP runtime

from .build import LIB_PATH

QATTN_OK = 0
ERRORS = {
    -1: "QATTN_ERR_ARG",
    -2: "QATTN_ERR_DTYPE",
    -3: "QATTN_ERR_HEAD_DIM",
    -4: "QATTN_ERR_LAYOUT",
    -5: "QATTN_ERR_WORKSPACE",
    -6: "QATTN_ERR_HIP",
}
QATTN_ERR_LAYOUT = -4

DTYPE_F16 = 0
DTYPE_BF16 = 1
ALGO_AUTO, ALGO_GATHER, ALGO_SUBTREE = 0, 1, 2

# Every symbol declared in include/qattn.h, with its ctypes signature.
_p = C.c_void_p
_i32 = C.c_int32
_i64 = C.c_int64
_f32 = C.c_float
_i64p = C.POINTER(C.c_int64)

SIGNATURES = {
    "qattn_version": (C.c_char_p, []),
    "qattn_last_error": (C.c_char_p, []),
    "qattn_init": (C.c_int, []),
    "qattn_sched_info": (C.c_int, [_i64p]),
    "qattn_debug_walk": (C.c_int, [_p]),
    "qattn_tree_fwd": (C.c_int, [
        _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p,
        _p, _i32, _i32, _i64, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _p]),
    "qattn_tree_parents_fwd": (C.c_int, [
        _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p,
        _p, _p, _i32, _i32, _i64, _i32, _i32, _i32, _i32, _f32, _i32, _p]),
    "qattn_tree_paged_fwd": (C.c_int, [
        _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p,
        _p, _p, _i32, _i32, _i32, _i32, _i32, _i64, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _p]),
    "qattn_ancestors": (C.c_int, [_p, _p, _i32, _i32, _i64, _i32, _i32, _p, _p]),
    "qattn_prefix_workspace_bytes": (C.c_int64, [_i32, _i32, _i64, _i32, _i32, _i32, _i32, _i32]),
    "qattn_prefix_tree_fwd": (C.c_int, [
        _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _i32,
        _p, _i64p, _p, _i64p, _p, _i32, _i32, _i64, _i64, _i64,
        _i32, _i32, _i32, _i32, _i32, _f32, _i32, _p, _i64, _i32, _p]),
    "qattn_prefix_fwd": (C.c_int, [
        _p, _i64p, _p, _i64p, _p, _i64p, _i32, _p, _i64p, _p, _i64p,
        _p, _i32, _i32, _i64, _i32, _i32, _i32, _f32, _i32, _p, _i64, _i32, _p]),
    "qattn_prefix_tree_parents_fwd": (C.c_int, [
        _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _i32,
        _p, _i64p, _p, _i64p, _p, _p, _i32, _i32, _i64, _i64, _i64,
        _i32, _i32, _i32, _i32, _f32, _i32, _p, _i64, _i32, _p]),
    "qattn_ragged_tree_attn_fwd": (C.c_int, [
        _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64,
        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _p, _i64, _i32, _p]),
    "qattn_ragged_tree_attn_fwd_noalloc": (C.c_int, [
        _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64,
        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _p]),
    "qattn_lse_merge": (C.c_int, [
        _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p,
        _i32, _i32, _i32, _i32, _i32, _p]),
}

_lib = None


class QAttnError(RuntimeError):
    pass


def lib():
    """Load libqattn.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise QAttnError(
                f"{LIB_PATH} is missing: build it with `python -m qattention_amd.build` "
                "(or __graft_entry__.build()); there is no non-HIP fallback")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


_initialised = set()


def ensure_init(device) -> None:
    """qattn_init() once per device, outside graph capture (the library then
    gives the subtree kernel its schedule counters on that device; a call
    made before it, e.g. the first one inside a capture, runs the static
    schedule)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx in _initialised or torch.cuda.is_current_stream_capturing():
        return
    with torch.cuda.device(idx):
        check(lib().qattn_init(), "qattn_init")
    _initialised.add(idx)


@contextlib.contextmanager
def debug_walk(table):
    """While active, attention calls on this thread also write the ancestor
    set each query attended, as the kernels used it, into `table` (a device
    int32 tensor [total_tokens, num_q_heads, max_depth + 1]; see
    qattn_debug_walk in include/qattn.h)."""
    check(lib().qattn_debug_walk(table.data_ptr()), "qattn_debug_walk")
    try:
        yield table
    finally:
        lib().qattn_debug_walk(None)


def sched_info(device=None) -> dict:
    """Schedule-counter use on a device (qattn_sched_info): slots held and
    how many subtree launches ran with counters or fell back to the static
    schedule."""
    arr = (C.c_int64 * 6)()
    with torch.cuda.device(device if device is not None else torch.cuda.current_device()):
        check(lib().qattn_sched_info(arr), "qattn_sched_info")
    keys = ("stream_slots", "capture_slots", "dynamic_launches", "static_launches",
            "stream_capacity", "capture_capacity")
    return dict(zip(keys, [int(x) for x in arr]))


def last_error() -> str:
    return lib().qattn_last_error().decode(errors="replace")


def check(rc: int, what: str) -> None:
    if rc != QATTN_OK:
        raise QAttnError(f"{what} failed: {ERRORS.get(rc, rc)}: {last_error()}")


def i64arr(vals):
    arr = (C.c_int64 * len(vals))(*[int(x) for x in vals])
    return arr


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()
