"""ctypes binding of oracle/qattn_oracle.c (TEST INFRASTRUCTURE ONLY)."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import build as _build

_lib = None


def lib():
    global _lib
    if _lib is None:
        if _build.needs_build():
            _build.build()
        L = C.CDLL(_build.LIB)
        i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
        f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
        L.oracle_num_tree_nodes.restype = C.c_int64
        L.oracle_num_tree_nodes.argtypes = [C.c_int, C.c_int]
        L.oracle_build_tree.restype = C.c_int64
        L.oracle_build_tree.argtypes = [C.c_int, C.c_int, i32p, C.c_int64]
        L.oracle_ancestor_table_heap.restype = None
        L.oracle_ancestor_table_heap.argtypes = [i32p, C.c_int, C.c_int, C.c_int, i32p]
        L.oracle_ancestor_table_parents.restype = None
        L.oracle_ancestor_table_parents.argtypes = [i32p, C.c_int, i32p, C.c_int, i32p]
        L.oracle_tree_attn.restype = None
        L.oracle_tree_attn.argtypes = [
            f32p, f32p, f32p, i32p, C.c_int, C.c_int, C.c_int, C.c_int,
            i32p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_double,
            f64p, C.c_void_p]
        L.oracle_lse_merge.restype = None
        L.oracle_lse_merge.argtypes = [f32p, f32p, f32p, f32p, C.c_int64, C.c_int, f64p]
        _lib = L
    return _lib


def num_tree_nodes(b: int, d: int) -> int:
    return int(lib().oracle_num_tree_nodes(b, d))


def build_tree(b: int, d: int) -> np.ndarray:
    n = num_tree_nodes(b, d)
    out = np.empty(max(n, 1), dtype=np.int32)
    got = lib().oracle_build_tree(b, d, out, out.size)
    assert got == n
    return out[:n]


def ancestor_table_heap(cu, b: int, max_depth: int) -> np.ndarray:
    cu = np.ascontiguousarray(np.asarray(cu, dtype=np.int32))
    T = int(cu[-1])
    out = np.empty((T, max_depth + 1), dtype=np.int32)
    lib().oracle_ancestor_table_heap(cu, len(cu) - 1, b, max_depth, out)
    return out


def ancestor_table_parents(cu, parents, max_depth: int) -> np.ndarray:
    cu = np.ascontiguousarray(np.asarray(cu, dtype=np.int32))
    parents = np.ascontiguousarray(np.asarray(parents, dtype=np.int32))
    T = int(cu[-1])
    out = np.empty((T, max_depth + 1), dtype=np.int32)
    lib().oracle_ancestor_table_parents(cu, len(cu) - 1, parents, max_depth, out)
    return out


def tree_attn(q, k, v, cu, anc, scale: float, kp=None, vp=None, want_lse: bool = True):
    """Double-precision sparse ancestor attention.

    q [T,Hq,D], k/v [T,Hkv,D] float arrays; anc [T,S1] int32 table;
    kp/vp optional [B,L,Hkv,D] all-attended prefix rows.
    Returns (o [T,Hq,D] float64, lse [T,Hq] float64 or None).
    """
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    cu = np.ascontiguousarray(np.asarray(cu, dtype=np.int32))
    anc = np.ascontiguousarray(anc, dtype=np.int32)
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    B = len(cu) - 1
    L = 0
    kp_ptr = vp_ptr = None
    if kp is not None:
        kp = np.ascontiguousarray(kp, dtype=np.float32)
        vp = np.ascontiguousarray(vp, dtype=np.float32)
        assert kp.shape[0] == B and kp.shape[2] == Hkv and kp.shape[3] == D
        L = kp.shape[1]
        kp_ptr = kp.ctypes.data
        vp_ptr = vp.ctypes.data
    o = np.empty((T, Hq, D), dtype=np.float64)
    lse = np.empty((T, Hq), dtype=np.float64) if want_lse else None
    lib().oracle_tree_attn(q, k, v, cu, B, Hq, Hkv, D, anc, anc.shape[1],
                           kp_ptr, vp_ptr, L, float(scale), o,
                           lse.ctypes.data if want_lse else None)
    return o, lse


def lse_merge(lse_p, lse_t, o_p, o_t) -> np.ndarray:
    lse_p = np.ascontiguousarray(lse_p, dtype=np.float32).reshape(-1)
    lse_t = np.ascontiguousarray(lse_t, dtype=np.float32).reshape(-1)
    shape = o_p.shape
    D = shape[-1]
    o_p = np.ascontiguousarray(o_p, dtype=np.float32).reshape(-1, D)
    o_t = np.ascontiguousarray(o_t, dtype=np.float32).reshape(-1, D)
    out = np.empty(o_p.shape, dtype=np.float64)
    lib().oracle_lse_merge(lse_p, lse_t, o_p, o_t, o_p.shape[0], D, out)
    return out.reshape(shape)
