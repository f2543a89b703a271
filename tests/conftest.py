"""Shared fixtures and case generators for the test suite.

Markers: `gpu` = needs a ROCm GPU and the built libqattn.so.  Run the CPU part
with `pytest -m "not gpu"`, the parity tests with `pytest -m gpu`.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libqattn.so")


def gpu_available() -> bool:
    try:
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if gpu_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def seed_of(B: int, b: int, d: int) -> int:
    """Input seed convention of the reference benchmarks (scripts/benchmark_micro.py:303)."""
    return B * 10000 + b * 100 + d


def num_tree_nodes(b: int, d: int) -> int:
    return d + 1 if b == 1 else (b ** (d + 1) - 1) // (b - 1)


def make_inputs(lens, Hq: int, D: int, seed: int, dtype=torch.float16, Hkv: int = None,
                sigma: float = 1.0):
    """CPU-generated packed inputs: Q, then K, then V, drawn fp32 N(0, sigma^2)
    from one explicit generator, cast to `dtype`.  Returns (Q, K, V, cu)."""
    Hkv = Hq if Hkv is None else Hkv
    T = int(sum(lens))
    g = torch.Generator().manual_seed(seed)
    Q = (torch.randn(T, Hq, D, generator=g) * sigma).to(dtype)
    K = (torch.randn(T, Hkv, D, generator=g) * sigma).to(dtype)
    V = (torch.randn(T, Hkv, D, generator=g) * sigma).to(dtype)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    return Q, K, V, cu


def tree_case(B: int, b: int, d: int, H: int, D: int, dtype=torch.float16, seed=None, Hkv=None):
    N = num_tree_nodes(b, d)
    s = seed_of(B, b, d) if seed is None else seed
    return make_inputs([N] * B, H, D, s, dtype, Hkv=Hkv)


def oracle_tree(Q, K, V, cu, b: int, max_depth: int, parents=None, Kp=None, Vp=None):
    """fp64 sparse-walk oracle on the (already rounded) inputs.
    Returns (O float64 [T,Hq,D], LSE float64 [T,Hq], ancestor table)."""
    from oracle import clib
    cu_np = cu.numpy().astype(np.int32)
    if parents is None:
        anc = clib.ancestor_table_heap(cu_np, b, max_depth)
    else:
        anc = clib.ancestor_table_parents(cu_np, np.asarray(parents, dtype=np.int32), max_depth)
    D = Q.shape[-1]
    kp = None if Kp is None else Kp.float().numpy()
    vp = None if Vp is None else Vp.float().numpy()
    o, lse = clib.tree_attn(Q.float().numpy(), K.float().numpy(), V.float().numpy(), cu_np, anc,
                            1.0 / np.sqrt(D), kp, vp)
    return o, lse, anc
