"""Tree topology and dense-mask helpers (the `src.tree_mask` API, complete trees).

Host-side numpy utilities for callers that build oracles, masks or parent
arrays around the HIP kernels.  Names and semantics follow the reference's
src/tree_mask.py; the implementations here use the heap closed form
parent(i) = (i - 1) // b (BFS order) and vectorised numpy.  The EAGLE-like
random pruned-tree generators of the reference (build_pruned_tree,
sample_balanced_tree_nodes) are out of scope: irregular trees enter through
ragged_attention_with_parents with a caller-supplied parent array.
"""
from __future__ import annotations

import numpy as np


def num_tree_nodes(branching_factor: int, depth: int) -> int:
    """Nodes of a complete b-ary tree of the given depth (src/tree_mask.py:78-83)."""
    b, d = branching_factor, depth
    if b == 1:
        return d + 1
    return (b ** (d + 1) - 1) // (b - 1)


def heap_parents(branching_factor: int, n: int) -> np.ndarray:
    """Parent array of the first n BFS nodes: (i - 1) // b, root -1."""
    parent = np.full(n, -1, dtype=np.int64)
    if n > 1:
        parent[1:] = (np.arange(1, n, dtype=np.int64) - 1) // branching_factor
    return parent


def build_tree(branching_factor: int, depth: int) -> list:
    """BFS parent array of a complete b-ary tree, root parent -1
    (src/tree_mask.py:86-113)."""
    if branching_factor <= 0:
        raise ValueError(f"branching_factor must be >= 1, got {branching_factor}")
    if depth < 0:
        raise ValueError(f"depth must be >= 0, got {depth}")
    return heap_parents(branching_factor, num_tree_nodes(branching_factor, depth)).tolist()


def ancestors(node: int, parent_array) -> set:
    """Nodes on the path from node to the root, node included (src/tree_mask.py:116-126)."""
    out = set()
    cur = node
    while cur != -1:
        out.add(cur)
        cur = parent_array[cur]
    return out


def _mask_from_parents(parent: np.ndarray) -> np.ndarray:
    n = len(parent)
    mask = np.zeros((n, n), dtype=bool)
    rows = np.arange(n)
    cur = rows.copy()
    live = np.ones(n, dtype=bool)
    while live.any():
        mask[rows[live], cur[live]] = True
        nxt = parent[cur]
        live = live & (nxt >= 0) & (nxt != cur)
        cur = np.where(live, nxt, cur)
    return mask


def tree_attention_mask(branching_factor: int, depth: int) -> np.ndarray:
    """[N, N] bool, mask[i, j] iff j is an ancestor of i or j == i
    (src/tree_mask.py:301-317)."""
    return _mask_from_parents(heap_parents(branching_factor, num_tree_nodes(branching_factor, depth)))


def tree_attention_mask_n(branching_factor: int, N: int) -> np.ndarray:
    """Ancestor mask of the first N BFS nodes (src/tree_mask.py:320-359)."""
    return _mask_from_parents(heap_parents(branching_factor, N))


def tree_attention_mask_pruned(parent_array) -> np.ndarray:
    """Ancestor mask of an irregular tree given its parent array, root -1
    (src/tree_mask.py:362-386)."""
    return _mask_from_parents(np.asarray(parent_array, dtype=np.int64))


def full_sequence_mask(ctx_len: int, branching_factor: int, depth: int) -> np.ndarray:
    """[ctx | tree] mask: causal context, every tree token sees all context and
    its ancestors (src/tree_mask.py:389-423)."""
    N = num_tree_nodes(branching_factor, depth)
    total = ctx_len + N
    mask = np.zeros((total, total), dtype=bool)
    mask[:ctx_len, :ctx_len] = np.tril(np.ones((ctx_len, ctx_len), dtype=bool))
    mask[ctx_len:, :ctx_len] = True
    mask[ctx_len:, ctx_len:] = tree_attention_mask(branching_factor, depth)
    return mask


def node_depths(parent_array) -> np.ndarray:
    p = np.asarray(parent_array, dtype=np.int64)
    depth = np.zeros(len(p), dtype=np.int64)
    for i in range(len(p)):
        if p[i] >= 0 and p[i] != i:
            depth[i] = depth[p[i]] + 1
    return depth


def verify_tree_mask(branching_factor: int, depth: int, verbose: bool = True) -> bool:
    """Structural self-check (src/tree_mask.py:436-494): reflexive, exact
    ancestor rule, siblings never see each other, row sum == depth + 1."""
    parent = np.asarray(build_tree(branching_factor, depth), dtype=np.int64)
    mask = tree_attention_mask(branching_factor, depth)
    n = len(parent)
    ok = bool(mask.diagonal().all())
    d = node_depths(parent)
    ok &= bool((mask.sum(1) == d + 1).all())
    for i in range(n):
        anc = ancestors(i, parent.tolist())
        row = np.zeros(n, dtype=bool)
        row[list(anc)] = True
        ok &= bool((row == mask[i]).all())
    sib = (parent[:, None] == parent[None, :]) & ~np.eye(n, dtype=bool) & (parent[:, None] >= 0)
    ok &= not bool((mask & sib).any())
    if verbose:
        print(f"[verify_tree_mask] b={branching_factor} d={depth} N={n}  ->  {'PASS' if ok else 'FAIL'}")
    return ok


def kernel_parents(parent_array) -> np.ndarray:
    """Parent array in the convention of ragged_attention_with_parents: the
    root self-loops instead of holding -1 (scripts/benchmark_micro.py:283-285)."""
    p = np.asarray(parent_array, dtype=np.int64).copy()
    roots = p < 0
    p[roots] = np.nonzero(roots)[0]
    return p.astype(np.int32)
