"""Complete-tree helpers restated from the reference's src/tree_mask.py.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
from __future__ import annotations

import numpy as np


def num_tree_nodes(branching_factor: int, depth: int) -> int:
    """src/tree_mask.py:78-83: (b^(d+1) - 1) / (b - 1); b == 1 gives d + 1."""
    b, d = branching_factor, depth
    if b == 1:
        return d + 1
    return (b ** (d + 1) - 1) // (b - 1)


def build_tree(branching_factor: int, depth: int) -> list:
    """src/tree_mask.py:86-113: BFS parent array, root parent -1.

    Written as an explicit frontier expansion (not the closed form (i-1)//b)
    so that agreement with the closed form is a real check.
    """
    b, d = branching_factor, depth
    if b <= 0:
        raise ValueError(f"branching_factor must be >= 1, got {b}")
    if d < 0:
        raise ValueError(f"depth must be >= 0, got {d}")
    parent = [-1]
    frontier = [0]
    for _ in range(d):
        nxt = []
        for node in frontier:
            for _ in range(b):
                parent.append(node)
                nxt.append(len(parent) - 1)
        frontier = nxt
    return parent


def ancestors(node: int, parent_array) -> set:
    """src/tree_mask.py:116-126: path to the root, node included."""
    out = set()
    cur = node
    while cur != -1:
        out.add(cur)
        cur = parent_array[cur]
    return out


def tree_attention_mask(branching_factor: int, depth: int) -> np.ndarray:
    """src/tree_mask.py:301-317: mask[i, j] iff j is an ancestor of i (or i)."""
    parent = build_tree(branching_factor, depth)
    n = len(parent)
    mask = np.zeros((n, n), dtype=bool)
    for i in range(n):
        for a in ancestors(i, parent):
            mask[i, a] = True
    return mask


def tree_attention_mask_n(branching_factor: int, n: int) -> np.ndarray:
    """src/tree_mask.py:320-359: ancestor mask of the first n BFS nodes."""
    b = branching_factor
    parent = np.full(n, -1, dtype=np.int64)
    if n > 1:
        parent[1:] = (np.arange(1, n) - 1) // b
    mask = np.zeros((n, n), dtype=bool)
    for i in range(n):
        j = i
        while j >= 0:
            mask[i, j] = True
            j = int(parent[j])
    return mask


def node_depth(i: int, parent_array) -> int:
    d = 0
    while parent_array[i] != -1:
        i = parent_array[i]
        d += 1
    return d


def verify_tree_mask(branching_factor: int, depth: int) -> bool:
    """src/tree_mask.py:436-494: reflexive, exact ancestor rule, anti-sibling,
    row-sum == depth + 1."""
    parent = build_tree(branching_factor, depth)
    mask = tree_attention_mask(branching_factor, depth)
    n = len(parent)
    for i in range(n):
        if not mask[i, i]:
            return False
        anc = ancestors(i, parent)
        for j in range(n):
            if bool(mask[i, j]) != (j in anc):
                return False
        if int(mask[i].sum()) != node_depth(i, parent) + 1:
            return False
    # anti-sibling: two distinct children of one parent never see each other
    for i in range(1, n):
        for j in range(1, n):
            if i != j and parent[i] == parent[j] and mask[i, j]:
                return False
    return True


def mask_from_table(table: np.ndarray, start: int, n: int) -> np.ndarray:
    """Dense [n, n] mask of one sequence from an ancestor table slice
    (rows start..start+n, entries sequence-local or -1)."""
    mask = np.zeros((n, n), dtype=bool)
    rows = table[start:start + n]
    for i in range(n):
        for a in rows[i]:
            if a >= 0:
                mask[i, a] = True
    return mask
