"""Pin the CPU oracle (oracle/) before trusting it (runs without a GPU).

The reference ships no golden vectors, so each oracle function is pinned by
checks chosen so that a plausible mistake fails one of them:
  * known answers (build_tree b=2 d=2, src/tree_mask.py:86-113 docstring case),
  * structural invariants of src/tree_mask.py:436-494,
  * agreement of two independent formulations (integer walk table vs dense
    mask from an explicit frontier expansion; fp64 sparse walk in C vs
    padded SDPA through torch's MATH backend),
  * special cases that reduce to a library routine (b=1 == causal SDPA,
    d=0 == V, full prefix == unmasked SDPA),
  * brute force on tiny inputs (pure-Python loops),
  * planted mistakes: mutated oracles that these checks must reject.
The committed fixtures in tests/golden are then checked against the oracle.
"""
from __future__ import annotations

import glob
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import GOLDEN_DIR, make_inputs, num_tree_nodes, oracle_tree
from oracle import clib, sdpa, tree


# ---------------------------------------------------------------------------
# tree topology
# ---------------------------------------------------------------------------

def test_build_tree_known_answer():
    assert tree.build_tree(2, 2) == [-1, 0, 0, 1, 1, 2, 2]
    assert clib.build_tree(2, 2).tolist() == [-1, 0, 0, 1, 1, 2, 2]
    assert tree.build_tree(3, 1) == [-1, 0, 0, 0]
    assert tree.build_tree(1, 3) == [-1, 0, 1, 2]


@pytest.mark.parametrize("b,d", [(1, 0), (1, 5), (2, 3), (3, 4), (4, 5), (8, 3), (28, 2)])
def test_num_tree_nodes(b, d):
    n = num_tree_nodes(b, d)
    assert tree.num_tree_nodes(b, d) == n == clib.num_tree_nodes(b, d)
    assert len(tree.build_tree(b, d)) == n
    assert clib.build_tree(b, d).tolist() == tree.build_tree(b, d)


@pytest.mark.parametrize("b,d", [(1, 4), (2, 3), (3, 2), (4, 2), (2, 5)])
def test_tree_mask_invariants(b, d):
    assert tree.verify_tree_mask(b, d)


@pytest.mark.parametrize("b,d", [(1, 6), (2, 4), (3, 3), (4, 3), (5, 2)])
def test_heap_closed_form_matches_frontier_expansion(b, d):
    par = tree.build_tree(b, d)
    n = len(par)
    closed = [-1] + [(i - 1) // b for i in range(1, n)]
    assert par == closed
    # first-n BFS prefix mask equals the complete-tree mask
    assert (tree.tree_attention_mask_n(b, n) == tree.tree_attention_mask(b, d)).all()


# ---------------------------------------------------------------------------
# ancestor tables (the walk of src/ragged_attn.py:323-377)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("b,d", [(1, 8), (2, 3), (2, 6), (3, 4), (4, 3), (8, 2)])
def test_heap_table_equals_tree_mask(b, d):
    n = num_tree_nodes(b, d)
    cu = np.array([0, n, 2 * n], dtype=np.int32)
    t = clib.ancestor_table_heap(cu, b, d)
    m = tree.tree_attention_mask(b, d)
    assert (tree.mask_from_table(t, 0, n) == m).all()
    assert (tree.mask_from_table(t, n, n) == m).all()
    # row sums = depth + 1 and the attended steps are a prefix of the row
    par = tree.build_tree(b, d)
    for i in range(n):
        row = t[i]
        k = tree.node_depth(i, par) + 1
        assert (row[:k] >= 0).all() and (row[k:] == -1).all()


@pytest.mark.parametrize("b,n,md", [(2, 31, 2), (3, 40, 1), (1, 9, 3), (4, 100, 0)])
def test_heap_table_truncation(b, n, md):
    """max_depth below the true depth: a node sees itself and its md nearest ancestors."""
    cu = np.array([0, n], dtype=np.int32)
    t = clib.ancestor_table_heap(cu, b, md)
    depth = 0
    while num_tree_nodes(b, depth) < n:
        depth += 1
    par = tree.build_tree(b, depth)[:n]
    for i in range(n):
        chain = [i]
        while par[chain[-1]] != -1 and len(chain) < md + 1:
            chain.append(par[chain[-1]])
        got = [a for a in t[i] if a >= 0]
        assert got == chain


def test_parents_table_equals_heap_table_for_complete_trees():
    for b, d in [(2, 4), (3, 3), (1, 6)]:
        n = num_tree_nodes(b, d)
        par = np.array(tree.build_tree(b, d))
        par[0] = 0  # root self-loop convention (scripts/benchmark_micro.py:283-285)
        cu = np.array([0, n, 2 * n], dtype=np.int32)
        assert (clib.ancestor_table_parents(cu, np.concatenate([par, par]), d)
                == clib.ancestor_table_heap(cu, b, d)).all()


def test_parents_table_out_of_range_stops():
    cu = np.array([0, 3], dtype=np.int32)
    t = clib.ancestor_table_parents(cu, np.array([0, 7, -1], dtype=np.int32), 3)
    assert t.tolist() == [[0, -1, -1, -1], [1, -1, -1, -1], [2, -1, -1, -1]]


def _mutant_table_no_clamp(n, b, md):
    """Planted mistake: divide before clamping, in the unsigned 32-bit
    arithmetic a multiply-high divider uses (src/ragged_attn.py:333-337)."""
    out = np.full((n, md + 1), -1)
    for q in range(n):
        cur, prev = q, -1
        for s in range(md + 1):
            out[q, s] = cur if cur != prev else -1
            prev, cur = cur, ((cur - 1) & 0xFFFFFFFF) // b
    return out


def _mutant_table_wrong_parent(n, b, md):
    """Planted mistake: parent(k) = k // b."""
    out = np.full((n, md + 1), -1)
    for q in range(n):
        cur, prev = q, -1
        for s in range(md + 1):
            out[q, s] = cur if cur != prev else -1
            prev, cur = cur, cur // b
    return out


def test_planted_walk_mistakes_are_caught():
    b, d = 2, 3
    n = num_tree_nodes(b, d)
    m = tree.tree_attention_mask(b, d)
    for mut in (_mutant_table_no_clamp, _mutant_table_wrong_parent):
        t = mut(n, b, d)
        bad = np.zeros((n, n), dtype=bool)
        for i in range(n):
            for a in t[i]:
                if 0 <= a < n:
                    bad[i, a] = True
        clean = all(0 <= a < n for a in t.flatten() if a != -1)
        assert (not clean) or not (bad == m).all(), mut.__name__


# ---------------------------------------------------------------------------
# attention outputs
# ---------------------------------------------------------------------------

def _masks_for(cu, b, md):
    t = clib.ancestor_table_heap(cu.numpy(), b, md)
    cu_l = cu.tolist()
    return [tree.mask_from_table(t, cu_l[i], cu_l[i + 1] - cu_l[i]) for i in range(len(cu_l) - 1)]


@pytest.mark.parametrize("B,b,d,H,D", [(2, 2, 3, 4, 64), (1, 3, 3, 2, 32), (3, 4, 2, 2, 128),
                                        (2, 1, 6, 4, 64), (4, 2, 5, 2, 64)])
def test_sparse_walk_matches_padded_sdpa(B, b, d, H, D):
    n = num_tree_nodes(b, d)
    Q, K, V, cu = make_inputs([n] * B, H, D, B * 10000 + b * 100 + d, torch.float32)
    o, lse, _ = oracle_tree(Q, K, V, cu, b, d)
    O, L = sdpa.packed_tree_attention(Q, K, V, cu, _masks_for(cu, b, d), return_lse=True)
    assert np.abs(o - O.numpy()).max() < 2e-5
    assert np.abs(lse - L.numpy()).max() < 2e-5


def test_ragged_and_truncated_match_padded_sdpa():
    lens = [13, 0, 40, 1, 7]
    Q, K, V, cu = make_inputs(lens, 3, 64, 4242, torch.float32)
    for b, md in [(3, 3), (2, 1), (1, 4)]:
        o, lse, _ = oracle_tree(Q, K, V, cu, b, md)
        O, L = sdpa.packed_tree_attention(Q, K, V, cu, _masks_for(cu, b, md), return_lse=True)
        assert np.abs(o - O.numpy()).max() < 2e-5
        assert np.abs(lse - L.numpy()).max() < 2e-5


def test_shifted_cu_equals_rebased_cu():
    """cu_seqlens that start past row 0 (and leave rows after cu[B]): the
    tokens in [cu[0], cu[B]) get the attention of the same sequences rebased
    to row 0, and the rows outside every sequence are never read or written."""
    lens = [15, 10, 0, 15]
    Q, K, V, cu = make_inputs([5] + lens + [7], 4, 64, 515, torch.float32)
    cu = cu[1:-1].clone()  # sequences start at row 5; rows 45..51 belong to none
    o, lse, _ = oracle_tree(Q, K, V, cu, 2, 3)
    lo, hi = int(cu[0]), int(cu[-1])
    o0, lse0, _ = oracle_tree(Q[lo:hi], K[lo:hi], V[lo:hi], cu - cu[0], 2, 3)
    assert np.array_equal(o[lo:hi], o0) and np.array_equal(lse[lo:hi], lse0)


def test_chain_is_causal_attention():
    """b=1 with max_depth >= n-1 is plain causal attention (tests/test_correctness.py:339-350)."""
    n, H, D = 9, 4, 64
    Q, K, V, cu = make_inputs([n, n], H, D, 40108, torch.float32)
    o, _, _ = oracle_tree(Q, K, V, cu, 1, n - 1)
    for s in range(2):
        q = Q[s * n:(s + 1) * n].permute(1, 0, 2)
        k = K[s * n:(s + 1) * n].permute(1, 0, 2)
        v = V[s * n:(s + 1) * n].permute(1, 0, 2)
        with torch.nn.attention.sdpa_kernel(torch.nn.attention.SDPBackend.MATH):
            ref = F.scaled_dot_product_attention(q, k, v, is_causal=True).permute(1, 0, 2)
        assert np.abs(o[s * n:(s + 1) * n] - ref.numpy()).max() < 2e-5


def test_single_token_is_v():
    """d=0: every query attends only itself, softmax of one score = 1 (:325-336)."""
    Q, K, V, cu = make_inputs([1, 1, 1], 4, 64, 40100, torch.float32)
    o, lse, _ = oracle_tree(Q, K, V, cu, 1, 0)
    assert np.array_equal(o, V.double().numpy())
    s = (Q.double() * K.double()).sum(-1) / 8.0
    assert np.abs(lse - s.numpy()).max() < 1e-12


def _brute(Q, K, V, cu, b, md):
    """Pure-Python loops straight from the definition."""
    T, H, D = Q.shape
    out = np.zeros((T, H, D))
    cu = [int(x) for x in cu]
    for s in range(len(cu) - 1):
        for x in range(cu[s + 1] - cu[s]):
            chain, cur = [], x
            for _ in range(md + 1):
                if cur not in chain:
                    chain.append(cur)
                cur = max(cur - 1, 0) // b
            for h in range(H):
                sc = [sum(float(Q[cu[s] + x, h, e]) * float(K[cu[s] + a, h, e]) for e in range(D)) / math.sqrt(D)
                      for a in chain]
                mx = max(sc)
                w = [math.exp(v - mx) for v in sc]
                for e in range(D):
                    out[cu[s] + x, h, e] = sum(wi * float(V[cu[s] + a, h, e]) for wi, a in zip(w, chain)) / sum(w)
    return out


def test_brute_force_tiny():
    Q, K, V, cu = make_inputs([7, 4], 2, 8, 11, torch.float32)
    o, _, _ = oracle_tree(Q, K, V, cu, 2, 2)
    assert np.abs(o - _brute(Q, K, V, cu, 2, 2)).max() < 1e-12


def test_planted_attention_mistakes_are_caught():
    """A dropped scale, a transposed head/key index or a log2 LSE must fail."""
    Q, K, V, cu = make_inputs([15, 15], 4, 64, 20203, torch.float32)
    o, lse, anc = oracle_tree(Q, K, V, cu, 2, 3)
    O, L = sdpa.packed_tree_attention(Q, K, V, cu, _masks_for(cu, 2, 3), return_lse=True)
    # dropped scale
    o_bad, _ = clib.tree_attn(Q.numpy(), K.numpy(), V.numpy(), cu.numpy(), anc, 1.0)
    assert np.abs(o_bad - O.numpy()).max() > 1e-2
    # transposed operand: keys of the wrong head
    o_bad, _ = clib.tree_attn(Q.numpy(), K.flip(1).numpy(), V.numpy(), cu.numpy(), anc, 1 / 8)
    assert np.abs(o_bad - O.numpy()).max() > 1e-2
    # log2 instead of ln in the LSE
    assert np.abs(lse / math.log(2) - L.numpy()).max() > 1e-2
    assert np.abs(lse - L.numpy()).max() < 2e-5


def test_gqa_equals_repeated_kv():
    Q, K, V, cu = make_inputs([31, 31], 8, 64, 9191, torch.float32, Hkv=2)
    o, lse, _ = oracle_tree(Q, K, V, cu, 2, 4)
    Kr, Vr = torch.repeat_interleave(K, 4, dim=1), torch.repeat_interleave(V, 4, dim=1)
    o2, lse2, _ = oracle_tree(Q, Kr, Vr, cu, 2, 4)
    assert np.abs(o - o2).max() < 1e-12 and np.abs(lse - lse2).max() < 1e-12
    O = sdpa.packed_tree_attention(Q, K, V, cu, _masks_for(cu, 2, 4))
    assert np.abs(o - O.numpy()).max() < 2e-5


def test_prefix_matches_sdpa_with_unmasked_prefix():
    """All-attended prefix rows (tests/test_correctness.py:444-469)."""
    n, L, B = num_tree_nodes(2, 3), 24, 2
    g = torch.Generator().manual_seed(6161)
    Q, K, V, cu = make_inputs([n] * B, 4, 64, 6161, torch.float32, Hkv=2)
    Kp = torch.randn(B, L, 2, 64, generator=g)
    Vp = torch.randn(B, L, 2, 64, generator=g)
    o, lse, _ = oracle_tree(Q, K, V, cu, 2, 3, Kp=Kp, Vp=Vp)
    O, Ls = sdpa.packed_tree_attention(Q, K, V, cu, _masks_for(cu, 2, 3), Kp=Kp, Vp=Vp, return_lse=True)
    assert np.abs(o - O.numpy()).max() < 2e-5
    assert np.abs(lse - Ls.numpy()).max() < 2e-5
    # L = 0 prefix reduces to the tree-only oracle
    o0, _, _ = oracle_tree(Q, K, V, cu, 2, 3, Kp=Kp[:, :0], Vp=Vp[:, :0])
    o1, _, _ = oracle_tree(Q, K, V, cu, 2, 3)
    assert np.array_equal(o0, o1)


def test_lse_merge_is_softmax_over_union():
    """FA2 identity: merging the prefix-only and tree-only states reproduces
    attention over both key sets (src/ragged_attn.py:1599-1616)."""
    n, L, B = num_tree_nodes(2, 3), 24, 2
    g = torch.Generator().manual_seed(6161)
    Q, K, V, cu = make_inputs([n] * B, 4, 64, 6161, torch.float32)
    Kp = torch.randn(B, L, 4, 64, generator=g)
    Vp = torch.randn(B, L, 4, 64, generator=g)
    o_all, lse_all, _ = oracle_tree(Q, K, V, cu, 2, 3, Kp=Kp, Vp=Vp)
    o_t, lse_t, _ = oracle_tree(Q, K, V, cu, 2, 3)
    # prefix-only: a tree table with no attended tree key
    anc_none = np.full((int(cu[-1]), 1), -1, dtype=np.int32)
    o_p, lse_p = clib.tree_attn(Q.numpy(), K.numpy(), V.numpy(), cu.numpy(), anc_none, 1 / 8,
                                Kp.numpy(), Vp.numpy())
    merged = clib.lse_merge(lse_p.astype(np.float32), lse_t.astype(np.float32),
                            o_p.astype(np.float32), o_t.astype(np.float32))
    assert np.abs(merged - o_all).max() < 1e-5
    # planted mistake: unnormalised (no division by w_p + w_t) merge fails
    wp = np.exp(lse_p - np.maximum(lse_p, lse_t))[..., None]
    wt = np.exp(lse_t - np.maximum(lse_p, lse_t))[..., None]
    assert np.abs((wp * o_p + wt * o_t) - o_all).max() > 1e-2


# ---------------------------------------------------------------------------
# committed fixtures reproduce from the oracle
# ---------------------------------------------------------------------------

FIXTURES = sorted(glob.glob(os.path.join(GOLDEN_DIR, "*.npz")))


def test_fixtures_present():
    assert len(FIXTURES) >= 10


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p)[:-4] for p in FIXTURES])
def test_fixture_reproduces(path):
    z = np.load(path)
    cu = torch.from_numpy(z["cu"])
    q, k, v = (torch.from_numpy(z[n].astype(np.float32)) for n in ("q", "k", "v"))
    kp = torch.from_numpy(z["kp"].astype(np.float32)) if "kp" in z else None
    vp = torch.from_numpy(z["vp"].astype(np.float32)) if "vp" in z else None
    parents = z["parents"] if "parents" in z else None
    o, lse, anc = oracle_tree(q, k, v, cu, int(z["b"]), int(z["max_depth"]), parents, kp, vp)
    assert np.array_equal(anc, z["anc"])
    assert np.abs(o - z["o"]).max() < 1e-6
    assert np.abs(lse - z["lse"]).max() < 1e-5
    if parents is None and kp is None:
        O, L = sdpa.packed_tree_attention(q, k, v, cu, _masks_for(cu, int(z["b"]), int(z["max_depth"])),
                                          return_lse=True)
        assert np.abs(O.numpy() - z["o"]).max() < 2e-5
