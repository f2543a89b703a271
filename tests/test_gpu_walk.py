"""Bit-exact ancestor index sets from the kernels that compute the outputs.

Each case runs an attention call with the walk export on (qattn_debug_walk):
the serving kernel writes, for every (token, q head) it computes, the
ancestor set that query attended as the kernel used it -- the subtree
kernel's row mask decoded through the row map its loads were issued with,
the gather walk's loaded node per step, the fused prefix epilogue's staged
LDS rows -- and the table must equal the oracle's walk
(oracle/qattn_oracle.c, src/ragged_attn.py:323-377 / :650-698) for every
head, bit for bit.  The outputs of the same call are checked against the
fp64 oracle (fp16 max abs <= 2e-3), so the exported walk is the one that
produced them.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import make_inputs, num_tree_nodes, oracle_tree
from oracle import clib

pytestmark = pytest.mark.gpu

DEV = "cuda"


def say(*a):
    print(*a, flush=True)


def _mods():
    from qattention_amd import _lib, ragged_attn
    return ragged_attn, _lib


def _table(T, Hq, md):
    return torch.full((T, Hq, md + 1), -3, dtype=torch.int32, device=DEV)


def _expect(got, ref_tab, what):
    """got [T, Hq, S1] from the kernel, ref_tab [T, S1] from the oracle."""
    g = got.cpu().numpy()
    ref = np.broadcast_to(ref_tab[:, None, :], g.shape)
    bad = np.argwhere(g != ref)
    assert bad.size == 0, (f"{what}: {len(bad)} entries differ, first (t, h, step) = {tuple(bad[0])}: "
                           f"kernel {g[tuple(bad[0][:2])]} oracle {ref_tab[bad[0][0]]}")


def _check_out(O, o_ref, what):
    err = float(np.abs(O.double().cpu().numpy() - o_ref).max()) if O.numel() else 0.0
    assert err <= 2e-3, f"{what}: max abs err {err:.3e}"


def _tree_call(Q, K, V, cu, b, md, algo, table, max_seqlen=None):
    ra, _lib = _mods()
    with _lib.debug_walk(table):
        O, _ = ra._tree_forward(Q.to(DEV), K.to(DEV), V.to(DEV), cu, b, md, max_seqlen, False, algo)
    torch.cuda.synchronize()
    return O


# (lens, b, max_depth, Hq, Hkv, D): cfg2 / cfg3 at full size, a
# many-band plan (b=4 d=7, N=21845), truncated walks, b=1 chains, ragged and
# empty sequences, GQA, every head dim
HEAP_CASES = [
    ([1365] * 4, 4, 5, 32, 32, 128),      # cfg2
    ([1023] * 8, 2, 9, 32, 32, 128),      # cfg3
    ([21845], 4, 7, 4, 4, 128),           # b=4 d=7: many bands
    ([1365, 700], 4, 2, 8, 8, 128),       # truncated (max_depth < depth), ragged
    ([9, 40, 1, 0, 17], 1, 8, 4, 4, 64),  # b=1 chains, an empty and a one-token sequence
    ([200], 1, 3, 4, 2, 32),              # long chain, truncated
    ([13, 0, 40, 1, 7], 3, 3, 8, 2, 128), # ragged + empty + GQA
    ([4681], 8, 4, 4, 4, 64),             # cfg5's tree
    ([3000, 511], 2, 11, 4, 1, 128),      # deep binary, ragged, GQA 4
    ([100], 7, 0, 4, 4, 32),              # max_depth 0: self only
    # enough tiles that the subtree kernel runs its last round as half tiles
    # (halves of root ranges, of one root's children, of chain levels)
    ([2000] * 8, 1, 8, 16, 16, 128),      # b=1 chains
    ([1365, 700] * 4, 4, 2, 32, 32, 128), # ragged + truncated
    ([4681] * 4, 8, 4, 32, 8, 64),        # cfg5's tree, GQA 4
    ([1093, 50, 0, 1093], 3, 6, 32, 16, 32),  # b=3, ragged + empty, GQA 2
]


@pytest.mark.parametrize("lens,b,md,Hq,Hkv,D", HEAP_CASES)
@pytest.mark.parametrize("algo", ["subtree", "gather"])
def test_heap_walk_bitexact(lens, b, md, Hq, Hkv, D, algo):
    ra, _lib = _mods()
    say("walk heap", algo, lens[:4], b, md, Hq, Hkv, D)
    code = _lib.ALGO_SUBTREE if algo == "subtree" else _lib.ALGO_GATHER
    Q, K, V, cu = make_inputs(lens, Hq, D, 4000 + b * 10 + md, Hkv=Hkv)
    T = Q.shape[0]
    table = _table(T, Hq, md)
    O = _tree_call(Q, K, V, cu, b, md, code, table)
    ref = clib.ancestor_table_heap(cu.numpy(), b, md)
    _expect(table, ref, f"{algo} walk")
    if T * Hq <= 400_000:  # the fp64 oracle's outputs on the smaller cases
        o_ref, _, _ = oracle_tree(Q, K, V, cu, b, md)
        _check_out(O, o_ref, f"{algo} outputs")


def _random_parents(lens, seed, window=None):
    rng = np.random.default_rng(seed)
    out = []
    for n in lens:
        p = np.zeros(n, dtype=np.int32)
        for i in range(1, n):
            lo = 0 if window is None else max(0, i - window)
            p[i] = rng.integers(lo, i)
        out.append(p)
    return np.concatenate(out) if out else np.zeros(0, dtype=np.int32)


@pytest.mark.parametrize("lens,md,window", [([60], 7, 10), ([20, 0, 33, 1], 5, 3), ([1024], 7, None),
                                            ([300, 200], 12, 2)])
def test_parents_walk_bitexact(lens, md, window):
    """The explicit-parent gather walk (src/ragged_attn.py:650-698)."""
    ra, _lib = _mods()
    say("walk parents", lens, md, window)
    Hq, D = 8, 128
    Q, K, V, cu = make_inputs(lens, Hq, D, 4100 + md)
    par = _random_parents(lens, 4101 + md, window)
    T = Q.shape[0]
    table = _table(T, Hq, md)
    L = _lib.lib()
    Qd, Kd, Vd, O = Q.to(DEV), K.to(DEV), V.to(DEV), torch.empty(T, Hq, D, dtype=torch.float16, device=DEV)
    pd, cud = torch.from_numpy(par).to(DEV), cu.to(DEV)
    st = _lib.i64arr(Qd.stride())
    with _lib.debug_walk(table):
        rc = L.qattn_tree_parents_fwd(Qd.data_ptr(), st, Kd.data_ptr(), st, Vd.data_ptr(), st, O.data_ptr(), st,
                                      None, None, cud.data_ptr(), pd.data_ptr(), len(lens), max(lens), T, Hq, Hq,
                                      D, md, 1.0 / math.sqrt(D), _lib.DTYPE_F16,
                                      torch.cuda.current_stream().cuda_stream)
        _lib.check(rc, "qattn_tree_parents_fwd")
    torch.cuda.synchronize()
    _expect(table, clib.ancestor_table_parents(cu.numpy(), par, md), "parents walk")
    o_ref, _, _ = oracle_tree(Q, K, V, cu, 2, md, parents=par)
    _check_out(O, o_ref, "parents outputs")


@pytest.mark.parametrize("algo", ["subtree", "gather"])
def test_paged_walk_bitexact(algo):
    """The paged walk of both kernels: 16-token pages in a shuffled physical
    order, one logical page missing from the table (its ancestors are
    skipped); the outputs of the same call match the oracle on that table."""
    ra, _lib = _mods()
    lens, b, md, H, D = [1365, 341], 4, 5, 8, 128
    say("walk paged", algo)
    code = _lib.ALGO_SUBTREE if algo == "subtree" else _lib.ALGO_GATHER
    Q, K, V, cu = make_inputs(lens, H, D, 4200)
    Kc, Vc, pt = ra.build_paged_kv([K[:1365], K[1365:]], [V[:1365], V[1365:]], 16)
    g = torch.Generator().manual_seed(4201)
    perm = torch.randperm(Kc.shape[0], generator=g)
    Kp, Vp = torch.empty_like(Kc), torch.empty_like(Vc)
    Kp[perm], Vp[perm] = Kc, Vc
    ptp = perm.to(torch.int32)[pt.long()]
    ptp[1, 3] = -1  # sequence 1, nodes 48..63: not in the cache
    T = Q.shape[0]
    table = _table(T, H, md)
    with _lib.debug_walk(table):
        O, _ = ra._paged_forward(Q.to(DEV), Kp.to(DEV), Vp.to(DEV), ptp, cu, b, md, None, False, code)
    torch.cuda.synchronize()
    ref = clib.ancestor_table_heap(cu.numpy(), b, md)
    seq1 = ref[1365:]
    seq1[(seq1 >= 48) & (seq1 < 64)] = -1  # missing page: those ancestors are not attended
    _expect(table, ref, f"{algo} paged walk")
    o_ref, _ = clib.tree_attn(Q.float().numpy(), K.float().numpy(), V.float().numpy(), cu.numpy(), ref,
                              1.0 / math.sqrt(D), want_lse=False)
    _check_out(O, o_ref, f"{algo} paged outputs")


def _prefix(B, L, Hkv, D, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(B, L, Hkv, D, generator=g).half(), torch.randn(B, L, Hkv, D, generator=g).half())


# (lens, b, md, Hq, Hkv, L, num_splits): one split runs the walk in the
# prefix kernel's epilogue (LDS-staged for wide trees, gathered for deep
# binary ones); several splits hand it to the tree kernels with the split
# states (gather, or the subtree kernel when its tiles are plentiful)
PREFIX_CASES = [
    ([4681] * 16, 8, 4, 32, 32, 2048, 0),   # cfg5 (one split: staged epilogue walk)
    ([85] * 4, 4, 3, 32, 8, 10240, 0),      # cfg4 (five splits: gather with split states)
    ([85] * 4, 4, 3, 32, 8, 10240, 1),      # cfg4 forced into one split
    ([1023, 500], 2, 9, 4, 4, 300, 1),      # deep binary: staged and gathered tiles
    ([1365] * 4, 4, 5, 32, 32, 256, 4),     # several splits, subtree kernel with split states
    ([40, 0, 13, 1], 3, 2, 6, 3, 200, 1),   # ragged + empty, GQA
]


@pytest.mark.parametrize("lens,b,md,Hq,Hkv,L,ns", PREFIX_CASES)
def test_prefix_walk_bitexact(lens, b, md, Hq, Hkv, L, ns):
    ra, _lib = _mods()
    say("walk prefix", lens[:3], b, md, Hq, Hkv, L, ns)
    D = 128
    Q, K, V, cu = make_inputs(lens, Hq, D, 4300 + b * 10 + md, Hkv=Hkv)
    Kp, Vp = _prefix(len(lens), L, Hkv, D, 4301 + L)
    T = Q.shape[0]
    table = _table(T, Hq, md)
    with _lib.debug_walk(table):
        O = ra.ragged_attention_prefix(Q.to(DEV), K.to(DEV), V.to(DEV), cu, Kp.to(DEV), Vp.to(DEV), b, md,
                                       num_splits=ns)
    torch.cuda.synchronize()
    _expect(table, clib.ancestor_table_heap(cu.numpy(), b, md), "prefix walk")
    if T * Hq * L <= 50_000_000:
        o_ref, _, _ = oracle_tree(Q, K, V, cu, b, md, Kp=Kp, Vp=Vp)
        _check_out(O, o_ref, "prefix outputs")


@pytest.mark.parametrize("ns", [0, 1])
def test_prefix_parents_walk_bitexact(ns):
    ra, _lib = _mods()
    lens, md, Hq, Hkv, D, L = [60, 33, 1], 7, 32, 8, 128, 2048
    say("walk prefix parents", ns)
    Q, K, V, cu = make_inputs(lens, Hq, D, 4400 + ns, Hkv=Hkv)
    par = _random_parents(lens, 4401, 6)
    Kp, Vp = _prefix(len(lens), L, Hkv, D, 4402)
    T = Q.shape[0]
    table = _table(T, Hq, md)
    with _lib.debug_walk(table):
        O = ra.ragged_attention_prefix(Q.to(DEV), K.to(DEV), V.to(DEV), cu, Kp.to(DEV), Vp.to(DEV), 2, md,
                                       num_splits=ns, parents=torch.from_numpy(par))
    torch.cuda.synchronize()
    _expect(table, clib.ancestor_table_parents(cu.numpy(), par, md), "prefix parents walk")
    o_ref, _, _ = oracle_tree(Q, K, V, cu, 2, md, parents=par, Kp=Kp, Vp=Vp)
    _check_out(O, o_ref, "prefix parents outputs")


# (dtype, with LSE): the instantiations that serve bf16 calls and the
# LSE-returning calls (ragged_attention_with_lse, return_lse=True prefix calls)
VARIANTS = [(torch.bfloat16, False), (torch.float16, True), (torch.bfloat16, True)]


def _check_out_dt(O, o_ref, dtype, what):
    """fp16: max abs <= 2e-3; bf16: half an ulp of max(1, |o|) (2^-8) plus the
    prefix path's P rounding, 2^-7 max(1, |o|) + 1e-3."""
    o = O.double().cpu().numpy()
    if dtype == torch.float16:
        _check_out(O, o_ref, what)
    else:
        bound = 2.0 ** -7 * np.maximum(1.0, np.abs(o_ref)) + 1e-3
        assert (np.abs(o - o_ref) <= bound).all(), f"{what}: bf16 err {np.abs(o - o_ref).max():.3e}"


def _check_lse(LSE, lse_ref, dtype, what):
    err = float(np.abs(LSE.double().cpu().numpy() - lse_ref).max()) if LSE.numel() else 0.0
    assert err <= (1e-4 if dtype == torch.float16 else 2e-3), f"{what}: LSE err {err:.3e}"


@pytest.mark.parametrize("dtype,lse", VARIANTS)
@pytest.mark.parametrize("lens,b,md,Hq,Hkv,D", [([1365] * 4, 4, 5, 32, 32, 128),   # cfg2
                                               ([4681] * 2, 8, 4, 32, 32, 128),   # cfg5's tree
                                               ([13, 0, 40, 1, 7], 3, 3, 8, 2, 64)])
@pytest.mark.parametrize("algo", ["subtree", "gather"])
def test_heap_walk_bitexact_bf16_lse(lens, b, md, Hq, Hkv, D, algo, dtype, lse):
    ra, _lib = _mods()
    say("walk heap", algo, dtype, "lse" if lse else "", lens[:3], b, md, Hq, Hkv, D)
    code = _lib.ALGO_SUBTREE if algo == "subtree" else _lib.ALGO_GATHER
    Q, K, V, cu = make_inputs(lens, Hq, D, 4600 + b * 10 + md, dtype=dtype, Hkv=Hkv)
    T = Q.shape[0]
    table = _table(T, Hq, md)
    with _lib.debug_walk(table):
        O, LSE = ra._tree_forward(Q.to(DEV), K.to(DEV), V.to(DEV), cu, b, md, None, lse, code)
    torch.cuda.synchronize()
    _expect(table, clib.ancestor_table_heap(cu.numpy(), b, md), f"{algo} {dtype} walk")
    if T * Hq <= 400_000:
        o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, b, md)
        _check_out_dt(O, o_ref, dtype, f"{algo} outputs")
        if lse:
            _check_lse(LSE, lse_ref, dtype, algo)


@pytest.mark.parametrize("dtype,lse", VARIANTS)
@pytest.mark.parametrize("algo", ["subtree", "gather"])
def test_paged_walk_bitexact_bf16_lse(algo, dtype, lse):
    ra, _lib = _mods()
    lens, b, md, H, D = [1365, 341], 4, 5, 8, 128
    say("walk paged", algo, dtype, lse)
    code = _lib.ALGO_SUBTREE if algo == "subtree" else _lib.ALGO_GATHER
    Q, K, V, cu = make_inputs(lens, H, D, 4700, dtype=dtype)
    Kc, Vc, pt = ra.build_paged_kv([K[:1365], K[1365:]], [V[:1365], V[1365:]], 16)
    perm = torch.randperm(Kc.shape[0], generator=torch.Generator().manual_seed(4701))
    Kp, Vp = torch.empty_like(Kc), torch.empty_like(Vc)
    Kp[perm], Vp[perm] = Kc, Vc
    ptp = perm.to(torch.int32)[pt.long()]
    T = Q.shape[0]
    table = _table(T, H, md)
    with _lib.debug_walk(table):
        O, LSE = ra._paged_forward(Q.to(DEV), Kp.to(DEV), Vp.to(DEV), ptp, cu, b, md, None, lse, code)
    torch.cuda.synchronize()
    _expect(table, clib.ancestor_table_heap(cu.numpy(), b, md), f"{algo} paged walk")
    o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, b, md)
    _check_out_dt(O, o_ref, dtype, f"{algo} paged outputs")
    if lse:
        _check_lse(LSE, lse_ref, dtype, f"{algo} paged")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_parents_walk_bitexact_bf16_lse(dtype):
    """ragged_attention_with_parents returns LSE: the LSE instantiations of
    the parents walk, in both dtypes."""
    ra, _lib = _mods()
    lens, md, Hq, D = [60, 0, 1024], 7, 8, 128
    say("walk parents", dtype)
    Q, K, V, cu = make_inputs(lens, Hq, D, 4800, dtype=dtype)
    par = _random_parents(lens, 4801, 10)
    T = Q.shape[0]
    table = _table(T, Hq, md)
    with _lib.debug_walk(table):
        O, LSE = ra.ragged_attention_with_parents(Q.to(DEV), K.to(DEV), V.to(DEV), cu, torch.from_numpy(par), md)
    torch.cuda.synchronize()
    _expect(table, clib.ancestor_table_parents(cu.numpy(), par, md), "parents walk")
    o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, 2, md, parents=par)
    _check_out_dt(O, o_ref, dtype, "parents outputs")
    _check_lse(LSE, lse_ref, dtype, "parents")


# prefix calls: cfg5 (one split, the fused epilogue's staged walk), cfg4
# (five splits merged by the gather walk, and forced into one split), and
# several splits merged by the subtree kernel
PREFIX_VARIANT_CASES = [
    ([4681] * 16, 8, 4, 32, 32, 2048, 0),
    ([85] * 4, 4, 3, 32, 8, 10240, 0),
    ([85] * 4, 4, 3, 32, 8, 10240, 1),
    ([1365] * 4, 4, 5, 32, 32, 256, 4),
]


@pytest.mark.parametrize("dtype,lse", VARIANTS)
@pytest.mark.parametrize("lens,b,md,Hq,Hkv,L,ns", PREFIX_VARIANT_CASES)
def test_prefix_walk_bitexact_bf16_lse(lens, b, md, Hq, Hkv, L, ns, dtype, lse):
    ra, _lib = _mods()
    say("walk prefix", dtype, lse, lens[:3], b, md, Hq, Hkv, L, ns)
    D = 128
    Q, K, V, cu = make_inputs(lens, Hq, D, 4900 + b * 10 + md, dtype=dtype, Hkv=Hkv)
    g = torch.Generator().manual_seed(4901 + L)
    Kp = torch.randn(len(lens), L, Hkv, D, generator=g).to(dtype)
    Vp = torch.randn(len(lens), L, Hkv, D, generator=g).to(dtype)
    T = Q.shape[0]
    table = _table(T, Hq, md)
    with _lib.debug_walk(table):
        out = ra.ragged_attention_prefix(Q.to(DEV), K.to(DEV), V.to(DEV), cu, Kp.to(DEV), Vp.to(DEV), b, md,
                                         num_splits=ns, return_lse=lse)
    torch.cuda.synchronize()
    O, LSE = out if lse else (out, None)
    _expect(table, clib.ancestor_table_heap(cu.numpy(), b, md), f"prefix walk {dtype}")
    if T * Hq * L <= 50_000_000:
        o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, b, md, Kp=Kp, Vp=Vp)
        _check_out_dt(O, o_ref, dtype, "prefix outputs")
        if lse:
            _check_lse(LSE, lse_ref, dtype, "prefix")


def test_walk_export_rejects_unsupported_calls():
    """The export covers calls over packed cu_seqlens (either dtype, with or
    without LSE); the uniform-batch [B, H, N, D] call fails loudly while it
    is on, and the export is off again afterwards."""
    ra, _lib = _mods()
    B, N, H, D = 2, 15, 4, 64
    Q, K, V, cu = make_inputs([N] * B, H, D, 4500)
    q4 = Q.view(B, N, H, D).permute(0, 2, 1, 3).to(DEV)
    k4 = K.view(B, N, H, D).permute(0, 2, 1, 3).to(DEV)
    v4 = V.view(B, N, H, D).permute(0, 2, 1, 3).to(DEV)
    table = _table(B * N, H, 3)
    with _lib.debug_walk(table):
        with pytest.raises(_lib.QAttnError):
            ra.ragged_tree_attn(q4, k4, v4, 2, 3)
    O4 = ra.ragged_tree_attn(q4, k4, v4, 2, 3)  # export off: works
    assert torch.isfinite(O4.float()).all()
