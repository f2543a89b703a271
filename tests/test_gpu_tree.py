"""GPU parity of the tree kernels against the pinned CPU oracle.

Every test generates inputs on the CPU (explicit torch.Generator), runs the
HIP path through libqattn.so's C ABI and compares with the fp64 oracle
evaluated on the same (already rounded) inputs.

Tolerances (written per test):
  fp16 outputs   max |o - o_ref| <= 2e-3 (fp16 rounding
                 of |o| < 8 is at most 2^-9 = 1.95e-3) and the reference's own
                 torch.allclose(atol=rtol=1e-2) (tests/test_correctness.py:219).
  bf16 outputs   max |o - o_ref| <= 2^-8 * max(1, |o_ref|) + 1e-4 (half an ulp)
  LSE (fp32)     max abs <= 1e-4
  ancestor sets  bit-exact
"""
from __future__ import annotations

import itertools
import glob
import math
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN_DIR, make_inputs, num_tree_nodes, oracle_tree, tree_case
from oracle import clib

pytestmark = pytest.mark.gpu

DEV = "cuda"
FP16_TOL = 2e-3


def _ra():
    from qattention_amd import _lib, ragged_attn
    return ragged_attn, _lib


def run_tree(Q, K, V, cu, b, md, algo=0, lse=True, max_seqlen=None):
    ra, _ = _ra()
    O, L = ra._tree_forward(Q.to(DEV), K.to(DEV), V.to(DEV), cu, b, md, max_seqlen, lse, algo)
    torch.cuda.synchronize()
    return O.float().cpu().double().numpy(), (L.cpu().double().numpy() if L is not None else None)


def check_fp16(o, o_ref, what=""):
    err = np.abs(o - o_ref).max() if o.size else 0.0
    assert err <= FP16_TOL, f"{what}: max abs err {err:.3e} > {FP16_TOL}"
    assert np.allclose(o, o_ref, atol=1e-2, rtol=1e-2), what


def check_bf16(o, o_ref, what=""):
    bound = 2.0 ** -8 * np.maximum(1.0, np.abs(o_ref)) + 1e-4
    assert (np.abs(o - o_ref) <= bound).all(), f"{what}: bf16 err {np.abs(o - o_ref).max():.3e}"


def say(*a):
    print(*a, flush=True)


# ---------------------------------------------------------------------------
# ancestor index sets: bit-exact
# ---------------------------------------------------------------------------

ANC_CASES = [([15, 15], 2, 3), ([1365] * 2, 4, 5), ([1023], 2, 9), ([9, 9, 9], 1, 8), ([13, 0, 40, 1, 7], 3, 3),
             ([31, 31], 2, 2), ([4681], 8, 4), ([100], 7, 1), ([50], 3, 0)]


@pytest.mark.parametrize("lens,b,md", ANC_CASES)
def test_ancestors_heap_bitexact(lens, b, md):
    ra, _ = _ra()
    say("ancestors heap", lens[:3], b, md)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    got = ra.ancestor_table(cu, b, md).cpu().numpy()
    ref = clib.ancestor_table_heap(cu.numpy(), b, md)
    assert np.array_equal(got, ref)


def test_ancestors_parents_bitexact():
    ra, _ = _ra()
    rng = np.random.default_rng(7)
    lens = [20, 33, 1, 64]
    par = []
    for n in lens:
        p = np.zeros(n, dtype=np.int32)
        for i in range(1, n):
            p[i] = rng.integers(0, i)
        par.append(p)
    par = np.concatenate(par)
    par[5] = 99  # out of range: the walk stops there
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    for md in (0, 3, 10):
        say("ancestors parents md", md)
        got = ra.ancestor_table(cu, 1, md, parents=torch.from_numpy(par)).cpu().numpy()
        ref = clib.ancestor_table_parents(cu.numpy(), par, md)
        assert np.array_equal(got, ref)


# ---------------------------------------------------------------------------
# the reference's parity matrix (tests/test_correctness.py:254-350)
# ---------------------------------------------------------------------------

REF_MATRIX = list(itertools.product([1, 2, 4, 8], [1, 2, 3], [1, 2, 3, 4, 5, 6]))


@pytest.mark.parametrize("B,b,d", REF_MATRIX)
def test_reference_matrix(B, b, d):
    say("matrix", B, b, d)
    Q, K, V, cu = tree_case(B, b, d, 4, 64)
    o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, b, d)
    og, lg = run_tree(Q, K, V, cu, b, d, algo=1)
    check_fp16(og, o_ref, "gather")
    assert np.abs(lg - lse_ref).max() <= 1e-4
    os_, ls = run_tree(Q, K, V, cu, b, d, algo=2)
    check_fp16(os_, o_ref, "subtree")
    assert np.abs(ls - lse_ref).max() <= 1e-4


BENCH_CONFIGS = [(4, 2, 5), (4, 3, 5), (8, 2, 5), (8, 3, 5), (4, 2, 6), (4, 3, 6)]


@pytest.mark.parametrize("B,b,d", BENCH_CONFIGS)
def test_benchmark_configs(B, b, d):
    say("bench config", B, b, d)
    Q, K, V, cu = tree_case(B, b, d, 8, 128)
    o_ref, _, _ = oracle_tree(Q, K, V, cu, b, d)
    for algo in (0, 1, 2):
        o, _ = run_tree(Q, K, V, cu, b, d, algo=algo, lse=False)
        check_fp16(o, o_ref, f"algo {algo}")


@pytest.mark.parametrize("D", [32, 64, 128])
def test_head_dims(D):
    say("head dim", D)
    Q, K, V, cu = tree_case(4, 2, 3, 4, D)
    o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, 2, 3)
    for algo in (1, 2):
        o, l = run_tree(Q, K, V, cu, 2, 3, algo=algo)
        check_fp16(o, o_ref, f"D={D} algo {algo}")
        assert np.abs(l - lse_ref).max() <= 1e-4


@pytest.mark.parametrize("b,d", [(1, 0), (1, 8)])
def test_single_token_and_chain(b, d):
    say("edge", b, d)
    Q, K, V, cu = tree_case(4, b, d, 4, 64)
    o_ref, _, _ = oracle_tree(Q, K, V, cu, b, d)
    for algo in (1, 2):
        o, _ = run_tree(Q, K, V, cu, b, d, algo=algo)
        check_fp16(o, o_ref, f"b={b} d={d} algo {algo}")
    if d == 0:
        o, _ = run_tree(Q, K, V, cu, b, d)
        assert np.array_equal(o, V.double().numpy())


def test_gather_and_subtree_agree():
    """The two kernels differ only in fp32 summation order, so their fp16
    outputs agree to one ulp and their LSEs to fp32 rounding."""
    for (B, b, d, H, D) in [(4, 4, 5, 8, 128), (2, 2, 7, 4, 64), (3, 3, 4, 4, 32), (2, 1, 40, 2, 64)]:
        say("gather~subtree", B, b, d)
        Q, K, V, cu = tree_case(B, b, d, H, D)
        o1, l1 = run_tree(Q, K, V, cu, b, d, algo=1)
        o2, l2 = run_tree(Q, K, V, cu, b, d, algo=2)
        # two fp16 roundings of fp32 values that differ by summation-order
        # noise (~1e-6 absolute): <= 2 ulp, with an absolute floor for
        # results near zero where that noise exceeds an fp16 ulp
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(o1), 2.0 ** -14))) - 10)
        bad = np.abs(o1 - o2) > 2 * ulp + 1e-5
        assert not bad.any(), f"{bad.sum()} elements differ by more than 2 ulp"
        assert np.abs(l1 - l2).max() <= 1e-5


# ---------------------------------------------------------------------------
# golden fixtures
# ---------------------------------------------------------------------------

FIXTURES = [p for p in sorted(glob.glob(os.path.join(GOLDEN_DIR, "*.npz")))
            if os.path.basename(p) not in ("cfg1.npz", "parents.npz", "prefix.npz")]


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p)[:-4] for p in FIXTURES])
def test_golden_fixture(path):
    say("fixture", os.path.basename(path))
    z = np.load(path)
    Q, K, V = (torch.from_numpy(z[n]) for n in ("q", "k", "v"))
    cu = torch.from_numpy(z["cu"])
    for algo in (0, 1, 2):
        o, l = run_tree(Q, K, V, cu, int(z["b"]), int(z["max_depth"]), algo=algo)
        check_fp16(o, z["o"].astype(np.float64), f"{os.path.basename(path)} algo {algo}")
        assert np.abs(l - z["lse"]).max() <= 1e-4


def test_golden_cfg1_fp16():
    """cfg1 fixture (the reference's CPU-runnable configuration, fp32 inputs)
    through the fp16 kernel: the kernel output matches the oracle evaluated on
    the fp16-rounded inputs."""
    z = np.load(os.path.join(GOLDEN_DIR, "cfg1.npz"))
    Q, K, V = (torch.from_numpy(z[n]).half() for n in ("q", "k", "v"))
    cu = torch.from_numpy(z["cu"])
    o_ref, _, _ = oracle_tree(Q, K, V, cu, 2, 3)
    o, _ = run_tree(Q, K, V, cu, 2, 3)
    check_fp16(o, o_ref, "cfg1")
    # and within fp16 input-rounding distance of the fp32-input fixture
    assert np.abs(o - z["o"]).max() < 2e-2


def test_golden_parents_fixture():
    ra, _ = _ra()
    z = np.load(os.path.join(GOLDEN_DIR, "parents.npz"))
    Q, K, V = (torch.from_numpy(z[n]).to(DEV) for n in ("q", "k", "v"))
    cu = torch.from_numpy(z["cu"])
    O, L = ra.ragged_attention_with_parents(Q, K, V, cu, torch.from_numpy(z["parents"]), int(z["max_depth"]))
    check_fp16(O.double().cpu().numpy(), z["o"].astype(np.float64), "parents fixture")
    assert np.abs(L.double().cpu().numpy() - z["lse"]).max() <= 1e-4


# ---------------------------------------------------------------------------
# layouts, dtypes, GQA, ragged batches
# ---------------------------------------------------------------------------

def test_bf16():
    for (B, b, d, H, D) in [(4, 2, 5, 8, 128), (2, 3, 3, 4, 64), (2, 4, 2, 4, 32)]:
        say("bf16", B, b, d, D)
        Q, K, V, cu = tree_case(B, b, d, H, D, dtype=torch.bfloat16)
        o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, b, d)
        for algo in (1, 2):
            o, l = run_tree(Q, K, V, cu, b, d, algo=algo)
            check_bf16(o, o_ref, f"bf16 algo {algo}")
            assert np.abs(l - lse_ref).max() <= 1e-4


def test_strided_views_e2e_layout():
    """[N, H, D] views of [H, N, D] storage (token stride D, head stride N*D),
    as the EAGLE-3 verify path passes them (scripts/e2e_benchmark.py:1455-1458)."""
    ra, _ = _ra()
    b, d, H, D = 3, 3, 4, 64
    N = num_tree_nodes(b, d)
    g = torch.Generator().manual_seed(5)
    base = [torch.randn(H, N, D, generator=g).half() for _ in range(3)]
    Qv, Kv, Vv = (t.to(DEV).transpose(0, 1) for t in base)
    assert Qv.stride() == (D, N * D, 1)
    cu = torch.tensor([0, N], dtype=torch.int32)
    o_ref, _, _ = oracle_tree(Qv.cpu(), Kv.cpu(), Vv.cpu(), cu, b, d)
    O = ra.ragged_attention(Qv, Kv, Vv, cu, b, d)
    assert O.stride() == Qv.stride()  # empty_like keeps the caller's layout
    check_fp16(O.double().cpu().numpy(), o_ref, "strided")


def test_non_vector_layout_is_copied():
    ra, _ = _ra()
    Q, K, V, cu = tree_case(2, 2, 3, 4, 64)
    Qw = torch.zeros(Q.shape[0], 4, 128, dtype=torch.float16)
    Qw[:, :, ::2] = Q
    Qs = Qw.to(DEV)[:, :, ::2]  # last-dim stride 2
    o_ref, _, _ = oracle_tree(Q, K, V, cu, 2, 3)
    O = ra.ragged_attention(Qs, K.to(DEV), V.to(DEV), cu, 2, 3)
    check_fp16(O.double().cpu().numpy(), o_ref, "copied layout")


def test_gqa():
    for (Hq, Hkv, D) in [(32, 8, 128), (8, 2, 64), (4, 1, 32), (6, 3, 64)]:
        say("gqa", Hq, Hkv, D)
        Q, K, V, cu = tree_case(2, 4, 3, Hq, D, Hkv=Hkv)
        o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, 4, 3)
        for algo in (1, 2):
            o, l = run_tree(Q, K, V, cu, 4, 3, algo=algo)
            check_fp16(o, o_ref, f"gqa algo {algo}")
            assert np.abs(l - lse_ref).max() <= 1e-4


@pytest.mark.parametrize("lens,b,md", [([13, 0, 40, 1, 7], 3, 3), ([31, 31], 2, 2), ([100, 37], 2, 9),
                                       ([341, 5, 200], 4, 2), ([64, 64], 1, 5), ([2000], 2, 12),
                                       ([700], 28, 2)])
def test_ragged_and_truncated(lens, b, md):
    say("ragged", lens, b, md)
    Q, K, V, cu = make_inputs(lens, 4, 64, 31337)
    o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, b, md)
    for algo in (0, 1, 2):
        o, l = run_tree(Q, K, V, cu, b, md, algo=algo)
        check_fp16(o, o_ref, f"algo {algo}")
        assert np.abs(l - lse_ref).max() <= 1e-4


@pytest.mark.parametrize("cu_list,max_seqlen,b,d,H", [
    ([5, 20, 30], 15, 2, 3, 4),
    ([0, 15, 25, 40], 15, 2, 3, 4),
    ([65, 1430, 2730, 4095, 5460], 1365, 4, 5, 8),
])
def test_shifted_cu_seqlens(cu_list, max_seqlen, b, d, H):
    """cu_seqlens that do not start at 0 or leave a sequence short of
    max_seqlen, with batch * max_seqlen rows (the subtree kernel reads each
    workgroup's first sequence bounds apart from its LDS copy of
    cu_seqlens); the last case is large enough for the counter schedule.
    Rows outside [cu[0], cu[B]) belong to no sequence and are not compared."""
    say("shifted cu", cu_list, max_seqlen, b, d, H)
    B = len(cu_list) - 1
    T = B * max_seqlen
    gen = torch.Generator().manual_seed(4242 + T)
    Q, K, V = [torch.randn(T, H, 128, generator=gen).half() for _ in range(3)]
    cu = torch.tensor(cu_list, dtype=torch.int32)
    o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, b, d)
    o, l = run_tree(Q, K, V, cu, b, d, algo=2, max_seqlen=max_seqlen)
    rows = slice(cu_list[0], cu_list[-1])
    check_fp16(o[rows], o_ref[rows], "shifted cu")
    assert np.abs(l[rows] - lse_ref[rows]).max() <= 1e-4


def test_max_seqlen_given_and_device_cu():
    """Graph-friendly call: device cu_seqlens + explicit max_seqlen (no host sync)."""
    Q, K, V, cu = make_inputs([13, 40, 7], 4, 64, 99)
    o_ref, _, _ = oracle_tree(Q, K, V, cu, 3, 3)
    o, _ = run_tree(Q, K, V, cu.to(DEV), 3, 3, max_seqlen=40)
    check_fp16(o, o_ref, "device cu")


def test_empty_inputs():
    ra, _ = _ra()
    Q = torch.zeros(0, 4, 64, dtype=torch.float16, device=DEV)
    cu = torch.zeros(1, dtype=torch.int32)
    O = ra.ragged_attention(Q, Q, Q, cu, 2, 3)
    assert O.shape == (0, 4, 64)
    O, L = ra.ragged_attention_with_lse(Q, Q, Q, torch.tensor([0, 0], dtype=torch.int32), 2, 3)
    assert O.shape == (0, 4, 64) and L.shape == (0, 4)


def test_sibling_aliases_match_base():
    ra, _ = _ra()
    Q, K, V, cu = tree_case(4, 4, 4, 4, 64)
    Qd, Kd, Vd = Q.to(DEV), K.to(DEV), V.to(DEV)
    O = ra.ragged_attention(Qd, Kd, Vd, cu, 4, 4)
    assert torch.equal(O, ra.ragged_attention_sibling(Qd, Kd, Vd, cu, 4, 4))
    O2, L2 = ra.ragged_attention_sibling_with_lse(Qd, Kd, Vd, cu, 4, 4)
    O3, L3 = ra.ragged_attention_with_lse(Qd, Kd, Vd, cu, 4, 4)
    assert torch.equal(O2, O) and torch.equal(O3, O) and torch.equal(L2, L3)


# ---------------------------------------------------------------------------
# explicit parents and paged K/V
# ---------------------------------------------------------------------------

def _random_parents(lens, seed, window=None):
    rng = np.random.default_rng(seed)
    out = []
    for n in lens:
        p = np.zeros(n, dtype=np.int32)
        for i in range(1, n):
            lo = 0 if window is None else max(0, i - window)
            p[i] = rng.integers(lo, i)
        out.append(p)
    return np.concatenate(out)


@pytest.mark.parametrize("lens,md,window", [([20, 33, 1], 7, 6), ([200, 300], 12, None), ([64], 3, 2),
                                            ([512, 512], 20, 4)])
def test_parents(lens, md, window):
    ra, _ = _ra()
    say("parents", lens, md)
    Q, K, V, cu = make_inputs(lens, 8, 128, 4711, Hkv=4)
    par = _random_parents(lens, 4711, window)
    o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, 1, md, parents=par)
    O, L = ra.ragged_attention_with_parents(Q.to(DEV), K.to(DEV), V.to(DEV), cu, torch.from_numpy(par), md)
    check_fp16(O.double().cpu().numpy(), o_ref, "parents")
    assert np.abs(L.double().cpu().numpy() - lse_ref).max() <= 1e-4


def test_parents_equals_heap_for_complete_trees():
    ra, _ = _ra()
    from qattention_amd.tree_mask import build_tree, kernel_parents
    b, d = 3, 4
    Q, K, V, cu = tree_case(2, b, d, 4, 64)
    par = np.tile(kernel_parents(build_tree(b, d)), 2)
    O1, L1 = ra.ragged_attention_with_parents(Q.to(DEV), K.to(DEV), V.to(DEV), cu, torch.from_numpy(par), d)
    O2, L2 = ra.ragged_attention_with_lse(Q.to(DEV), K.to(DEV), V.to(DEV), cu, b, d)
    assert torch.equal(O1, O2) and torch.equal(L1, L2)


@pytest.mark.parametrize("page_size", [16, 5])
def test_paged(page_size):
    ra, _ = _ra()
    say("paged", page_size)
    lens = [85, 21, 40]
    Q, K, V, cu = make_inputs(lens, 4, 64, 2024, Hkv=2)
    cuL = cu.tolist()
    ks = [K[cuL[i]:cuL[i + 1]].to(DEV) for i in range(3)]
    vs = [V[cuL[i]:cuL[i + 1]].to(DEV) for i in range(3)]
    Kc, Vc, pt = ra.build_paged_kv(ks, vs, page_size=page_size)
    # shuffle the physical pages to make the indirection matter
    perm = torch.randperm(Kc.shape[0], generator=torch.Generator().manual_seed(1))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    Kc, Vc = Kc[perm.to(DEV)].contiguous(), Vc[perm.to(DEV)].contiguous()
    pt = inv[pt.long()].to(torch.int32)
    o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, 4, 3)
    O = ra.ragged_attention_paged(Q.to(DEV), Kc, Vc, pt, cu, 4, 3)
    check_fp16(O.double().cpu().numpy(), o_ref, "paged")
    # both kernels, with the LSE
    for algo in (_lib_algo("gather"), _lib_algo("subtree")):
        O, L = ra._paged_forward(Q.to(DEV), Kc, Vc, pt, cu, 4, 3, None, True, algo)
        check_fp16(O.double().cpu().numpy(), o_ref, f"paged algo {algo}")
        assert np.abs(L.double().cpu().numpy() - lse_ref).max() <= 1e-4, f"paged LSE algo {algo}"


def _lib_algo(name):
    _, lib = _ra()
    return {"auto": lib.ALGO_AUTO, "gather": lib.ALGO_GATHER, "subtree": lib.ALGO_SUBTREE}[name]


def _shuffled_paged(ra, K, V, cu, H, page_size, seed):
    """build_paged_kv over the packed K/V, physical pages in a shuffled order."""
    cuL = cu.tolist()
    B = len(cuL) - 1
    ks = [K[cuL[i]:cuL[i + 1]].to(DEV) for i in range(B)]
    vs = [V[cuL[i]:cuL[i + 1]].to(DEV) for i in range(B)]
    Kc, Vc, pt = ra.build_paged_kv(ks, vs, page_size=page_size)
    perm = torch.randperm(Kc.shape[0], generator=torch.Generator().manual_seed(seed))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    return Kc[perm.to(DEV)].contiguous(), Vc[perm.to(DEV)].contiguous(), inv[pt.long()].to(torch.int32)


# (lens, b, max_depth, Hq, Hkv, D, page_size): the subtree kernel on paged K/V
# -- cfg2's trees, pages of 1, 5 (not a power of two), 16 and 4096 (one page
# per sequence), bf16-sized heads, GQA, ragged and empty sequences
PAGED_SUBTREE_CASES = [
    ([1365] * 2, 4, 5, 8, 8, 128, 16),
    ([1365, 300], 4, 5, 4, 4, 128, 5),
    ([121, 0, 40, 1], 3, 4, 8, 2, 128, 1),
    ([1023], 2, 9, 4, 4, 64, 16),
    ([700, 33], 4, 2, 6, 3, 32, 4096),
]


@pytest.mark.parametrize("lens,b,md,Hq,Hkv,D,ps", PAGED_SUBTREE_CASES)
def test_paged_subtree(lens, b, md, Hq, Hkv, D, ps):
    """The paged subtree kernel against the oracle and the paged gather kernel
    (same cache, same page table): O within the fp16 bound, LSE 1e-4."""
    ra, _ = _ra()
    say("paged subtree", lens[:4], b, md, Hq, Hkv, D, ps)
    Q, K, V, cu = make_inputs(lens, Hq, D, 2100 + ps, Hkv=Hkv)
    Kc, Vc, pt = _shuffled_paged(ra, K, V, cu, Hkv, ps, 7)
    o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, b, md)
    Qd = Q.to(DEV)
    for algo in (_lib_algo("subtree"), _lib_algo("gather")):
        O, L = ra._paged_forward(Qd, Kc, Vc, pt, cu, b, md, None, True, algo)
        torch.cuda.synchronize()
        check_fp16(O.double().cpu().numpy(), o_ref, f"paged algo {algo}")
        assert np.abs(L.double().cpu().numpy() - lse_ref).max() <= 1e-4, f"paged LSE algo {algo}"


def test_paged_subtree_bf16():
    ra, _ = _ra()
    say("paged subtree bf16")
    lens, b, md = [1365, 85], 4, 5
    Q, K, V, cu = make_inputs(lens, 8, 128, 2150, dtype=torch.bfloat16, Hkv=4)
    Kc, Vc, pt = _shuffled_paged(ra, K, V, cu, 4, 16, 9)
    o_ref, _, _ = oracle_tree(Q, K, V, cu, b, md)
    O, _ = ra._paged_forward(Q.to(DEV), Kc, Vc, pt, cu, b, md, None, False, _lib_algo("subtree"))
    check_bf16(O.float().double().cpu().numpy(), o_ref, "paged subtree bf16")


def test_paged_subtree_table_limit():
    """A page table of more than 2048 entries: the automatic choice runs the
    gather kernel (same results), the forced subtree kernel is an error."""
    ra, lib = _ra()
    say("paged table limit")
    lens, b, md = [121] * 3, 3, 4
    Q, K, V, cu = make_inputs(lens, 4, 64, 2160)
    Kc, Vc, pt = _shuffled_paged(ra, K, V, cu, 4, 16, 3)
    wide = torch.full((3, 700), -1, dtype=torch.int32)  # 2100 entries
    wide[:, :pt.shape[1]] = pt
    o_ref, _, _ = oracle_tree(Q, K, V, cu, b, md)
    O, _ = ra._paged_forward(Q.to(DEV), Kc, Vc, wide, cu, b, md, None, False, lib.ALGO_AUTO)
    check_fp16(O.double().cpu().numpy(), o_ref, "paged, wide table")
    with pytest.raises(lib.QAttnError, match="page-table entries"):
        ra._paged_forward(Q.to(DEV), Kc, Vc, wide, cu, b, md, None, False, lib.ALGO_SUBTREE)


def test_paged_subtree_needs_equal_strides():
    """The paged subtree kernel addresses K and V with one offset: a V cache
    with other strides (here every page padded by one slot) runs on the
    gather kernel under the automatic choice, and is an error when the
    subtree kernel is forced."""
    ra, lib = _ra()
    say("paged strides")
    lens, b, md = [121] * 3, 3, 4
    Q, K, V, cu = make_inputs(lens, 4, 64, 2170)
    Kc, Vc, pt = _shuffled_paged(ra, K, V, cu, 4, 16, 5)
    big = torch.zeros(Vc.shape[0], 17, *Vc.shape[2:], dtype=Vc.dtype, device=DEV)
    big[:, :16] = Vc
    Vs = big[:, :16]  # same values, page stride 17 slots
    assert Vs.stride() != Kc.stride()
    o_ref, _, _ = oracle_tree(Q, K, V, cu, b, md)
    O, _ = ra._paged_forward(Q.to(DEV), Kc, Vs, pt, cu, b, md, None, False, lib.ALGO_AUTO)
    check_fp16(O.double().cpu().numpy(), o_ref, "paged, V strides differ")
    with pytest.raises(lib.QAttnError, match="strides"):
        ra._paged_forward(Q.to(DEV), Kc, Vs, pt, cu, b, md, None, False, lib.ALGO_SUBTREE)


def test_paged_missing_pages():
    """Page-table entries that are negative or past num_pages skip the
    ancestors on those pages (qattn.h); a query whose own page and every
    ancestor's page are missing attends nothing and gets O = 0.  The oracle
    is the heap walk's ancestor table with those entries removed."""
    ra, _ = _ra()
    ps, b, d = 4, 3, 3
    lens = [40, 17]
    Q, K, V, cu = make_inputs(lens, 4, 64, 2031, Hkv=2)
    cuL = cu.tolist()
    ks = [K[cuL[i]:cuL[i + 1]].to(DEV) for i in range(2)]
    vs = [V[cuL[i]:cuL[i + 1]].to(DEV) for i in range(2)]
    Kc, Vc, pt = ra.build_paged_kv(ks, vs, page_size=ps)
    pt = pt.clone()
    pt[0, 0] = -1                 # sequence 0's root page: tokens 0..3 and every root step
    pt[0, 5] = Kc.shape[0] + 5    # past num_pages
    pt[1, 2] = -7
    anc = clib.ancestor_table_heap(cu.numpy().astype(np.int32), b, d)
    for t in range(anc.shape[0]):
        seq = 0 if t < cuL[1] else 1
        for s1 in range(anc.shape[1]):
            a = anc[t, s1]
            if a >= 0:
                page = int(pt[seq, a // ps])
                if page < 0 or page >= Kc.shape[0]:
                    anc[t, s1] = -1
    assert (anc[:cuL[1]] < 0).all(axis=1).any()  # some query attends nothing
    o_ref, lse_ref = clib.tree_attn(Q.float().numpy(), K.float().numpy(), V.float().numpy(), cu.numpy(), anc,
                                    1.0 / 8.0)
    O = ra.ragged_attention_paged(Q.to(DEV), Kc, Vc, pt, cu, b, d)
    check_fp16(O.double().cpu().numpy(), o_ref, "paged, missing pages")
    empty = np.isneginf(lse_ref)
    assert empty.any()
    for algo in (_lib_algo("gather"), _lib_algo("subtree")):
        O, L = ra._paged_forward(Q.to(DEV), Kc, Vc, pt, cu, b, d, None, True, algo)
        check_fp16(O.double().cpu().numpy(), o_ref, f"paged, missing pages, algo {algo}")
        L = L.double().cpu().numpy()
        assert (np.isneginf(L) == empty).all(), f"algo {algo}: LSE -inf exactly where nothing is attended"
        assert np.abs(L[~empty] - lse_ref[~empty]).max() <= 1e-4, f"algo {algo}: LSE"


@pytest.mark.parametrize("algo", ["gather", "subtree"])
def test_paged_graph_capture_replay(algo):
    """With max_seqlen (and device cu / page table) the paged call makes no
    host read and records into a HIP graph; replays after new cache contents
    are copied in match eager calls on the same contents."""
    ra, _ = _ra()
    code = _lib_algo(algo)
    b, d, N, B, ps = 3, 4, 121, 3, 16
    Q, K, V, cu = make_inputs([N] * B, 8, 128, 2040, Hkv=4)
    Kc, Vc, pt = ra.build_paged_kv(list(K.to(DEV).view(B, N, 4, 128)), list(V.to(DEV).view(B, N, 4, 128)), ps)
    Qd, cud, ptd = Q.to(DEV), cu.to(DEV), pt.to(DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ra._paged_forward(Qd, Kc, Vc, ptd, cud, b, d, N, False, code)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out, _ = ra._paged_forward(Qd, Kc, Vc, ptd, cud, b, d, N, False, code)
    g = torch.Generator().manual_seed(2041)
    for i in range(3):
        Kc.copy_(torch.randn(Kc.shape, generator=g).half())
        Vc.copy_(torch.randn(Vc.shape, generator=g).half())
        Qd.copy_(torch.randn(Qd.shape, generator=g).half())
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager, _ = ra._paged_forward(Qd, Kc, Vc, ptd, cud, b, d, N, False, code)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"


# ---------------------------------------------------------------------------
# LSE merge
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_lse_merge(dtype):
    ra, _ = _ra()
    say("merge", dtype)
    B, H, Nq, D = 3, 4, 37, 128
    g = torch.Generator().manual_seed(8)
    lp = torch.randn(B, H, Nq, generator=g) * 3
    lt = torch.randn(B, H, Nq, generator=g) * 3
    op = torch.randn(B, H, Nq, D, generator=g).to(dtype)
    ot = torch.randn(B, H, Nq, D, generator=g).to(dtype)
    ref = clib.lse_merge(lp.numpy(), lt.numpy(), op.float().numpy(), ot.float().numpy())
    # a permuted (non-contiguous) out_tree view, as the reference's callers pass
    ot_view = ot.to(DEV).permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    got = ra.fused_lse_merge(lp.to(DEV), lt.to(DEV), op.to(DEV), ot_view).double().cpu().numpy()
    if dtype == torch.float16:
        check_fp16(got, ref, "merge")
    else:
        check_bf16(got, ref, "merge")


# ---------------------------------------------------------------------------
# full-size tree-only configurations of the reference benchmark (cfg2, cfg3)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("B,b,d", [(4, 4, 5), (8, 2, 9)])
def test_baseline_full_size(B, b, d):
    say("full size", B, b, d)
    Q, K, V, cu = tree_case(B, b, d, 32, 128)
    o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, b, d)
    for algo in (0, 1, 2):
        o, l = run_tree(Q, K, V, cu, b, d, algo=algo)
        check_fp16(o, o_ref, f"full algo {algo}")
        assert np.abs(l - lse_ref).max() <= 1e-4


def test_subtree_schedule_repeats():
    """The subtree kernel hands out tiles from counters that each launch
    leaves at zero when it completes, taken from a ring of 32 per device:
    140 launches at a size that uses them (mixed with small launches that do
    not) reuse every slot, and every result is bit-identical to the first."""
    ra, _ = _ra()
    B, b, d = 4, 4, 5
    Q, K, V, cu = tree_case(B, b, d, 32, 128)
    o_ref, _, _ = oracle_tree(Q, K, V, cu, b, d)
    Qd, Kd, Vd, cud = Q.to(DEV), K.to(DEV), V.to(DEV), cu.to(DEV)
    N = num_tree_nodes(b, d)
    first, _ = ra._tree_forward(Qd, Kd, Vd, cud, b, d, N, False, 2)
    check_fp16(first.float().cpu().double().numpy(), o_ref, "first launch")
    q2, k2, v2, cu2 = tree_case(2, 2, 3, 4, 64)
    small_ref, _ = ra._tree_forward(q2.to(DEV), k2.to(DEV), v2.to(DEV), cu2.to(DEV), 2, 3, None, False, 2)
    for i in range(140):
        if i % 9 == 4:
            small, _ = ra._tree_forward(q2.to(DEV), k2.to(DEV), v2.to(DEV), cu2.to(DEV), 2, 3, None, False, 2)
            assert torch.equal(small, small_ref), f"small launch {i}"
        o, _ = ra._tree_forward(Qd, Kd, Vd, cud, b, d, N, False, 2)
        if i % 10 == 9 or i > 125:
            assert torch.equal(o, first), f"launch {i}"
    torch.cuda.synchronize()


def test_subtree_concurrent_streams():
    """Eager subtree launches in flight on four streams at once take
    different counter slots of the per-device ring: every stream's results
    are bit-identical to its inputs run alone (a slot shared by two running
    launches would hand tiles of one to the other's workgroups)."""
    ra, _ = _ra()
    B, b, d, H = 4, 4, 5, 32
    N = num_tree_nodes(b, d)
    say("concurrent streams", B, b, d, H)
    cu = torch.arange(0, (B + 1) * N, N, dtype=torch.int32, device=DEV)
    sets, refs = [], []
    for sidx in range(4):
        Q, K, V, _ = make_inputs([N] * B, H, 128, 900 + sidx)
        sets.append((Q.to(DEV), K.to(DEV), V.to(DEV)))
        refs.append(ra._tree_forward(*sets[-1], cu, b, d, N, False, 2)[0].clone())
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(4)]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    outs = [[] for _ in range(4)]
    for it in range(6):
        for sidx, st in enumerate(streams):
            with torch.cuda.stream(st):
                outs[sidx].append(ra._tree_forward(*sets[sidx], cu, b, d, N, False, 2)[0])
    torch.cuda.synchronize()
    for sidx in range(4):
        for it, o in enumerate(outs[sidx]):
            assert torch.equal(o, refs[sidx]), f"stream {sidx} launch {it}"


@pytest.mark.parametrize("B,b,d,H", [(4, 4, 4, 8), (4, 4, 5, 32)])
def test_graph_capture_replay(B, b, d, H):
    """The entry point records into a HIP graph (device cu + max_seqlen) and
    every replay matches the eager result, with eager work in between (the
    full-size case records the subtree kernel with its counter slot, which
    every replay reuses)."""
    say("graph", B, b, d, H)
    ra, _ = _ra()
    Q, K, V, cu = tree_case(B, b, d, H, 128)
    Qd, Kd, Vd, cud = Q.to(DEV), K.to(DEV), V.to(DEV), cu.to(DEV)
    N = num_tree_nodes(b, d)
    eager = ra.ragged_attention(Qd, Kd, Vd, cud, b, d, max_seqlen=N)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ra.ragged_attention(Qd, Kd, Vd, cud, b, d, max_seqlen=N)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ra.ragged_attention(Qd, Kd, Vd, cud, b, d, max_seqlen=N)
    for i in range(4):
        out.zero_()
        junk = torch.randn(1000, device=DEV).sum()  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        del junk
