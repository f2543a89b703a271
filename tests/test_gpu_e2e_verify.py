"""GPU tests of ragged_tree_attn: tree verification over the model's own
[B, H, N, D] tensors (the replacement for _ragged_tree_attn,
scripts/e2e_benchmark.py:1394-1502).

Each case checks the result against the fp64 oracle on the packed form of
the same inputs, and against the packed-layout entry point
(ragged_attention_prefix), which runs the same kernels over the same rows and
must therefore agree bit for bit: a wrong per-sequence offset anywhere in the
[B, H, N, D] addressing changes rows and fails that equality."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import num_tree_nodes, oracle_tree

pytestmark = pytest.mark.gpu

DEV = "cuda"


def say(*a):
    print(*a, flush=True)


def _ra():
    from qattention_amd import ragged_attn
    return ragged_attn


def _inputs(B, Hq, Hkv, N, L, D, seed, dtype=torch.float16, token_major=False, cache_len=None):
    """Q [B, Hq, N, D], K/V [B, Hkv, L + N, D] drawn on the CPU.  token_major
    lays them out as [B, N, H, D] transposed views (the layout SDPA returns);
    cache_len > L + N makes K/V slices of a longer cache."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, N, D, generator=g).to(dtype)
    k = torch.randn(B, Hkv, L + N, D, generator=g).to(dtype)
    v = torch.randn(B, Hkv, L + N, D, generator=g).to(dtype)
    Qd, Kd, Vd = q.to(DEV), k.to(DEV), v.to(DEV)
    if token_major:
        Qd = Qd.transpose(1, 2).contiguous().transpose(1, 2)
        Kd = Kd.transpose(1, 2).contiguous().transpose(1, 2)
        Vd = Vd.transpose(1, 2).contiguous().transpose(1, 2)
    if cache_len is not None:
        Kc = torch.zeros(B, Hkv, cache_len, D, dtype=dtype, device=DEV)
        Vc = torch.zeros(B, Hkv, cache_len, D, dtype=dtype, device=DEV)
        Kc[:, :, :L + N] = Kd
        Vc[:, :, :L + N] = Vd
        Kd, Vd = Kc[:, :, :L + N], Vc[:, :, :L + N]
    return (q, k, v), (Qd, Kd, Vd)


def _packed(q, k, v, L):
    """The packed form: Q/K/V tree rows [B*N, H, D], prefix [B, L, Hkv, D]."""
    B, Hq, N, D = q.shape
    Hkv = k.shape[1]
    Qp = q.permute(0, 2, 1, 3).reshape(B * N, Hq, D)
    Kt = k[:, :, L:].permute(0, 2, 1, 3).reshape(B * N, Hkv, D)
    Vt = v[:, :, L:].permute(0, 2, 1, 3).reshape(B * N, Hkv, D)
    Kp = k[:, :, :L].permute(0, 2, 1, 3).contiguous()
    Vp = v[:, :, :L].permute(0, 2, 1, 3).contiguous()
    cu = torch.arange(0, (B + 1) * N, N, dtype=torch.int32)
    return Qp, Kt, Vt, Kp, Vp, cu


def _check(O, LSE, q, k, v, L, b, md, parents_packed=None, dtype=torch.float16):
    B, Hq, N, D = q.shape
    Qp, Kt, Vt, Kp, Vp, cu = _packed(q, k, v, L)
    o_ref, lse_ref, _ = oracle_tree(Qp, Kt, Vt, cu, b, md, parents=parents_packed,
                                    Kp=Kp if L else None, Vp=Vp if L else None)
    o = O.permute(0, 2, 1, 3).reshape(B * N, Hq, D).double().cpu().numpy()
    if dtype == torch.float16:
        err = float(np.abs(o - o_ref).max())
        assert err <= 2e-3, f"max abs err {err:.3e}"
    else:
        bound = 2.0 ** -7 * np.maximum(1.0, np.abs(o_ref)) + 1e-3
        assert (np.abs(o - o_ref) <= bound).all()
    if LSE is not None:
        lse = LSE.permute(0, 2, 1).reshape(B * N, Hq).double().cpu().numpy()
        assert np.abs(lse - lse_ref).max() <= 1e-4


def _packed_call(ra, q, k, v, L, b, md, parents_packed, ns):
    B, Hq, N, D = q.shape
    Qp, Kt, Vt, Kp, Vp, cu = _packed(q, k, v, L)
    par = None if parents_packed is None else torch.from_numpy(parents_packed)
    O, LSE = ra.ragged_attention_prefix(Qp.to(DEV), Kt.to(DEV), Vt.to(DEV), cu, Kp.to(DEV), Vp.to(DEV), b, md,
                                        max_seqlen=N, return_lse=True, num_splits=ns, parents=par)
    return O.view(B, N, Hq, D).permute(0, 2, 1, 3), LSE.view(B, N, Hq).permute(0, 2, 1)


@pytest.mark.parametrize("B,b,d,Hq,Hkv,L,ns,token_major", [
    (3, 3, 3, 8, 2, 300, 0, False),    # split prefix + gather merge/walk
    (3, 3, 3, 8, 2, 300, 1, True),     # fused single-split epilogue, token-major views
    (2, 4, 4, 4, 4, 0, 0, False),      # no prefix: the subtree kernel
    (2, 4, 4, 4, 4, 0, 0, True),
    (1, 2, 5, 8, 8, 130, 0, False),    # one sequence
    (4, 4, 3, 32, 8, 1000, 0, False),  # the E2E shape (Llama-3-8B heads)
])
def test_verify_heap(B, b, d, Hq, Hkv, L, ns, token_major):
    ra = _ra()
    D, N = 128, num_tree_nodes(b, d)
    say("verify heap", B, b, d, Hq, Hkv, L, ns, token_major)
    (q, k, v), (Qd, Kd, Vd) = _inputs(B, Hq, Hkv, N, L, D, 7000 + B * 10 + d, token_major=token_major)
    O, LSE = ra.ragged_tree_attn(Qd, Kd, Vd, b, d, return_lse=True, num_splits=ns)
    assert O.shape == (B, Hq, N, D) and LSE.shape == (B, Hq, N)
    _check(O, LSE, q, k, v, L, b, d)
    if L:
        Op, LSEp = _packed_call(ra, q, k, v, L, b, d, None, ns)
        assert torch.equal(O, Op) and torch.equal(LSE, LSEp)


def test_verify_max_depth_truncated_and_cache_slice():
    """max_depth below the tree depth, K/V read from slices of a longer cache."""
    ra = _ra()
    B, b, d, Hq, Hkv, L, D = 2, 2, 6, 8, 4, 260, 64
    N = num_tree_nodes(b, d)
    say("verify truncated", B, b, d, L)
    (q, k, v), (Qd, Kd, Vd) = _inputs(B, Hq, Hkv, N, L, D, 7100, cache_len=L + N + 37)
    O, LSE = ra.ragged_tree_attn(Qd, Kd, Vd, b, 3, return_lse=True)
    _check(O, LSE, q, k, v, L, b, 3)


def _tree_parents(N, seed):
    rng = np.random.default_rng(seed)
    p = np.zeros(N, dtype=np.int32)
    for i in range(1, N):
        p[i] = rng.integers(0, i)
    return p


@pytest.mark.parametrize("shared,L,ns", [(True, 400, 0), (True, 0, 0), (False, 400, 1), (False, 64, 0)])
def test_verify_parents(shared, L, ns):
    """tree_parents [N] shared by every sequence (the reference's case), or
    [B, N] one tree per sequence."""
    ra = _ra()
    B, N, Hq, Hkv, D, md = 3, 61, 8, 2, 128, 9
    say("verify parents", shared, L, ns)
    (q, k, v), (Qd, Kd, Vd) = _inputs(B, Hq, Hkv, N, L, D, 7200 + L + ns)
    if shared:
        p1 = _tree_parents(N, 7201)
        par_dev = torch.from_numpy(p1).to(DEV)
        packed = np.tile(p1, B)
    else:
        pb = np.stack([_tree_parents(N, 7202 + s) for s in range(B)])
        par_dev = torch.from_numpy(pb).to(DEV)
        packed = pb.reshape(-1)
    O, LSE = ra.ragged_tree_attn(Qd, Kd, Vd, 2, md, tree_parents=par_dev, return_lse=True, num_splits=ns)
    _check(O, LSE, q, k, v, L, 2, md, parents_packed=packed)
    if L:
        Op, LSEp = _packed_call(ra, q, k, v, L, 2, md, packed, ns)
        assert torch.equal(O, Op) and torch.equal(LSE, LSEp)


def test_verify_parents_wrong_length_falls_back_to_heap():
    """A tree_parents whose length is not N_q is ignored, as in the reference
    (scripts/e2e_benchmark.py:1470, :1475)."""
    ra = _ra()
    B, b, d, H, L, D = 2, 3, 2, 4, 50, 64
    N = num_tree_nodes(b, d)
    (_, _, _), (Qd, Kd, Vd) = _inputs(B, H, H, N, L, D, 7300)
    heap = ra.ragged_tree_attn(Qd, Kd, Vd, b, d)
    other = ra.ragged_tree_attn(Qd, Kd, Vd, b, d, tree_parents=torch.zeros(N + 1, dtype=torch.int32, device=DEV))
    assert torch.equal(heap, other)


def test_verify_bf16():
    ra = _ra()
    B, b, d, Hq, Hkv, L, D = 2, 4, 3, 8, 2, 333, 128
    N = num_tree_nodes(b, d)
    (q, k, v), (Qd, Kd, Vd) = _inputs(B, Hq, Hkv, N, L, D, 7400, dtype=torch.bfloat16)
    O = ra.ragged_tree_attn(Qd, Kd, Vd, b, d)
    _check(O, None, q, k, v, L, b, d, dtype=torch.bfloat16)


def test_verify_graph_replay():
    """Captured once, replayed with new inputs copied in between: every replay
    matches the eager call on the same inputs (no host sync, no allocation in
    the captured region)."""
    ra = _ra()
    B, b, d, Hq, Hkv, L, D = 2, 4, 3, 8, 2, 500, 128
    N = num_tree_nodes(b, d)
    (_, _, _), (Qd, Kd, Vd) = _inputs(B, Hq, Hkv, N, L, D, 7500)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        ra.ragged_tree_attn(Qd, Kd, Vd, b, d)  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(st)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        Og = ra.ragged_tree_attn(Qd, Kd, Vd, b, d)
    for r in range(3):
        (_, _, _), (Qn, Kn, Vn) = _inputs(B, Hq, Hkv, N, L, D, 7501 + r)
        Qd.copy_(Qn)
        Kd.copy_(Kn)
        Vd.copy_(Vn)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ref = ra.ragged_tree_attn(Qd, Kd, Vd, b, d)
        torch.cuda.synchronize()
        assert torch.equal(Og, ref), f"replay {r}"


def test_verify_empty():
    ra = _ra()
    Q = torch.zeros(0, 4, 5, 64, dtype=torch.float16, device=DEV)
    K = torch.zeros(0, 4, 9, 64, dtype=torch.float16, device=DEV)
    assert ra.ragged_tree_attn(Q, K, K, 2, 2).shape == (0, 4, 5, 64)
    Q = torch.zeros(2, 4, 0, 64, dtype=torch.float16, device=DEV)
    K = torch.zeros(2, 4, 9, 64, dtype=torch.float16, device=DEV)
    assert ra.ragged_tree_attn(Q, K, K, 2, 2).shape == (2, 4, 0, 64)
