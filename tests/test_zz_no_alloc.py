"""qattn_ragged_tree_attn_fwd_noalloc (the allocation-free variant of the
[B, H, N, D] verify entry point, split states in the library's static scratch
array) against qattn_ragged_tree_attn_fwd with a caller workspace, through
the C ABI: bit-equal outputs and LSE on two calls in a row, the second with
a smaller input (the scratch keeps the first call's contents), plus the
split-count limit of the 32 MiB scratch (sized by dtype: fp16 split states
hold fp16 numerators, bf16 ones fp32)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import oracle_tree

pytestmark = pytest.mark.gpu

DEV = "cuda"


def say(*a):
    print(*a, flush=True)


def _case(B, N, L, Hq, Hkv, D, seed, parents=False, dtype=torch.float16):
    """Q [B, Hq, N, D], K/V [B, Hkv, L + N, D] (prefix rows then tree rows),
    optional shared parent array [N] (the root its own parent)."""
    g = torch.Generator().manual_seed(seed)
    Q = torch.randn(B, Hq, N, D, generator=g).to(dtype)
    K = torch.randn(B, Hkv, L + N, D, generator=g).to(dtype)
    V = torch.randn(B, Hkv, L + N, D, generator=g).to(dtype)
    par = None
    if parents:
        rng = np.random.default_rng(seed)
        par = np.array([0] + [int(rng.integers(max(0, i - 5), i)) for i in range(1, N)], dtype=np.int32)
    return Q, K, V, par


def _call(Q, K, V, par, b, md, num_splits, noalloc):
    """One call through the C ABI; returns (rc, O, LSE)."""
    from qattention_amd import _lib
    lib = _lib.lib()
    B, Hq, N, D = Q.shape
    Hkv, NK = K.shape[1], K.shape[2]
    L = NK - N
    Qd, Kd, Vd = Q.to(DEV), K.to(DEV), V.to(DEV)
    O = torch.full((B, Hq, N, D), float("nan"), dtype=Q.dtype, device=DEV)
    LSE = torch.full((B, Hq, N), float("nan"), dtype=torch.float32, device=DEV)
    pd = torch.from_numpy(par).to(DEV) if par is not None else None
    head = (Qd.data_ptr(), _lib.i64arr(Qd.stride()), Kd.data_ptr(), _lib.i64arr(Kd.stride()),
            Vd.data_ptr(), _lib.i64arr(Vd.stride()), O.data_ptr(), _lib.i64arr(O.stride()),
            LSE.data_ptr(), _lib.i64arr(LSE.stride()), _lib.ptr(pd), 0,
            B, N, L, Hq, Hkv, D, b, md, 1.0 / math.sqrt(D),
            _lib.DTYPE_F16 if Q.dtype == torch.float16 else _lib.DTYPE_BF16)
    st = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.qattn_ragged_tree_attn_fwd_noalloc(*head, num_splits, st)
    else:
        ws_bytes = int(lib.qattn_prefix_workspace_bytes(B, N, B * N, Hq, Hkv, D, L, num_splits))
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
        rc = lib.qattn_ragged_tree_attn_fwd(*head, ws.data_ptr(), ws_bytes, num_splits, st)
    torch.cuda.synchronize()
    return rc, O, LSE


def test_noalloc_matches_workspace_entry():
    from qattention_amd import _lib
    # call 1 (large, bf16): 4 automatic splits would need 34.1 MB of fp32
    # split state, more than the 32 MiB scratch: the automatic count drops to 3
    say("noalloc call 1: B=2 N=256 L=10240 Hq=32 Hkv=8 heap b=4 bf16")
    Qb, Kb, Vb, _ = _case(2, 256, 10240, 32, 8, 128, 11, dtype=torch.bfloat16)
    rc, O1, L1 = _call(Qb, Kb, Vb, None, 4, 4, 0, True)
    assert rc == 0, _lib.last_error()
    rc, O1w, L1w = _call(Qb, Kb, Vb, None, 4, 4, 3, False)
    assert rc == 0, _lib.last_error()
    assert torch.equal(O1, O1w) and torch.equal(L1, L1w)
    # an explicit split count whose states do not fit is refused
    rc, _, _ = _call(Qb, Kb, Vb, None, 4, 4, 4, True)
    assert rc == -5  # QATTN_ERR_WORKSPACE
    assert "scratch" in _lib.last_error()
    # the same shape in fp16: 4 splits hold 17.3 MB of split state (fp16
    # numerators) and run as asked for; 8 would need 34.6 MB and are refused
    say("noalloc call 1b: the same shape in fp16")
    Q, K, V, _ = _case(2, 256, 10240, 32, 8, 128, 11)
    rc, O1, L1 = _call(Q, K, V, None, 4, 4, 0, True)
    assert rc == 0, _lib.last_error()
    rc, O1w, L1w = _call(Q, K, V, None, 4, 4, 4, False)
    assert rc == 0, _lib.last_error()
    assert torch.equal(O1, O1w) and torch.equal(L1, L1w)
    rc, _, _ = _call(Q, K, V, None, 4, 4, 8, True)
    assert rc == -5  # QATTN_ERR_WORKSPACE
    # call 2 (smaller, right after): an EAGLE-3-like step over a parent
    # array, automatic split count (fits), same result as the workspace entry
    say("noalloc call 2: B=1 N=60 L=2048 Hq=32 Hkv=8 parents")
    Q2, K2, V2, par = _case(1, 60, 2048, 32, 8, 128, 12, parents=True)
    rc, O2, L2 = _call(Q2, K2, V2, par, 1, 7, 0, True)
    assert rc == 0, _lib.last_error()
    rc, O2w, L2w = _call(Q2, K2, V2, par, 1, 7, 0, False)
    assert rc == 0, _lib.last_error()
    assert torch.equal(O2, O2w) and torch.equal(L2, L2w)
    # and both agree with the oracle (prefix rows all attended + ancestors)
    N, L = 60, 2048
    Qp = Q2[0].permute(1, 0, 2).contiguous()                 # [N, Hq, D]
    Kt = K2[0, :, L:].permute(1, 0, 2).contiguous()          # [N, Hkv, D]
    Vt = V2[0, :, L:].permute(1, 0, 2).contiguous()
    Kp = K2[0, :, :L].permute(1, 0, 2).unsqueeze(0).contiguous()  # [1, L, Hkv, D]
    Vp = V2[0, :, :L].permute(1, 0, 2).unsqueeze(0).contiguous()
    cu = torch.tensor([0, N], dtype=torch.int32)
    o_ref, lse_ref, _ = oracle_tree(Qp, Kt, Vt, cu, 1, 7, parents=par, Kp=Kp, Vp=Vp)
    o = O2[0].permute(1, 0, 2).double().cpu().numpy()
    assert np.abs(o - o_ref).max() <= 2e-3
    assert np.abs(L2[0].permute(1, 0).double().cpu().numpy() - lse_ref).max() <= 1e-4


def test_noalloc_single_split_and_tree_only():
    """A short prefix runs as one split (no split state: the scratch is not
    touched) and num_prefix 0 is the tree-only path; both bit-equal the
    workspace entry."""
    from qattention_amd import _lib
    for (B, N, L) in ((2, 85, 64), (3, 85, 0)):
        say("noalloc", B, N, L)
        Q, K, V, _ = _case(B, N, L, 8, 2, 128, 13 + L)
        rc, O, Ls = _call(Q, K, V, None, 4, 3, 0, True)
        assert rc == 0, _lib.last_error()
        rc, Ow, Lw = _call(Q, K, V, None, 4, 3, 0, False)
        assert rc == 0, _lib.last_error()
        assert torch.equal(O, Ow) and torch.equal(Ls, Lw)
