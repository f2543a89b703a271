"""Host-side checks that need no GPU: the C ABI library loads and exports every
declared symbol, argument validation returns the documented error codes
before touching the device, and the host utilities match the oracle."""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np
import pytest
import torch

from conftest import ROOT, make_inputs, num_tree_nodes
from oracle import clib, tree
from qattention_amd import _lib
from qattention_amd import ragged_attn as ra
from qattention_amd import tree_mask as tm

HEADER = os.path.join(ROOT, "include", "qattn.h")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qattn_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = _declared_symbols()
    for s in ("qattn_tree_fwd", "qattn_tree_parents_fwd", "qattn_tree_paged_fwd",
              "qattn_ancestors", "qattn_lse_merge", "qattn_last_error", "qattn_version"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for s in _declared_symbols():
        assert hasattr(L, s), s
        assert s in _lib.SIGNATURES, f"{s} has no ctypes signature"
    assert L.qattn_version().startswith(b"qattention_amd")


def test_single_hip_runtime_mapped():
    _lib.lib()
    maps = open(f"/proc/{os.getpid()}/maps").read()
    hip = {l.split()[-1] for l in maps.splitlines() if "libamdhip64" in l}
    assert len(hip) == 1, hip


def _divide(x, d):
    """Python restatement of qattn::make_divider / divide (qattn_common.h)."""
    l = 0
    while (1 << l) < d:
        l += 1
    m = ((1 << 32) * ((1 << l) - d)) // d + 1
    hi = (x * m) >> 32
    return ((hi + x) & 0xFFFFFFFF) >> l


def test_divider_exact():
    rng = np.random.default_rng(0)
    xs = list(range(0, 4097)) + [2**31 - 1, 2**31 - 2, 2**30, 2**24 + 1] + \
        [int(v) for v in rng.integers(0, 2**31, 2000)]
    for d in list(range(1, 70)) + [100, 127, 1000, 4096, 65535, 65537, 2**20 + 7, 2**30 + 1, 2**31 - 1]:
        for x in xs:
            assert _divide(x, d) == x // d, (x, d)


# ---------------------------------------------------------------------------
# C ABI argument validation (returns before any device call)
# ---------------------------------------------------------------------------

FAKE = 1 << 20  # a non-null, 16-byte aligned address that is never dereferenced


def _tree_call(dtype=0, head_dim=64, q=FAKE, qs=(256, 64, 1), hq=4, hkv=4, b=2, md=3, batch=1):
    L = _lib.lib()
    st = _lib.i64arr(qs)
    ok = _lib.i64arr((256, 64, 1))
    return L.qattn_tree_fwd(q, st, FAKE, ok, FAKE, ok, FAKE, ok, None, None, FAKE, batch, 15, 15,
                            hq, hkv, head_dim, b, md, 0.125, dtype, 0, None)


def test_abi_validation_codes():
    assert _tree_call(dtype=7) == -2
    assert _tree_call(head_dim=96) == -3
    assert _tree_call(q=0) == -1
    assert _tree_call(qs=(256, 64, 2)) == -4
    assert _tree_call(qs=(250, 64, 1)) == -4
    assert _tree_call(q=FAKE + 2) == -4
    assert _tree_call(hq=6, hkv=4) == -1
    assert _tree_call(b=0) == -1
    assert _tree_call(md=-1) == -1
    assert "head_dim" in _lib.last_error() or _tree_call(head_dim=96) == -3
    assert _tree_call(batch=0) == 0  # nothing to do: no launch


def test_abi_validation_other_entry_points():
    L = _lib.lib()
    ok3 = _lib.i64arr((256, 64, 1))
    ok4 = _lib.i64arr((4096, 256, 64, 1))
    assert L.qattn_tree_parents_fwd(FAKE, ok3, FAKE, ok3, FAKE, ok3, FAKE, ok3, FAKE, _lib.i64arr((4, 1)),
                                    FAKE, None, 1, 15, 15, 4, 4, 64, 3, 0.125, 0, None) == -1
    assert L.qattn_tree_paged_fwd(FAKE, ok3, FAKE, ok4, FAKE, ok4, FAKE, ok3, None, None, FAKE, FAKE,
                                  4, 4, 0, 1, 15, 15, 4, 4, 64, 2, 3, 0.125, 0, 0, None) == -1
    ok_pt = (FAKE, ok3, FAKE, ok4, FAKE, ok4, FAKE, ok3, None, None, FAKE, FAKE, 4, 4, 16, 1, 15, 15, 4, 4, 64, 2, 3,
             0.125, 0)
    assert L.qattn_tree_paged_fwd(*ok_pt, 3, None) == -1  # unknown algo
    assert "algo" in _lib.last_error()
    assert L.qattn_ancestors(FAKE, None, 1, 15, 15, 0, 3, FAKE, None) == -1
    s3 = _lib.i64arr((60, 15, 1))
    assert L.qattn_lse_merge(FAKE, s3, FAKE, s3, FAKE, ok4, FAKE, ok4, FAKE, ok4, 1, 4, 15, 48, 0, None) == -3
    assert L.qattn_lse_merge(FAKE, s3, FAKE, s3, FAKE, ok4, FAKE, ok4, FAKE, ok4, 1, 4, 15, 64, 3, None) == -2


def test_abi_prefix_stride_limits():
    """The prefix kernel addresses a 64-key block with 32-bit byte offsets:
    token strides of 2^25 elements or more, or negative ones, are a layout
    error; an in-range layout gets past that check (and stops at the missing
    workspace, before any launch)."""
    L = _lib.lib()
    ok3 = _lib.i64arr((256, 64, 1))

    def call(kp):
        return L.qattn_prefix_tree_fwd(FAKE, ok3, FAKE, ok3, FAKE, ok3, FAKE, _lib.i64arr(kp), FAKE,
                                       _lib.i64arr((512 * 256, 256, 64)), 512, FAKE, ok3, None, None, FAKE,
                                       1, 15, 15, 0, 0, 4, 4, 64, 2, 3, 0.125, 0, None, 0, 0, None)

    assert call((1 << 40, 1 << 25, 64)) == -4
    assert call((512 * 256, -256, 64)) == -4
    assert call((512 * 256, (1 << 25) - 8, 64)) == -5
    assert call((512 * 256, 256, 64)) == -5
    # the explicit-parents variant needs a parent array
    kp = _lib.i64arr((512 * 256, 256, 64))
    assert L.qattn_prefix_tree_parents_fwd(FAKE, ok3, FAKE, ok3, FAKE, ok3, FAKE, kp, FAKE, kp, 512, FAKE, ok3,
                                           None, None, FAKE, None, 1, 15, 15, 0, 0, 4, 4, 64, 3, 0.125, 0,
                                           None, 0, 0, None) == -1


def test_abi_prefix_only_validation():
    """qattn_prefix_fwd: no tree keys, so null k/v are fine; an empty prefix,
    a non-positive scale or a bad prefix layout is rejected before any launch,
    and a valid layout with forced splits stops at the missing workspace."""
    L = _lib.lib()
    ok3 = _lib.i64arr((256, 64, 1))
    kp = (512 * 256, 256, 64)

    def call(prefix_len=512, kps=kp, scale=0.125, dtype=0, head_dim=64, splits=2, batch=1):
        return L.qattn_prefix_fwd(FAKE, ok3, FAKE, _lib.i64arr(kps), FAKE, _lib.i64arr(kp), prefix_len,
                                  FAKE, ok3, None, None, FAKE, batch, 15, 15, 4, 4, head_dim, scale, dtype,
                                  None, 0, splits, None)

    assert call(prefix_len=0) == -1
    assert call(scale=0.0) == -1
    assert call(scale=-0.1) == -1
    assert call(dtype=3) == -2
    assert call(head_dim=48) == -3
    assert call(kps=(512 * 256, 1 << 25, 64)) == -4
    assert call(kps=(512 * 256, 252, 64)) == -4
    assert call() == -5
    assert call(batch=0) == 0
    # two splits of (m, l, numerator / l) over 15 tokens x 4 heads, sized for
    # fp32 states (bf16 inputs; fp16 ones store the numerator in half of it),
    # each array 256-byte aligned
    a256 = lambda x: (x + 255) // 256 * 256
    assert L.qattn_prefix_workspace_bytes(1, 15, 15, 4, 4, 64, 512, 2) == 2 * a256(2 * 60 * 4) + a256(2 * 60 * 64 * 4)


def test_abi_prefix_split_rule():
    """The automatic prefix split count, read back through the workspace size
    (one (m, l, acc) state per split; a single split fuses the walk and needs
    none): enough (sequence, kv head, 128-row tile) units for ~512 workgroups,
    at least an eighth of the 64-key blocks (2..8) per split."""
    L = _lib.lib()
    a256 = lambda x: (x + 255) // 256 * 256

    def ws(splits, T, Hq, D):
        return 0 if splits <= 1 else 2 * a256(splits * T * Hq * 4) + a256(splits * T * Hq * D * 4)

    # one EAGLE-3 step: 16 units, 32 blocks -> 8 splits of 4 blocks
    assert L.qattn_prefix_workspace_bytes(1, 60, 60, 32, 8, 128, 2048, 0) == ws(8, 60, 32, 128)
    # cfg4: 96 units -> 5 splits (of 32 blocks)
    assert L.qattn_prefix_workspace_bytes(4, 85, 340, 32, 8, 128, 10240, 0) == ws(5, 340, 32, 128)
    # cfg5: 18944 units fill the GPU -> one split
    assert L.qattn_prefix_workspace_bytes(16, 4681, 16 * 4681, 32, 32, 128, 2048, 0) == 0
    # a 2-block prefix stays whole; a 16-block one splits into 8 of 2
    assert L.qattn_prefix_workspace_bytes(1, 60, 60, 32, 8, 128, 128, 0) == 0
    assert L.qattn_prefix_workspace_bytes(1, 60, 60, 32, 8, 128, 1024, 0) == ws(8, 60, 32, 128)


def test_abi_ragged_tree_attn_validation():
    """qattn_ragged_tree_attn_fwd over [B, H, N, D] strides: every layout it
    cannot address is rejected before any launch; a valid layout with L = 512
    and two forced splits stops at the missing workspace."""
    L = _lib.lib()
    B, H, N, P, D = 2, 4, 15, 512, 64
    q4 = (H * N * D, N * D, D, 1)
    k4 = (H * (P + N) * D, (P + N) * D, D, 1)

    def call(qs=q4, ks=k4, vs=k4, dtype=0, head_dim=D, batch=B, num_prefix=P, par=None, par_stride=0,
             lse=None, lss=None):
        arr = lambda t: None if t is None else _lib.i64arr(t)
        return L.qattn_ragged_tree_attn_fwd(FAKE, arr(qs), FAKE, arr(ks), FAKE, arr(vs), FAKE, arr(q4), lse,
                                            arr(lss), par, par_stride, batch, N, num_prefix, H, H, head_dim,
                                            2, 3, 0.125, dtype, None, 0, 2, None)

    assert call(dtype=5) == -2
    assert call(head_dim=96) == -3
    assert call(qs=None) == -1
    assert call(lse=FAKE) == -1                                       # lse without strides
    assert call(num_prefix=-1) == -1
    assert call(par=FAKE, par_stride=-1) == -1
    assert call(qs=(q4[0] + 4,) + q4[1:]) == -4                       # batch stride breaks row alignment
    assert call(ks=(k4[0] + 8,) + k4[1:]) == -4                       # not a whole number of rows
    assert call(vs=(2 * k4[0],) + k4[1:]) == -4                       # k and v place sequences differently
    assert call(ks=(0,) + k4[1:], vs=(0,) + k4[1:]) == -4             # sequences sharing one k/v
    assert call(qs=q4[:3] + (2,)) == -4                               # stride_dim != 1
    assert call() == -5
    assert call(par=FAKE, par_stride=N, lse=FAKE, lss=(H * N, N, 1)) == -5
    # one sequence: its batch strides are never used
    assert call(batch=1, qs=(3,) + q4[1:], ks=(5,) + k4[1:], vs=(7,) + k4[1:]) == -5
    assert call(batch=0) == 0


# ---------------------------------------------------------------------------
# Python API behaviour on the host
# ---------------------------------------------------------------------------

def test_dtype_assertion_matches_reference():
    Q, K, V, cu = make_inputs([7], 4, 64, 1, torch.float32)
    with pytest.raises(AssertionError):
        ra.ragged_attention(Q, K, V, cu, 2, 2)
    Q16 = Q.half()
    with pytest.raises(AssertionError):
        ra.ragged_attention(Q16, K.bfloat16(), V.half(), cu, 2, 2)


def test_cpu_tensors_fail_loudly():
    Q, K, V, cu = make_inputs([7], 4, 64, 1, torch.float16)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ra.ragged_attention(Q, K, V, cu, 2, 2)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ra.ragged_attention_with_parents(Q, K, V, cu, torch.zeros(7, dtype=torch.int32), 2)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ra.ragged_tree_attn(Q.view(1, 7, 4, 64).transpose(1, 2), K.view(1, 7, 4, 64).transpose(1, 2),
                            V.view(1, 7, 4, 64).transpose(1, 2), 2, 2)


def test_pack_inputs():
    qs = [torch.randn(n, 2, 8) for n in (3, 0, 5)]
    Q, K, V, cu = ra.pack_inputs(qs, qs, qs)
    assert cu.dtype == torch.int32 and cu.tolist() == [0, 3, 3, 8]
    assert torch.equal(Q, torch.cat(qs, 0)) and Q.shape == (8, 2, 8)


def test_build_paged_kv_roundtrip():
    g = torch.Generator().manual_seed(3)
    ks = [torch.randn(n, 2, 8, generator=g) for n in (5, 16, 17, 1)]
    vs = [torch.randn(n, 2, 8, generator=g) for n in (5, 16, 17, 1)]
    Kc, Vc, pt = ra.build_paged_kv(ks, vs, page_size=4)
    assert pt.dtype == torch.int32 and pt.shape == (4, 5)
    assert Kc.shape == (2 + 4 + 5 + 1, 4, 2, 8)
    for b, (k, v) in enumerate(zip(ks, vs)):
        for c in range(k.shape[0]):
            page = int(pt[b, c // 4])
            assert torch.equal(Kc[page, c % 4], k[c]) and torch.equal(Vc[page, c % 4], v[c])


@pytest.mark.parametrize("b,d", [(1, 5), (2, 3), (3, 3), (4, 2), (8, 2)])
def test_tree_mask_module_matches_oracle(b, d):
    assert tm.num_tree_nodes(b, d) == tree.num_tree_nodes(b, d)
    assert tm.build_tree(b, d) == tree.build_tree(b, d)
    assert (tm.tree_attention_mask(b, d) == tree.tree_attention_mask(b, d)).all()
    n = num_tree_nodes(b, d)
    assert (tm.tree_attention_mask_n(b, n - 1) == tree.tree_attention_mask_n(b, n - 1)).all()
    assert tm.verify_tree_mask(b, d, verbose=False)
    assert (tm.tree_attention_mask_pruned(tm.build_tree(b, d)) == tree.tree_attention_mask(b, d)).all()
    fm = tm.full_sequence_mask(3, b, d)
    assert fm.shape == (3 + n, 3 + n) and fm[3:, :3].all() and not fm[0, 1]


def test_kernel_parents_self_loop():
    p = tm.kernel_parents([-1, 0, 0, 1])
    assert p.tolist() == [0, 0, 0, 1] and p.dtype == np.int32
    cu = np.array([0, 4], dtype=np.int32)
    assert (clib.ancestor_table_parents(cu, p, 3) == clib.ancestor_table_heap(cu, 2, 3)).all()


def test_src_shim_reexports():
    import src.ragged_attn as sra
    import src.tree_mask as stm
    for name in ("pack_inputs", "ragged_attention", "ragged_attention_with_lse", "ragged_attention_sibling",
                 "ragged_attention_sibling_with_lse", "ragged_attention_with_parents",
                 "ragged_attention_paged", "build_paged_kv", "fused_lse_merge", "ragged_tree_attn"):
        assert getattr(sra, name) is getattr(ra, name)
    assert stm.tree_attention_mask is tm.tree_attention_mask


def test_layout_copies_switch():
    """Inputs the kernels cannot read as 16-byte rows are copied by default
    (any strides work, as in the reference); with set_layout_copies(False)
    they raise instead, so a call allocates nothing beyond its outputs."""
    import torch
    from qattention_amd import ragged_attn as ra

    base = torch.zeros(16, 4, 130, dtype=torch.float16)
    ok = base[:, :, :128]              # outer strides 520 and 130: 130 % 8 != 0
    assert not ra._vec_ok(ok)
    assert ra._vec(ok).is_contiguous()
    good = torch.zeros(16, 4, 128, dtype=torch.float16)
    assert ra._vec(good) is good
    prev = ra.set_layout_copies(False)
    try:
        assert prev is True
        assert ra._vec(good) is good
        with pytest.raises(ValueError, match="layout copies are off"):
            ra._vec(ok)
    finally:
        ra.set_layout_copies(prev)
    assert ra._vec(ok).is_contiguous()
