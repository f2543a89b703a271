"""Ancestor-sparse tree-verify attention on MI355X -- the `src.ragged_attn` API.

Host side of the drop-in replacement for the reference module
src/ragged_attn.py (saifmb0/QAttention).  Names, argument order, defaults,
return values and error behaviour follow the reference; the work is done by
hand-written gfx950 HIP kernels in libqattn.so, called through its C ABI
(include/qattn.h) on torch's current HIP stream.  Outputs are allocated here
through the torch caching allocator.  A call is HIP-graph capturable when
max_seqlen is given (no host sync).  The library itself allocates nothing;
the first call on a device runs qattn_init() there (outside graph capture),
which sets up the subtree kernel's schedule counters.

Differences from the reference, all supersets:
  * K/V may carry fewer heads than Q (GQA): q head h reads kv head
    h // (Hq // Hkv), exactly what repeat_kv would have produced.
  * Inputs whose last dim is not unit-stride or whose rows are not 16-byte
    aligned are copied to a contiguous layout first (the reference accepts any
    strides; the HIP kernels read 16-byte vectors).  Such a copy is the only
    allocation a call makes besides its outputs and workspace (under graph
    capture it comes from the graph's pool); set_layout_copies(False) makes
    those inputs raise ValueError instead.
  * bf16 runs natively (the reference casts bf16 to fp16 below SM 8.9,
    src/ragged_attn.py:1118-1127; gfx950 has bf16 dot/MFMA instructions).
"""
from __future__ import annotations

import math
from typing import List, Optional, Tuple

import torch

from . import _lib

_SUPPORTED = (torch.float16, torch.bfloat16)


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------

def _check_dtypes(Q, K, V):
    # src/ragged_attn.py:1113-1116
    assert Q.dtype in _SUPPORTED and Q.dtype == K.dtype == V.dtype, (
        f"Inputs must be fp16 or bf16 (got {Q.dtype})"
    )


def _dtype_code(t: torch.Tensor) -> int:
    return _lib.DTYPE_F16 if t.dtype == torch.float16 else _lib.DTYPE_BF16


def _vec_ok(t: torch.Tensor) -> bool:
    """Rows readable as 16-byte vectors: unit last stride, 8-element aligned
    outer strides, 16-byte aligned base."""
    if t.numel() == 0:
        return True
    st = t.stride()
    return st[-1] == 1 and all(s % 8 == 0 for s in st[:-1]) and t.data_ptr() % 16 == 0


_LAYOUT_COPIES = [True]


def set_layout_copies(allowed: bool) -> bool:
    """Whether inputs the kernels cannot read as 16-byte rows are copied to a
    contiguous layout (True, the default: any strides work, as in the
    reference) or rejected with ValueError (False: a call then never allocates
    beyond its outputs and workspace).  Returns the previous setting."""
    prev = _LAYOUT_COPIES[0]
    _LAYOUT_COPIES[0] = bool(allowed)
    return prev


def _vec(t: torch.Tensor) -> torch.Tensor:
    if _vec_ok(t):
        return t
    if not _LAYOUT_COPIES[0]:
        raise ValueError(f"tensor of shape {tuple(t.shape)} and strides {tuple(t.stride())} is not readable as "
                         "16-byte rows (unit last stride, 8-element aligned strides, 16-byte aligned base) and "
                         "layout copies are off (set_layout_copies)")
    return t.contiguous()


def _require_device(*ts):
    dev = ts[0].device
    if dev.type != "cuda":
        raise RuntimeError(
            "qattention_amd runs on a ROCm GPU only (got tensors on "
            f"{dev}); there is no CPU path")
    for t in ts[1:]:
        if t.device != dev:
            raise RuntimeError(f"all tensors must be on {dev} (got {t.device})")
    return dev


def _stream(device) -> int:
    _lib.ensure_init(device)
    return torch.cuda.current_stream(device).cuda_stream


def _seqlens(cu_seqlens: torch.Tensor, B: int, device, max_seqlen: Optional[int]):
    """max_seqlen and a device int32 copy of cu_seqlens (src/ragged_attn.py:1136-1142).

    When max_seqlen is None it is computed from a host copy of cu_seqlens
    (a device->host sync only if cu_seqlens lives on the GPU, as in the
    reference); pass it explicitly for graph capture."""
    if max_seqlen is None:
        cu_cpu = cu_seqlens.cpu()
        sl = cu_cpu.tolist()
        max_seqlen = int(max(sl[i + 1] - sl[i] for i in range(B))) if B else 1
        cu_dev = cu_cpu.to(device=device, dtype=torch.int32, non_blocking=True)
    else:
        cu_dev = cu_seqlens.to(device=device, dtype=torch.int32, non_blocking=True)
    return max(int(max_seqlen), 0), cu_dev.contiguous()


_ONE_SEQ_CU: dict = {}


def _one_sequence_cu(T: int, device) -> torch.Tensor:
    """Device cu_seqlens [0, T] for queries that form one sequence, made by
    fill kernels (no host-to-device copy, so a call under graph capture
    records it); kept per (device, T) when made outside capture."""
    key = (device.index if device.index is not None else torch.cuda.current_device(), T)
    cu = _ONE_SEQ_CU.get(key)
    if cu is None:
        cu = torch.full((2,), T, dtype=torch.int32, device=device)
        cu[:1].fill_(0)  # (a fill kernel; `cu[0] = 0` would copy a host scalar)
        if not torch.cuda.is_current_stream_capturing():
            if len(_ONE_SEQ_CU) >= 256:
                _ONE_SEQ_CU.clear()
            _ONE_SEQ_CU[key] = cu
    return cu


def _heads(Q, K, V):
    T, Hq, D = Q.shape
    Hkv = K.shape[1]
    if K.shape[-1] != D or V.shape[-1] != D or V.shape[-2] != Hkv:
        raise ValueError(f"shape mismatch: Q {tuple(Q.shape)} K {tuple(K.shape)} V {tuple(V.shape)}")
    if Hkv < 1 or Hq % Hkv != 0:
        raise ValueError(f"num q heads {Hq} must be a multiple of num kv heads {Hkv}")
    return T, Hq, Hkv, D


# ---------------------------------------------------------------------------
# core launcher for the heap walk
# ---------------------------------------------------------------------------

def _tree_forward(Q, K, V, cu_seqlens, branching_factor: int, max_depth: int,
                  max_seqlen: Optional[int], want_lse: bool, algo: int = _lib.ALGO_AUTO):
    _check_dtypes(Q, K, V)
    device = _require_device(Q, K, V)
    T, Hq, Hkv, D = _heads(Q, K, V)
    if K.shape[0] != T or V.shape[0] != T:
        raise ValueError("packed Q, K, V must have the same number of tokens")
    B = int(cu_seqlens.shape[0]) - 1
    ms, cu_dev = _seqlens(cu_seqlens, B, device, max_seqlen)
    Q, K, V = _vec(Q), _vec(K), _vec(V)
    O = torch.empty_like(Q)
    if not _vec_ok(O):
        O = torch.empty(Q.shape, dtype=Q.dtype, device=device)
    LSE = torch.empty(T, Hq, dtype=torch.float32, device=device) if want_lse else None
    scale = 1.0 / math.sqrt(D)
    L = _lib.lib()
    with torch.cuda.device(device):
        rc = L.qattn_tree_fwd(
            Q.data_ptr(), _lib.i64arr(Q.stride()), K.data_ptr(), _lib.i64arr(K.stride()),
            V.data_ptr(), _lib.i64arr(V.stride()), O.data_ptr(), _lib.i64arr(O.stride()),
            _lib.ptr(LSE), _lib.i64arr(LSE.stride()) if LSE is not None else None,
            cu_dev.data_ptr(), B, ms, T, Hq, Hkv, D, int(branching_factor), int(max_depth),
            scale, _dtype_code(Q), int(algo), _stream(device))
    _lib.check(rc, "qattn_tree_fwd")
    return O, LSE


# ---------------------------------------------------------------------------
# public API (src/ragged_attn.py:1054-1166, 499-572, 1423-1556)
# ---------------------------------------------------------------------------

def pack_inputs(
    qs: List[torch.Tensor],
    ks: List[torch.Tensor],
    vs: List[torch.Tensor],
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Concatenate per-sequence [L_i, H, D] tensors into the packed ragged
    layout; cu_seqlens is a CPU int32 [B+1] prefix sum (src/ragged_attn.py:1054-1077)."""
    assert len(qs) == len(ks) == len(vs)
    lens = torch.tensor([0] + [q.shape[0] for q in qs], dtype=torch.int64)
    cu_seqlens = torch.cumsum(lens, 0).to(torch.int32)
    return torch.cat(qs, 0), torch.cat(ks, 0), torch.cat(vs, 0), cu_seqlens


def ragged_attention(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    cu_seqlens: torch.Tensor,
    branching_factor: int,
    max_depth: int,
    max_seqlen: int = None,
) -> torch.Tensor:
    """Ancestor-sparse attention for BFS-ordered complete b-ary trees.

    Query token x of each sequence attends to {parent^s(x) : s = 0..max_depth}
    with parent(k) = max(k - 1, 0) // b (src/ragged_attn.py:1080-1166).
    Q, K, V: packed [sum L_i, H, D] fp16/bf16 on the GPU (K/V may have fewer
    heads, GQA); cu_seqlens: [B+1] int32 on host or device.
    Returns O with Q's dtype and shape.
    """
    return _tree_forward(Q, K, V, cu_seqlens, branching_factor, max_depth, max_seqlen, False)[0]


def ragged_attention_with_lse(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    cu_seqlens: torch.Tensor,
    branching_factor: int,
    max_depth: int,
    max_seqlen: int = None,
) -> tuple:
    """As ragged_attention, also returning LSE [sum L_i, H] fp32 (natural log)
    for merging with another attention block (src/ragged_attn.py:499-572)."""
    return _tree_forward(Q, K, V, cu_seqlens, branching_factor, max_depth, max_seqlen, True)


def ragged_attention_sibling(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    cu_seqlens: torch.Tensor,
    branching_factor: int,
    max_depth: int,
    max_seqlen: int = None,
) -> torch.Tensor:
    """Same function as ragged_attention (src/ragged_attn.py:1423-1492).

    The reference keeps a second Triton kernel that only reorders load issue;
    here both names run the same HIP kernels, which already issue every
    ancestor load of a step chunk before the softmax chain."""
    return _tree_forward(Q, K, V, cu_seqlens, branching_factor, max_depth, max_seqlen, False)[0]


def ragged_attention_sibling_with_lse(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    cu_seqlens: torch.Tensor,
    branching_factor: int,
    max_depth: int,
    max_seqlen: int = None,
) -> tuple:
    """Same function as ragged_attention_with_lse (src/ragged_attn.py:1495-1556)."""
    return _tree_forward(Q, K, V, cu_seqlens, branching_factor, max_depth, max_seqlen, True)


def ragged_attention_with_parents(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    cu_seqlens: torch.Tensor,
    parents: torch.Tensor,
    max_depth: int,
    max_seqlen: int = None,
) -> tuple:
    """Ancestor-sparse attention over an explicit parent array
    (src/ragged_attn.py:716-795).

    parents: int32 [sum L_i], sequence-local parent of every token; a root
    must self-loop (parents[root] == root).  Returns (O, LSE)."""
    _check_dtypes(Q, K, V)
    device = _require_device(Q, K, V)
    T, Hq, Hkv, D = _heads(Q, K, V)
    if K.shape[0] != T or V.shape[0] != T:
        raise ValueError("packed Q, K, V must have the same number of tokens")
    if parents.numel() < T:
        raise ValueError(f"parents has {parents.numel()} entries for {T} tokens")
    B = int(cu_seqlens.shape[0]) - 1
    ms, cu_dev = _seqlens(cu_seqlens, B, device, max_seqlen)
    par = parents.to(device=device, dtype=torch.int32, non_blocking=True).contiguous()
    Q, K, V = _vec(Q), _vec(K), _vec(V)
    O = torch.empty_like(Q)
    if not _vec_ok(O):
        O = torch.empty(Q.shape, dtype=Q.dtype, device=device)
    LSE = torch.empty(T, Hq, dtype=torch.float32, device=device)
    L = _lib.lib()
    with torch.cuda.device(device):
        rc = L.qattn_tree_parents_fwd(
            Q.data_ptr(), _lib.i64arr(Q.stride()), K.data_ptr(), _lib.i64arr(K.stride()),
            V.data_ptr(), _lib.i64arr(V.stride()), O.data_ptr(), _lib.i64arr(O.stride()),
            LSE.data_ptr(), _lib.i64arr(LSE.stride()), cu_dev.data_ptr(), par.data_ptr(),
            B, ms, T, Hq, Hkv, D, int(max_depth), 1.0 / math.sqrt(D), _dtype_code(Q),
            _stream(device))
    _lib.check(rc, "qattn_tree_parents_fwd")
    return O, LSE


def ragged_attention_paged(
    Q: torch.Tensor,
    K_cache: torch.Tensor,
    V_cache: torch.Tensor,
    page_table: torch.Tensor,
    cu_seqlens: torch.Tensor,
    branching_factor: int,
    max_depth: int,
    max_seqlen: int = None,
) -> torch.Tensor:
    """Ancestor-sparse attention reading K/V from a paged cache
    (src/ragged_attn.py:932-1003).  max_seqlen (not in the reference, which
    always reads cu_seqlens on the host) skips that read, as in
    ragged_attention, so the call can be captured in a graph.

    K_cache/V_cache: [pages, PAGE_SIZE, Hkv, D]; page_table: [B, max_pages]
    int32 logical->physical page map; ancestor position c of sequence b is
    slot c % PAGE_SIZE of page page_table[b, c // PAGE_SIZE]."""
    return _paged_forward(Q, K_cache, V_cache, page_table, cu_seqlens, branching_factor, max_depth, max_seqlen,
                          False)[0]


def _paged_forward(Q, K_cache, V_cache, page_table, cu_seqlens, branching_factor, max_depth, max_seqlen,
                   want_lse: bool, algo: int = _lib.ALGO_AUTO):
    """ragged_attention_paged with an optional LSE ([T, Hq] fp32; -inf for a
    query that attends nothing) and a kernel choice (tests time and check
    both kernels)."""
    assert K_cache.shape == V_cache.shape, "K and V cache shapes must match"
    _check_dtypes(Q, K_cache, V_cache)
    device = _require_device(Q, K_cache, V_cache)
    T, Hq, D = Q.shape
    num_pages, page_size, Hkv, Dk = K_cache.shape
    if Dk != D or Hkv < 1 or Hq % Hkv != 0:
        raise ValueError(f"cache shape {tuple(K_cache.shape)} incompatible with Q {tuple(Q.shape)}")
    B = int(cu_seqlens.shape[0]) - 1
    ms, cu_dev = _seqlens(cu_seqlens, B, device, max_seqlen)
    pt = page_table.to(device=device, dtype=torch.int32, non_blocking=True).contiguous()
    if pt.dim() != 2 or pt.shape[0] < B:
        raise ValueError(f"page_table must be [B, max_pages] (got {tuple(page_table.shape)})")
    Q, K_cache, V_cache = _vec(Q), _vec(K_cache), _vec(V_cache)
    O = torch.empty_like(Q)
    if not _vec_ok(O):
        O = torch.empty(Q.shape, dtype=Q.dtype, device=device)
    lse = torch.empty(T, Hq, dtype=torch.float32, device=device) if want_lse else None
    L = _lib.lib()
    with torch.cuda.device(device):
        rc = L.qattn_tree_paged_fwd(
            Q.data_ptr(), _lib.i64arr(Q.stride()), K_cache.data_ptr(), _lib.i64arr(K_cache.stride()),
            V_cache.data_ptr(), _lib.i64arr(V_cache.stride()), O.data_ptr(), _lib.i64arr(O.stride()),
            lse.data_ptr() if want_lse else None, _lib.i64arr(lse.stride()) if want_lse else None,
            cu_dev.data_ptr(), pt.data_ptr(), int(pt.stride(0)), num_pages, page_size,
            B, ms, T, Hq, Hkv, D, int(branching_factor), int(max_depth), 1.0 / math.sqrt(D),
            _dtype_code(Q), int(algo), _stream(device))
    _lib.check(rc, "qattn_tree_paged_fwd")
    return O, lse


def build_paged_kv(
    ks: List[torch.Tensor],
    vs: List[torch.Tensor],
    page_size: int = 16,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Pack per-sequence [L_i, H, D] K/V into a paged cache
    (src/ragged_attn.py:1006-1047): pages are assigned in sequence order,
    unused slots are zero; page_table is a CPU int32 [B, max_pages] tensor."""
    B = len(ks)
    H, D = ks[0].shape[1], ks[0].shape[2]
    device, dtype = ks[0].device, ks[0].dtype
    pages = [(k.shape[0] + page_size - 1) // page_size for k in ks]
    max_pages, total = max(pages), sum(pages)
    K_cache = torch.zeros(total, page_size, H, D, device=device, dtype=dtype)
    V_cache = torch.zeros(total, page_size, H, D, device=device, dtype=dtype)
    page_table = torch.zeros(B, max_pages, dtype=torch.int32)
    phys = 0
    for b, (k, v) in enumerate(zip(ks, vs)):
        n = k.shape[0]
        full = n // page_size
        if full:
            K_cache[phys:phys + full] = k[:full * page_size].reshape(full, page_size, H, D)
            V_cache[phys:phys + full] = v[:full * page_size].reshape(full, page_size, H, D)
        if n % page_size:
            r = n % page_size
            K_cache[phys + full, :r] = k[full * page_size:]
            V_cache[phys + full, :r] = v[full * page_size:]
        page_table[b, :pages[b]] = torch.arange(phys, phys + pages[b], dtype=torch.int32)
        phys += pages[b]
    return K_cache, V_cache, page_table


def _prefix_tree_forward(Q, K, V, cu_dev, B: int, max_seqlen: int, Kp, kp_stride, Vp, vp_stride,
                         prefix_len: int, branching_factor: int, max_depth: int, tree_seq_stride: int,
                         tree_row0: int, want_lse: bool, num_splits: int = 0, parents=None):
    """Launch qattn_prefix_tree_fwd (heap walk) or qattn_prefix_tree_parents_fwd
    (parents given, a device int32 tensor): MFMA prefix splits + ancestor walk,
    one normalisation.  K/V hold the tree rows (addressed through cu_dev or
    tree_seq_stride/tree_row0); Kp/Vp + 3 strides address the prefix rows."""
    device = Q.device
    T, Hq, D = Q.shape
    Hkv = K.shape[1]
    O = torch.empty_like(Q)
    if not _vec_ok(O):
        O = torch.empty(Q.shape, dtype=Q.dtype, device=device)
    LSE = torch.empty(T, Hq, dtype=torch.float32, device=device) if want_lse else None
    L = _lib.lib()
    ws_bytes = int(L.qattn_prefix_workspace_bytes(B, max_seqlen, T, Hq, Hkv, D, int(prefix_len), int(num_splits)))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    head = (Q.data_ptr(), _lib.i64arr(Q.stride()), K.data_ptr(), _lib.i64arr(K.stride()),
            V.data_ptr(), _lib.i64arr(V.stride()), _lib.ptr(Kp), _lib.i64arr(kp_stride),
            _lib.ptr(Vp), _lib.i64arr(vp_stride), int(prefix_len),
            O.data_ptr(), _lib.i64arr(O.stride()), _lib.ptr(LSE),
            _lib.i64arr(LSE.stride()) if LSE is not None else None, cu_dev.data_ptr())
    sizes = (B, max_seqlen, T, int(tree_seq_stride), int(tree_row0), Hq, Hkv, D)
    tail = (ws.data_ptr(), ws_bytes, int(num_splits), _stream(device))
    with torch.cuda.device(device):
        if parents is None:
            rc = L.qattn_prefix_tree_fwd(*head, *sizes, int(branching_factor), int(max_depth), 1.0 / math.sqrt(D),
                                         _dtype_code(Q), *tail)
            what = "qattn_prefix_tree_fwd"
        else:
            rc = L.qattn_prefix_tree_parents_fwd(*head, parents.data_ptr(), *sizes, int(max_depth),
                                                 1.0 / math.sqrt(D), _dtype_code(Q), *tail)
            what = "qattn_prefix_tree_parents_fwd"
    _lib.check(rc, what)
    return O, LSE


def ragged_attention_hybrid(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    prefix_length: int,
    tree_size: int,
    branching_factor: int,
    max_depth: int,
) -> torch.Tensor:
    """Dense prefix + ancestor-sparse tree in one state (src/ragged_attn.py:1851-1888).

    Q: [B*N, H, D]; K, V: [B*(L+N), Hkv, D] with each sequence's L prefix rows
    followed by its N tree rows (Hkv may divide H: GQA).  Every query attends
    all L prefix rows of its sequence plus its tree ancestors."""
    _check_dtypes(Q, K, V)
    device = _require_device(Q, K, V)
    T, Hq, Hkv, D = _heads(Q, K, V)
    N, L = int(tree_size), int(prefix_length)
    if N <= 0 or T % N:
        raise ValueError(f"Q has {T} rows, not a multiple of tree_size {N}")
    B = T // N
    if K.shape[0] != B * (L + N) or V.shape[0] != B * (L + N):
        raise ValueError(f"K/V must have B*(L+N) = {B * (L + N)} rows (got {K.shape[0]})")
    Q, K, V = _vec(Q), _vec(K), _vec(V)
    cu = torch.arange(0, (B + 1) * N, N, dtype=torch.int32, device=device)
    kp_stride = (K.stride(0) * (L + N), K.stride(0), K.stride(1))
    vp_stride = (V.stride(0) * (L + N), V.stride(0), V.stride(1))
    return _prefix_tree_forward(Q, K, V, cu, B, N, K if L else None, kp_stride, V if L else None, vp_stride,
                                L, branching_factor, max_depth, L + N, L, False)[0]


def ragged_attention_prefix(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    cu_seqlens: torch.Tensor,
    K_prefix: torch.Tensor,
    V_prefix: torch.Tensor,
    branching_factor: int,
    max_depth: int,
    max_seqlen: int = None,
    return_lse: bool = False,
    num_splits: int = 0,
    parents: torch.Tensor = None,
):
    """Tree-verify attention over a prefix KV cache, GQA-native, in one pass.

    Replaces the reference's verify pipeline "prefix flash attention with LSE +
    ragged_attention_with_lse + fused_lse_merge" (scripts/benchmark_micro.py:568-593,
    scripts/e2e_benchmark.py:1394-1502) without repeat_kv and without the
    intermediate O/LSE round trips.

    Q: packed [T, Hq, D]; K, V: packed tree rows [T, Hkv, D]; cu_seqlens [B+1];
    K_prefix, V_prefix: [B, L, Hkv, D] per-sequence or [L, Hkv, D] shared by
    all sequences, any strides with a unit last dim (e.g. a permuted view of a
    [B, Hkv, L, D] cache).  parents (optional): int32 [T] sequence-local
    parent of every token, roots self-looping, as in ragged_attention_with_parents
    -- the EAGLE-3 dynamic tree of scripts/e2e_benchmark.py:1469-1474; then
    branching_factor is ignored.  Returns O (and LSE [T, Hq] if return_lse)."""
    _check_dtypes(Q, K, V)
    assert K_prefix.dtype == Q.dtype and V_prefix.dtype == Q.dtype, "prefix dtype must match Q"
    device = _require_device(Q, K, V, K_prefix, V_prefix)
    T, Hq, Hkv, D = _heads(Q, K, V)
    if K.shape[0] != T or V.shape[0] != T:
        raise ValueError("packed Q, K, V must have the same number of tokens")
    B = int(cu_seqlens.shape[0]) - 1
    if K_prefix.dim() == 3:
        K_prefix, V_prefix = K_prefix.unsqueeze(0), V_prefix.unsqueeze(0)
        shared = True
    else:
        shared = False
    if K_prefix.shape != V_prefix.shape or K_prefix.shape[2:] != (Hkv, D) or (not shared and K_prefix.shape[0] != B):
        raise ValueError(f"prefix shape {tuple(K_prefix.shape)} incompatible with B={B}, Hkv={Hkv}, D={D}")
    L = int(K_prefix.shape[1])
    ms, cu_dev = _seqlens(cu_seqlens, B, device, max_seqlen)
    Q, K, V = _vec(Q), _vec(K), _vec(V)
    K_prefix, V_prefix = _vec(K_prefix), _vec(V_prefix)
    kp_stride = (0 if shared else K_prefix.stride(0), K_prefix.stride(1), K_prefix.stride(2))
    vp_stride = (0 if shared else V_prefix.stride(0), V_prefix.stride(1), V_prefix.stride(2))
    par = None
    if parents is not None:
        if parents.numel() < T:
            raise ValueError(f"parents has {parents.numel()} entries for {T} tokens")
        par = parents.to(device=device, dtype=torch.int32, non_blocking=True).contiguous()
    O, LSE = _prefix_tree_forward(Q, K, V, cu_dev, B, ms, K_prefix if L else None, kp_stride,
                                  V_prefix if L else None, vp_stride, L, branching_factor, max_depth, 0, 0,
                                  return_lse, num_splits, par)
    return (O, LSE) if return_lse else O


def prefix_attention(
    Q: torch.Tensor,
    K_prefix: torch.Tensor,
    V_prefix: torch.Tensor,
    cu_seqlens: Optional[torch.Tensor] = None,
    max_seqlen: int = None,
    return_lse: bool = True,
    num_splits: int = 0,
):
    """Attention of packed queries over a prefix KV cache only, with LSE: the
    prefix pass of the reference's verify pipelines, GQA-native.

    Replaces flashinfer.single_prefill_with_kv_cache_return_lse(Q, K_sh, V_sh,
    causal=False) as scripts/benchmark_micro.py:574-580 calls it (a prefix
    [L, Hkv, D] shared by every query; cu_seqlens None: all of Q is one
    sequence) and the aten flash prefix pass with LSE of the E2E verify step
    (scripts/e2e_benchmark.py:1438-1448; K_prefix [B, L, Hkv, D], one prefix
    per sequence of cu_seqlens).  Its output merges with a tree pass through
    fused_lse_merge.  Returns O [T, Hq, D] (and LSE [T, Hq] fp32, natural
    log, if return_lse)."""
    if Q.dtype not in _SUPPORTED or K_prefix.dtype != Q.dtype or V_prefix.dtype != Q.dtype:
        raise AssertionError(f"Inputs must be fp16 or bf16 (got {Q.dtype})")
    device = _require_device(Q, K_prefix, V_prefix)
    T, Hq, D = Q.shape
    shared = K_prefix.dim() == 3
    if shared:
        K_prefix, V_prefix = K_prefix.unsqueeze(0), V_prefix.unsqueeze(0)
    Hkv = K_prefix.shape[2]
    if cu_seqlens is None:
        cu_seqlens = _one_sequence_cu(T, device)  # capturable: no host copy
        max_seqlen = T
    B = int(cu_seqlens.shape[0]) - 1
    if (K_prefix.shape != V_prefix.shape or K_prefix.shape[3] != D or Hkv < 1 or Hq % Hkv
            or (not shared and K_prefix.shape[0] != B)):
        raise ValueError(f"prefix shape {tuple(K_prefix.shape)} incompatible with Q {tuple(Q.shape)}, B={B}")
    L = int(K_prefix.shape[1])
    if L < 1:
        raise ValueError("prefix_attention needs a prefix of at least one row")
    ms, cu_dev = _seqlens(cu_seqlens, B, device, max_seqlen)
    Q, K_prefix, V_prefix = _vec(Q), _vec(K_prefix), _vec(V_prefix)
    kp_stride = (0 if shared else K_prefix.stride(0), K_prefix.stride(1), K_prefix.stride(2))
    vp_stride = (0 if shared else V_prefix.stride(0), V_prefix.stride(1), V_prefix.stride(2))
    O = torch.empty_like(Q)
    if not _vec_ok(O):
        O = torch.empty(Q.shape, dtype=Q.dtype, device=device)
    LSE = torch.empty(T, Hq, dtype=torch.float32, device=device) if return_lse else None
    lib = _lib.lib()
    ws_bytes = int(lib.qattn_prefix_workspace_bytes(B, ms, T, Hq, Hkv, D, L, int(num_splits))) if T else 0
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    with torch.cuda.device(device):
        rc = lib.qattn_prefix_fwd(
            Q.data_ptr(), _lib.i64arr(Q.stride()), K_prefix.data_ptr(), _lib.i64arr(kp_stride),
            V_prefix.data_ptr(), _lib.i64arr(vp_stride), L, O.data_ptr(), _lib.i64arr(O.stride()),
            _lib.ptr(LSE), _lib.i64arr(LSE.stride()) if LSE is not None else None, cu_dev.data_ptr(),
            B, ms, T, Hq, Hkv, D, 1.0 / math.sqrt(D), _dtype_code(Q), ws.data_ptr(), ws_bytes,
            int(num_splits), _stream(device))
    _lib.check(rc, "qattn_prefix_fwd")
    return (O, LSE) if return_lse else O


def ragged_tree_attn(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    branching_factor: int,
    max_depth: int,
    tree_parents: Optional[torch.Tensor] = None,
    return_lse: bool = False,
    num_splits: int = 0,
):
    """EAGLE-3 tree verification over the attention layer's own [B, H, N, D]
    tensors, in one launch sequence with no copies: the replacement for
    _ragged_tree_attn (scripts/e2e_benchmark.py:1394-1502), same arguments
    and result.

    Q: [B, Hq, N_q, D]; K, V: [B, Hkv, N_kv, D] with N_kv = N_prefix + N_q
    (each sequence's prefix rows, visible to every tree token, then its tree
    tokens in BFS order); Hkv may divide Hq (GQA, no repeat_kv needed).  Any
    strides with a unit last dim work in place (permuted views, slices of a
    larger cache).  tree_parents: int32 [N_q] sequence-local parents shared
    by every sequence (the reference's case, :1470) or [B, N_q] one tree per
    sequence; the root is its own parent.  Otherwise the heap tree of
    branching_factor is walked (:1475-1478).  Returns O [B, Hq, N_q, D] (and
    LSE [B, Hq, N_q] fp32, natural log, if return_lse)."""
    _check_dtypes(Q, K, V)
    device = _require_device(Q, K, V)
    if Q.dim() != 4 or K.dim() != 4 or V.dim() != 4 or K.shape != V.shape:
        raise ValueError(f"expected [B, H, N, D] tensors: Q {tuple(Q.shape)} K {tuple(K.shape)} V {tuple(V.shape)}")
    B, Hq, N, D = Q.shape
    Hkv, N_kv = K.shape[1], K.shape[2]
    if K.shape[0] != B or K.shape[3] != D or N_kv < N:
        raise ValueError(f"K/V {tuple(K.shape)} incompatible with Q {tuple(Q.shape)}")
    if Hkv < 1 or Hq % Hkv:
        raise ValueError(f"num q heads {Hq} must be a multiple of num kv heads {Hkv}")
    L = N_kv - N
    Q = _vec(Q)
    K, V = _vec(K), _vec(V)
    if B > 1:
        # the kernels place sequence s's k/v rows at s * (batch stride / token
        # stride): both tensors need the same whole-row batch stride
        kr = K.stride(0) // K.stride(2) if K.stride(2) > 0 and K.stride(0) % K.stride(2) == 0 else -1
        vr = V.stride(0) // V.stride(2) if V.stride(2) > 0 and V.stride(0) % V.stride(2) == 0 else -1
        if kr <= 0 or kr != vr:
            K, V = K.contiguous(), V.contiguous()
    O = torch.empty(B, Hq, N, D, dtype=Q.dtype, device=device)
    LSE = torch.empty(B, Hq, N, dtype=torch.float32, device=device) if return_lse else None
    par, par_stride = None, 0
    if tree_parents is not None:
        if tree_parents.dim() == 1 and tree_parents.shape[0] == N:
            par_stride = 0
        elif tree_parents.dim() == 2 and tuple(tree_parents.shape) == (B, N):
            par_stride = N
        else:
            tree_parents = None  # the reference falls back to the heap walk (:1470, :1475)
        if tree_parents is not None:
            par = tree_parents.to(device=device, dtype=torch.int32, non_blocking=True).contiguous()
    lib = _lib.lib()
    ws_bytes = int(lib.qattn_prefix_workspace_bytes(B, N, B * N, Hq, Hkv, D, L, int(num_splits))) if B * N else 0
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    with torch.cuda.device(device):
        rc = lib.qattn_ragged_tree_attn_fwd(
            Q.data_ptr(), _lib.i64arr(Q.stride()), K.data_ptr(), _lib.i64arr(K.stride()),
            V.data_ptr(), _lib.i64arr(V.stride()), O.data_ptr(), _lib.i64arr(O.stride()),
            _lib.ptr(LSE), _lib.i64arr(LSE.stride()) if LSE is not None else None,
            _lib.ptr(par), par_stride, B, N, L, Hq, Hkv, D, int(branching_factor), int(max_depth),
            1.0 / math.sqrt(D), _dtype_code(Q), ws.data_ptr(), ws_bytes, int(num_splits), _stream(device))
    _lib.check(rc, "qattn_ragged_tree_attn_fwd")
    return (O, LSE) if return_lse else O


def fused_lse_merge(
    lse_pre: torch.Tensor,
    lse_tree: torch.Tensor,
    out_pre: torch.Tensor,
    out_tree: torch.Tensor,
) -> torch.Tensor:
    """Online-softmax merge of two attention blocks (src/ragged_attn.py:1619-1653).

    lse_*: [B, H, Nq] (any float dtype; read as fp32), out_*: [B, H, Nq, D]
    fp16/bf16 of any layout with a unit last stride.  Returns a contiguous
    [B, H, Nq, D] tensor in out_pre's dtype."""
    B, H, Nq, D = out_pre.shape
    if out_tree.shape != out_pre.shape or lse_pre.shape != (B, H, Nq) or lse_tree.shape != (B, H, Nq):
        raise ValueError("fused_lse_merge: shape mismatch")
    device = _require_device(out_pre, out_tree, lse_pre, lse_tree)
    if out_pre.dtype not in _SUPPORTED:
        raise AssertionError(f"Inputs must be fp16 or bf16 (got {out_pre.dtype})")
    out_tree = out_tree.to(out_pre.dtype)
    lse_p = lse_pre.float()
    lse_t = lse_tree.float()
    op, ot = _vec(out_pre), _vec(out_tree)
    result = torch.empty(B, H, Nq, D, dtype=out_pre.dtype, device=device)
    L = _lib.lib()
    with torch.cuda.device(device):
        rc = L.qattn_lse_merge(
            lse_p.data_ptr(), _lib.i64arr(lse_p.stride()), lse_t.data_ptr(), _lib.i64arr(lse_t.stride()),
            op.data_ptr(), _lib.i64arr(op.stride()), ot.data_ptr(), _lib.i64arr(ot.stride()),
            result.data_ptr(), _lib.i64arr(result.stride()), B, H, Nq, D, _dtype_code(op),
            _stream(device))
    _lib.check(rc, "qattn_lse_merge")
    return result


def ancestor_table(cu_seqlens: torch.Tensor, branching_factor: int, max_depth: int,
                   parents: Optional[torch.Tensor] = None, max_seqlen: int = None,
                   device=None) -> torch.Tensor:
    """Ancestor index table [sum L_i, max_depth+1] int32 from the device walk
    (entry -1 = step not attended).  Exposes the walk the attention kernels
    use (src/ragged_attn.py:323-377, :650-698) for bit-exact checks."""
    device = torch.device(device) if device is not None else torch.device("cuda")
    B = int(cu_seqlens.shape[0]) - 1
    T = int(cu_seqlens[-1])
    ms, cu_dev = _seqlens(cu_seqlens, B, device, max_seqlen)
    out = torch.full((T, max_depth + 1), -1, dtype=torch.int32, device=device)
    par = None
    if parents is not None:
        par = parents.to(device=device, dtype=torch.int32).contiguous()
    L = _lib.lib()
    with torch.cuda.device(device):
        rc = L.qattn_ancestors(cu_dev.data_ptr(), _lib.ptr(par), B, ms, T, int(branching_factor),
                               int(max_depth), out.data_ptr(), _stream(device))
    _lib.check(rc, "qattn_ancestors")
    return out
