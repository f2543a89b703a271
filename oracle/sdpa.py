"""The reference's own oracle: padded SDPA with an additive tree-mask bias.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates tests/test_correctness.py:50-124 (padded SDPA, MATH backend, fp32,
bias 0 / finfo(fp32).min/2, scale 1/sqrt(D), padding trimmed) and its prefix
variant :444-469 (prefix columns all-attend).  GQA is handled by
repeat-interleaving K/V heads as repeat_kv does
(scripts/e2e_benchmark.py:1581).  Runs on the CPU.
"""
from __future__ import annotations

import math
from typing import List, Optional

import numpy as np
import torch
import torch.nn.functional as F

NEG_INF = torch.finfo(torch.float32).min / 2


def _expand_kv(t: torch.Tensor, hq: int) -> torch.Tensor:
    """[.., Hkv, D] -> [.., Hq, D] by repeat-interleave along the head dim."""
    hkv = t.shape[-2]
    if hkv == hq:
        return t
    return torch.repeat_interleave(t, hq // hkv, dim=-2)


def padded_sdpa(qs: List[torch.Tensor], ks: List[torch.Tensor], vs: List[torch.Tensor],
                masks: List[np.ndarray],
                kps: Optional[List[torch.Tensor]] = None,
                vps: Optional[List[torch.Tensor]] = None,
                return_lse: bool = False):
    """Per-sequence lists: q [n_i,Hq,D], k/v [n_i,Hkv,D], mask [n_i,n_i] bool,
    optional prefix kp/vp [L,Hkv,D] (attended by every query).

    Returns (list of fp32 [n_i,Hq,D], list of fp32 [n_i,Hq] LSE or None).
    """
    B = len(qs)
    Hq, D = qs[0].shape[1], qs[0].shape[2]
    L = 0 if kps is None else kps[0].shape[0]
    lens = [q.shape[0] for q in qs]
    nmax = max(lens) if lens else 0

    def pad(ts, rows):
        out = torch.zeros(B, rows, Hq, D, dtype=torch.float32)
        for i, t in enumerate(ts):
            out[i, :t.shape[0]] = _expand_kv(t.float(), Hq)
        return out.permute(0, 2, 1, 3)  # [B, H, rows, D]

    Qp = pad(qs, nmax)
    if L:
        kcat = [torch.cat([kp.float(), k.float()], 0) for kp, k in zip(kps, ks)]
        vcat = [torch.cat([vp.float(), v.float()], 0) for vp, v in zip(vps, vs)]
    else:
        kcat, vcat = ks, vs
    Kp = pad(kcat, L + nmax)
    Vp = pad(vcat, L + nmax)

    bias = torch.full((B, 1, nmax, L + nmax), NEG_INF, dtype=torch.float32)
    for i, (n, m) in enumerate(zip(lens, masks)):
        mt = torch.from_numpy(np.asarray(m, dtype=bool))
        bias[i, 0, :n, :L] = 0.0
        bias[i, 0, :n, L:L + n] = torch.where(mt, torch.zeros(()), torch.full((), NEG_INF))

    scale = 1.0 / math.sqrt(D)
    with torch.nn.attention.sdpa_kernel(torch.nn.attention.SDPBackend.MATH):
        out = F.scaled_dot_product_attention(Qp, Kp, Vp, attn_mask=bias, scale=scale)
    out = out.permute(0, 2, 1, 3)  # [B, nmax, H, D]
    outs = [out[i, :lens[i]].contiguous() for i in range(B)]
    lses = None
    if return_lse:
        # LSE of the same masked scores (src/ragged_attn.py:484-488 defines
        # lse = m + log(l) in natural log): logsumexp(scale*QK^T + bias).
        s = torch.matmul(Qp, Kp.transpose(-1, -2).contiguous()) * scale + bias
        lse = torch.logsumexp(s, dim=-1)  # [B, H, nmax]
        lses = [lse[i, :, :lens[i]].transpose(0, 1).contiguous() for i in range(B)]
    return outs, lses


def split_packed(t: torch.Tensor, cu) -> List[torch.Tensor]:
    cu = [int(x) for x in cu]
    return [t[cu[i]:cu[i + 1]] for i in range(len(cu) - 1)]


def packed_tree_attention(Q, K, V, cu, masks, Kp=None, Vp=None, return_lse=False):
    """Packed-layout convenience wrapper around padded_sdpa.

    Q [T,Hq,D], K/V [T,Hkv,D], cu [B+1]; masks: list of per-sequence bool
    masks; Kp/Vp optional [B,L,Hkv,D].  Returns fp32 O [T,Hq,D] (and LSE
    [T,Hq])."""
    qs, ks, vs = split_packed(Q, cu), split_packed(K, cu), split_packed(V, cu)
    kps = vps = None
    if Kp is not None:
        kps = [Kp[i] for i in range(Kp.shape[0])]
        vps = [Vp[i] for i in range(Vp.shape[0])]
    outs, lses = padded_sdpa(qs, ks, vs, masks, kps, vps, return_lse=return_lse)
    O = torch.cat(outs, 0) if outs else torch.zeros(0, *Q.shape[1:])
    if return_lse:
        return O, torch.cat(lses, 0)
    return O
