"""Seeded random GPU parity sweep across the entry points.

Each case draws a shape (ragged sequence lengths, branching factor,
max_depth, head dim, GQA group, dtype, input scale) and one of the call
paths: the packed heap walk (gather or subtree kernel), the explicit-parents
walk, paged K/V, the prefix path (split or fused), and the [B, H, N, D]
verify call.  Every case is checked against the fp64 oracle on the same
rounded inputs, O and, where the path returns it, LSE.  Sizes are small so
the CPU oracle finishes in well under a second per case."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import make_inputs, oracle_tree

pytestmark = pytest.mark.gpu

DEV = "cuda"
PATHS = ("heap", "parents", "paged", "prefix", "verify")
CASES = 256


def say(*a):
    print(*a, flush=True)


def _ra():
    from qattention_amd import ragged_attn
    return ragged_attn


def _close(o, o_ref, dtype, what, sigma=1.0):
    # fp16, inputs of scale sigma <= 1: the north-star bound as stated,
    # max |o - o_ref| <= 2e-3 absolute.  For sigma > 1 (outside the
    # north-star's N(0, 1) inputs) rounding errors grow with the size of the
    # V rows an output mixes, not only with |O| (split states and P round
    # before the weights cancel): 2e-3 * max(sigma, |O|).
    s = max(1.0, sigma)
    if dtype == torch.float16:
        bound = 2e-3 if sigma <= 1.0 else 2e-3 * np.maximum(sigma, np.abs(o_ref))
        err = np.abs(o - o_ref)
        assert (err <= bound).all(), f"{what}: max abs err {err.max():.3e} (bound {np.min(bound):.1e}+)"
    else:
        bound = 2.0 ** -7 * np.maximum(s, np.abs(o_ref)) + 1e-3 * s
        assert (np.abs(o - o_ref) <= bound).all(), f"{what}: bf16 err {np.abs(o - o_ref).max():.3e}"


def _draw(seed):
    rng = np.random.default_rng(9000 + seed)
    path = PATHS[seed % len(PATHS)]
    D = int(rng.choice([32, 64, 128]))
    Hkv = int(rng.choice([1, 2, 4]))
    Hq = Hkv * int(rng.choice([1, 2, 4]))
    dtype = torch.float16 if rng.random() < 0.7 else torch.bfloat16
    b = int(rng.integers(1, 7))
    md = int(rng.integers(0, 9))
    B = int(rng.integers(1, 5))
    uniform = path == "verify"
    n = int(rng.integers(1, 200))
    lens = [n] * B if uniform else [int(rng.integers(0, 200)) for _ in range(B)]
    if sum(lens) == 0:
        lens[0] = 1
    sigma = float(rng.choice([0.5, 1.0, 2.0]))
    return rng, path, dict(D=D, Hq=Hq, Hkv=Hkv, dtype=dtype, b=b, md=md, lens=lens, sigma=sigma)


def _random_parents(rng, lens):
    out = []
    for n in lens:
        p = np.zeros(n, dtype=np.int32)
        for i in range(1, n):
            p[i] = rng.integers(max(0, i - 8), i)
        out.append(p)
    return np.concatenate(out) if out else np.zeros(0, dtype=np.int32)


@pytest.mark.parametrize("seed", range(CASES))
def test_random_case(seed):
    ra = _ra()
    rng, path, c = _draw(seed)
    D, Hq, Hkv, dtype, b, md, lens = c["D"], c["Hq"], c["Hkv"], c["dtype"], c["b"], c["md"], c["lens"]
    say("random", seed, path, {k: (str(v) if k == "dtype" else v) for k, v in c.items()})
    Q, K, V, cu = make_inputs(lens, Hq, D, 9100 + seed, dtype=dtype, Hkv=Hkv, sigma=c["sigma"])
    B = len(lens)
    if path == "heap":
        algo = int(rng.integers(0, 3))  # auto, gather, subtree (subtree needs a plan that fits)
        try:
            O, LSE = ra._tree_forward(Q.to(DEV), K.to(DEV), V.to(DEV), cu, b, md, None, True, algo)
        except RuntimeError as e:
            assert algo == 2 and "no subtree plan fits" in str(e), e
            O, LSE = ra._tree_forward(Q.to(DEV), K.to(DEV), V.to(DEV), cu, b, md, None, True, 0)
        o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, b, md)
    elif path == "parents":
        par = _random_parents(rng, lens)
        O, LSE = ra.ragged_attention_with_parents(Q.to(DEV), K.to(DEV), V.to(DEV), cu, torch.from_numpy(par), md)
        o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, b, md, parents=par)
    elif path == "paged":
        ps = int(rng.choice([1, 3, 16, 64]))
        cuL = cu.tolist()
        ks = [K[cuL[i]:cuL[i + 1]].to(DEV) for i in range(B)]
        vs = [V[cuL[i]:cuL[i + 1]].to(DEV) for i in range(B)]
        if min(lens) == 0:  # build_paged_kv needs a row per sequence; pad empty ones
            ks = [k if k.shape[0] else torch.zeros(1, Hkv, D, dtype=dtype, device=DEV) for k in ks]
            vs = [v if v.shape[0] else torch.zeros(1, Hkv, D, dtype=dtype, device=DEV) for v in vs]
        Kc, Vc, pt = ra.build_paged_kv(ks, vs, page_size=ps)
        perm = torch.from_numpy(rng.permutation(Kc.shape[0]))
        inv = torch.empty_like(perm)
        inv[perm] = torch.arange(perm.numel())
        Kc, Vc = Kc[perm.to(DEV)].contiguous(), Vc[perm.to(DEV)].contiguous()
        pt = inv[pt.long()].to(torch.int32)
        O = ra.ragged_attention_paged(Q.to(DEV), Kc, Vc, pt, cu, b, md)
        LSE = None
        o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, b, md)
    elif path == "prefix":
        L = int(rng.integers(1, 400))
        g = torch.Generator().manual_seed(9200 + seed)
        Kp = (torch.randn(B, L, Hkv, D, generator=g) * c["sigma"]).to(dtype)
        Vp = (torch.randn(B, L, Hkv, D, generator=g) * c["sigma"]).to(dtype)
        ns = int(rng.choice([0, 1, 3]))
        par = _random_parents(rng, lens) if rng.random() < 0.4 else None
        O, LSE = ra.ragged_attention_prefix(Q.to(DEV), K.to(DEV), V.to(DEV), cu, Kp.to(DEV), Vp.to(DEV), b, md,
                                            return_lse=True, num_splits=ns,
                                            parents=None if par is None else torch.from_numpy(par))
        o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, b, md, parents=par, Kp=Kp, Vp=Vp)
    else:  # verify: [B, H, N, D] views with the prefix rows ahead of the tree rows
        N = lens[0]
        L = int(rng.integers(0, 300))
        g = torch.Generator().manual_seed(9300 + seed)
        Kp = (torch.randn(B, L, Hkv, D, generator=g) * c["sigma"]).to(dtype)
        Vp = (torch.randn(B, L, Hkv, D, generator=g) * c["sigma"]).to(dtype)
        q4 = Q.view(B, N, Hq, D).permute(0, 2, 1, 3)
        k4 = torch.cat([Kp, K.view(B, N, Hkv, D)], 1).permute(0, 2, 1, 3)
        v4 = torch.cat([Vp, V.view(B, N, Hkv, D)], 1).permute(0, 2, 1, 3)
        shared = rng.random() < 0.5
        par = _random_parents(rng, [N]) if shared else None
        O4, L4 = ra.ragged_tree_attn(q4.to(DEV), k4.to(DEV), v4.to(DEV), b, md,
                                     tree_parents=None if par is None else torch.from_numpy(par).to(DEV),
                                     return_lse=True)
        O = O4.permute(0, 2, 1, 3).reshape(B * N, Hq, D)
        LSE = L4.permute(0, 2, 1).reshape(B * N, Hq)
        o_ref, lse_ref, _ = oracle_tree(Q, K, V, cu, b, md, parents=None if par is None else np.tile(par, B),
                                        Kp=Kp if L else None, Vp=Vp if L else None)
    _close(O.double().cpu().numpy(), o_ref, dtype, f"case {seed} ({path})", c["sigma"])
    if LSE is not None:
        err = float(np.abs(LSE.double().cpu().numpy() - lse_ref).max()) if LSE.numel() else 0.0
        assert err <= (1e-4 if dtype == torch.float16 else 1e-3) * max(1.0, c["sigma"] ** 2), \
            f"case {seed} ({path}): LSE err {err:.3e}"
