"""Generate the committed golden fixtures (tests/golden/*.npz).

    python tests/golden/make_golden.py

The reference repository commits no golden vectors (its tests draw inputs
from the CUDA device RNG, tests/test_correctness.py:180-185), so the fixtures
are produced by this repository's oracle (oracle/, pinned by
tests/test_oracle.py) on inputs drawn on the CPU from an explicit
torch.Generator with the reference's seed convention B*10000 + b*100 + d
(scripts/benchmark_micro.py:303).  Each .npz holds the inputs (as stored:
fp32 for the CPU config, fp16-rounded values for GPU cases), cu_seqlens, the
walk parameters, the ancestor table, and the output and LSE (computed in
fp64, stored as fp32).

Cases
  cfg1            BASELINE configs[0]: B=2, b=2 d=3 (N=15), H=4, D=64, fp32
  chain_b1_d8     linear chain = causal attention (tests/test_correctness.py:339-350)
  single_b1_d0    single-token trees (:325-336)
  b3_d3_D128      H=2, D=128
  b4_d2_D32       H=4, D=32
  trunc_b2        31-node binary trees walked with max_depth=2 < depth 4
  ragged          unequal and empty sequences, b=3, max_depth=3
  gqa             Hq=8, Hkv=2, b=2, d=4
  parents         irregular trees through an explicit parent array
  prefix          L=24 all-attended prefix rows + b=2 d=3 tree, Hq=4, Hkv=2
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import clib  # noqa: E402


def _inputs(lens, Hq, D, seed, dtype, Hkv=None, extra_prefix=0):
    Hkv = Hq if Hkv is None else Hkv
    T = int(sum(lens))
    g = torch.Generator().manual_seed(seed)
    Q = torch.randn(T, Hq, D, generator=g).to(dtype)
    K = torch.randn(T, Hkv, D, generator=g).to(dtype)
    V = torch.randn(T, Hkv, D, generator=g).to(dtype)
    Kp = Vp = None
    if extra_prefix:
        B = len(lens)
        Kp = torch.randn(B, extra_prefix, Hkv, D, generator=g).to(dtype)
        Vp = torch.randn(B, extra_prefix, Hkv, D, generator=g).to(dtype)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    return Q, K, V, cu, Kp, Vp


def _case(name, lens, Hq, D, b, max_depth, seed, dtype=torch.float16, Hkv=None, parents=None,
          prefix=0):
    Q, K, V, cu, Kp, Vp = _inputs(lens, Hq, D, seed, dtype, Hkv, prefix)
    if parents is None:
        anc = clib.ancestor_table_heap(cu, b, max_depth)
    else:
        anc = clib.ancestor_table_parents(cu, parents, max_depth)
    o, lse = clib.tree_attn(Q.float().numpy(), K.float().numpy(), V.float().numpy(), cu, anc,
                            1.0 / np.sqrt(D),
                            None if Kp is None else Kp.float().numpy(),
                            None if Vp is None else Vp.float().numpy())
    np_dtype = np.float32 if dtype == torch.float32 else np.float16
    out = dict(q=Q.numpy().astype(np_dtype), k=K.numpy().astype(np_dtype), v=V.numpy().astype(np_dtype),
               cu=cu, b=np.int32(b), max_depth=np.int32(max_depth), anc=anc,
               o=o.astype(np.float32), lse=lse.astype(np.float32))
    if parents is not None:
        out["parents"] = np.asarray(parents, dtype=np.int32)
    if prefix:
        out["kp"] = Kp.numpy().astype(np_dtype)
        out["vp"] = Vp.numpy().astype(np_dtype)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **out)
    print(f"{name}: T={int(cu[-1])} Hq={Hq} D={D} b={b} max_depth={max_depth}")


def _random_parents(lens, seed):
    """Irregular trees in BFS-compatible order: parent(i) < i, root self-loops."""
    rng = np.random.default_rng(seed)
    out = []
    for n in lens:
        p = np.zeros(n, dtype=np.int32)
        for i in range(1, n):
            p[i] = rng.integers(max(0, i - 6), i)
        out.append(p)
    return np.concatenate(out)


def main():
    def nodes(b, d):
        return d + 1 if b == 1 else (b ** (d + 1) - 1) // (b - 1)

    _case("cfg1", [15, 15], 4, 64, 2, 3, 2 * 10000 + 2 * 100 + 3, dtype=torch.float32)
    _case("chain_b1_d8", [9] * 4, 4, 64, 1, 8, 4 * 10000 + 1 * 100 + 8)
    _case("single_b1_d0", [1] * 4, 4, 64, 1, 0, 4 * 10000 + 1 * 100 + 0)
    _case("b3_d3_D128", [nodes(3, 3)] * 3, 2, 128, 3, 3, 3 * 10000 + 3 * 100 + 3)
    _case("b4_d2_D32", [nodes(4, 2)] * 2, 4, 32, 4, 2, 2 * 10000 + 4 * 100 + 2)
    _case("trunc_b2", [31] * 2, 4, 64, 2, 2, 777)
    _case("ragged", [13, 0, 40, 1, 7], 4, 64, 3, 3, 4242)
    _case("gqa", [nodes(2, 4)] * 2, 8, 64, 2, 4, 9191, Hkv=2)
    lens = [20, 33, 1]
    _case("parents", lens, 4, 64, 1, 7, 5151, parents=_random_parents(lens, 5151))
    _case("prefix", [nodes(2, 3)] * 2, 4, 64, 2, 3, 6161, Hkv=2, prefix=24)


if __name__ == "__main__":
    main()
