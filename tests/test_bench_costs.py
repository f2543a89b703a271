"""Host checks of bench.py: the algorithmic bytes and FLOPs every roofline
figure is computed from, against independent arithmetic for each config
(compulsory Q+K+V+O bytes at the head counts; FLOPs from the mean ancestor
chain of the heap walk), and the single-GPU contract."""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

from conftest import ROOT

sys.path.insert(0, ROOT)
import bench  # noqa: E402


def _chain_sum(b, d, n):
    """Attended (query, key) pairs of one heap-indexed sequence of n nodes:
    every node attends itself and its ancestors up to d steps."""
    total = 0
    for i in range(n):
        depth, x = 0, i
        while x > 0:
            x = (x - 1) // b
            depth += 1
        total += min(depth, d) + 1
    return total


@pytest.mark.parametrize("name,bytes_,mean_chain", [
    ("cfg2", 178_913_280, 5.668),   # 4 * T*H*D*2 with T = 5460, H = 32, D = 128
    ("cfg3", 268_173_312, 9.010),   # T = 8184
    ("gen1024", 33_554_432, None),  # B = 1, N = 1024
])
def test_tree_configs(name, bytes_, mean_chain):
    c = bench.CONFIGS[name]
    alg_bytes, flops, prefix_flops = bench.model_costs(c)
    assert alg_bytes == bytes_ and prefix_flops == 0
    N = bench.tree_size(c)
    pairs = _chain_sum(c["b"], c["d"], N)
    assert flops == 4 * c["D"] * c["H"] * c["B"] * pairs
    if mean_chain is not None:
        assert abs(pairs / N - mean_chain) < 5e-4


def test_prefix_configs():
    # cfg4: GQA-native bytes (prefix K/V at Hkv = 8) and the prefix FLOPs
    alg_bytes, flops, prefix_flops = bench.model_costs(bench.CONFIGS["cfg4"])
    assert alg_bytes == 174_735_360
    assert prefix_flops == 4 * 4 * 85 * 32 * 10240 * 128 == 57_042_534_400
    assert flops - prefix_flops == 4 * 128 * 32 * 4 * _chain_sum(4, 3, 85)
    # cfg5: tree Q+K+V+O 2454.2 MB + prefix K/V 536.9 MB
    alg_bytes, flops, prefix_flops = bench.model_costs(bench.CONFIGS["cfg5"])
    assert alg_bytes == 2_454_192_128 + 536_870_912
    assert prefix_flops == 4 * 16 * 4681 * 32 * 2048 * 128
    # eagle3: a 60-node draft tree of depth 7 (levels as even as 59 nodes
    # allow: 9, 9, 9, 8, 8, 8, 8) over a 2048-token cache at Hkv = 8
    par = bench.eagle_parents(60, 7)
    depth = [0] * 60
    for i in range(1, 60):
        assert par[i] < i
        depth[i] = depth[par[i]] + 1
    assert max(depth) == 7 and [depth.count(k) for k in range(8)] == [1, 9, 9, 9, 8, 8, 8, 8]
    alg_bytes, flops, prefix_flops = bench.model_costs(bench.CONFIGS["eagle3"])
    assert alg_bytes == 2 * 60 * 128 * (2 * 32 + 2 * 8) + 2 * 2 * 2048 * 8 * 128 == 9_617_408
    assert prefix_flops == 4 * 60 * 32 * 2048 * 128
    assert flops - prefix_flops == 4 * 128 * 32 * sum(x + 1 for x in depth)
    # merge4: two O blocks + two fp32 LSEs read, one O written
    T = 4 * 85
    assert bench.model_costs(bench.CONFIGS["merge4"])[0] == 3 * 2 * T * 32 * 128 + 2 * 4 * T * 32
    # the same workload in other layouts costs the same
    assert bench.model_costs(bench.CONFIGS["cfg4_bhnd"]) == bench.model_costs(bench.CONFIGS["cfg4"])
    assert bench.model_costs(bench.CONFIGS["cfg2_paged"]) == bench.model_costs(bench.CONFIGS["cfg2"])
    # bf16 moves the same number of 2-byte elements
    assert bench.model_costs(bench.CONFIGS["cfg2_bf16"]) == bench.model_costs(bench.CONFIGS["cfg2"])
    assert bench.model_costs(bench.CONFIGS["cfg4_bf16"]) == bench.model_costs(bench.CONFIGS["cfg4"])


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stdout + r.stderr


def test_prefix_only_costs():
    """cfg4's prefix pass alone: Q + O at Hq and the prefix K/V at Hkv; the
    prefix FLOPs of the verify call."""
    c = bench.CONFIGS["cfg4_prefix"]
    alg_bytes, flops, prefix_flops = bench.model_costs(c)
    T = 4 * 85
    assert alg_bytes == 2 * T * 128 * 2 * 32 + 2 * 2 * 4 * 10240 * 8 * 128
    assert flops == prefix_flops == 4 * 4 * 85 * 32 * 10240 * 128
    assert prefix_flops == bench.model_costs(bench.CONFIGS["cfg4"])[2]


@pytest.mark.parametrize("name", sorted(bench.CONFIGS))
def test_rotation_defeats_the_infinity_cache(name):
    """Every config rotates enough input sets that a set comes back only after
    more than 256 MB of other sets (or one set exceeds it), at least 4 sets
    below 512 MB per set, and the graphs' calls cover the run in order with
    no call reading the set of the call before it."""
    alg_bytes = bench.model_costs(bench.CONFIGS[name])[0]
    n = bench.n_sets(alg_bytes)
    assert n >= 2
    if alg_bytes <= 512_000_000:
        assert n >= 4 and (n * alg_bytes > 512_000_000 or n == 64)
    assert (n - 1) * alg_bytes > 256_000_000 or n == 64
    for start, steps in ((0, 20), (5, 20), (3, 1), (0, 8), (16, 200)):
        chunks = bench.rotation_chunks(start, steps)
        calls = [s0 + k for s0, m in chunks for k in range(m)]
        assert calls == list(range(start, start + steps))
        assert all(m <= bench.CALLS_PER_GRAPH for _, m in chunks)
        sets = [k % n for k in calls]
        assert all(a != b for a, b in zip(sets, sets[1:]))
    # a prefix shared by the batch is read once: cfg4's bytes less 3 of its 4
    # prefixes (K + V, 10240 x 8 x 128 fp16 each), the same FLOPs
    b4, f4, p4 = bench.model_costs(bench.CONFIGS["cfg4"])
    bs, fs, ps = bench.model_costs(bench.CONFIGS["cfg4_shared"])
    assert (bs, fs, ps) == (b4 - 3 * 2 * 2 * 10240 * 8 * 128, f4, p4)
    assert bs == 48_906_240
