"""Benchmark of the tree-verify attention hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config cfg2|cfg3|cfg4|cfg4_prefix|cfg5|gen1024|cfg4_bhnd|cfg2_paged|eagle3|merge4
                    |cfg2_bf16|cfg4_bf16|cfg4_shared|micro28_B1|micro28_B4|micro28_B8|micro28_B8_L4096]
                    [--algo auto|gather|subtree] [--no-extra] [--no-cpu-baseline]
    python bench.py --config cfg4 --eager-calls 4     (counter passes: N eager calls, no graphs)

A step is one full verify-attention call (all sequences, all heads, and the
prefix KV cache when the config has one) over one batch of synthetic input,
what the reference times per call (scripts/benchmark_micro.py:585-609).
Inputs are drawn on the CPU with the reference seed convention
(B*10000 + b*100 + d, set i adds i), copied to HBM before timing, and every
call reads a different input set than the call before it: call k of the run
uses set k mod nsets, with at least 4 sets totalling more than 512 MB (two
sets when one is larger than 512 MB), so MI355X's 256 MB Infinity Cache holds
none of a call's inputs when it starts.  The calls are captured in HIP graphs
(the reference times CUDA-graph replays, scripts/benchmark_micro.py:169-187),
up to 32 consecutive calls per graph (kernels inside a graph run back to
back; each graph launch leaves ~8 µs idle, 0.26 µs per call at 32 calls per
graph); the rotation runs through the graphs.  Before the warmup the
graphs are replayed, untimed, for SETTLE_S seconds so the GPU's clocks reach
their steady state; then exactly W warmup calls and exactly K timed calls,
the timed region bracketed by torch.cuda.synchronize() and HIP events on the
stream the kernels run on.

Prints ONE JSON line with the driver's fields plus
  roofline      tree-only configs: algorithmic bytes (Q+K+V+O) / kernel time
                vs 8 TB/s HBM.  Prefix configs: t_min = max(bytes / 8 TB/s,
                flops / 2.5 PFLOP/s) and frac = t_min / t.
  hbm_ceiling   (tree-only configs) torch.addcmul over rotating sets with the
                workload's bytes (3 reads, 1 write): what a plain streaming
                kernel reaches under the same cache conditions
  extra         (default cfg2 run) cfg3, the cfg4 verify call, the cfg4
                prefix-only call (same queries and prefix, no tree keys) and
                their ratio, cfg5, one EAGLE-3 step and the reference's
                published balanced micro-benchmark shapes, each timed the
                same way
  sched_static_launches  subtree launches of the run that fell back to the
                static schedule for want of a counter slot (expected 0)
  cpu_baseline  the reference's CPU path (padded SDPA + tree mask, fp32, MATH
                backend; restated in oracle/sdpa.py) timed on this host's cores
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "verify-attn µs/call + achieved HBM GB/s, b=4 d=5 N=1365 H=32 D=128 fp16"
PEAK_HBM = 8.0e12     # B/s, MI355X HBM3E (vendor figure)
PEAK_MFMA = 2.5e15    # FLOP/s, MI355X dense fp16 MFMA (vendor figure)
CALLS_PER_GRAPH = 32  # a graph launch leaves ~8 µs between graphs; 32 calls amortise it
SETTLE_S = 0.1        # untimed replays before the warmup steps (clock settling)

# The reference's configs cfg2..cfg5, and the explicit-parents workload of its
# model-generality benchmark (scripts/benchmark_model_generality.py:19-53:
# B=1, heap parents (i-1)//b with the root its own parent, b=10 d=7 capped at
# N=1024 nodes, Llama-3.1-8B heads; results/generality/
# model_generality_benchmark.csv:6 records 113.0 µs on unrecorded hardware)
CONFIGS = {
    "cfg2": dict(B=4, b=4, d=5, H=32, Hkv=32, D=128, L=0, sigma=1.0),
    "cfg3": dict(B=8, b=2, d=9, H=32, Hkv=32, D=128, L=0, sigma=1.0),
    "cfg4": dict(B=4, b=4, d=3, H=32, Hkv=8, D=128, L=10240, sigma=1.0),
    "cfg5": dict(B=16, b=8, d=4, H=32, Hkv=32, D=128, L=2048, sigma=0.5),
    "gen1024": dict(B=1, b=10, d=7, H=32, Hkv=32, D=128, L=0, sigma=1.0, N=1024, walk="parents"),
    # cfg4 as the reference's E2E verify step holds it (scripts/e2e_benchmark.py:
    # 1394-1502): Q [B, H, N, D], K/V [B, Hkv, L + N, D], one ragged_tree_attn call
    "cfg4_bhnd": dict(B=4, b=4, d=3, H=32, Hkv=8, D=128, L=10240, sigma=1.0, layout="bhnd"),
    # cfg2 with K/V in a paged cache of 16-token pages (the reference's page
    # size, src/ragged_attn.py:945) placed in a shuffled physical order
    "cfg2_paged": dict(B=4, b=4, d=5, H=32, Hkv=32, D=128, L=0, sigma=1.0, layout="paged"),
    # one EAGLE-3 verify step of Llama-3.1-8B as the reference's E2E harness
    # runs it (scripts/e2e_benchmark.py:741-744, 875: total_token 60, depth 7,
    # top_k 10; B = 1) over a 2048-token KV cache: [B, H, N, D] tensors, the
    # draft tree as a parent array, one ragged_tree_attn call
    "eagle3": dict(B=1, b=10, d=7, H=32, Hkv=8, D=128, L=2048, sigma=1.0, N=60, walk="eagle",
                   layout="bhnd"),
    # fused_lse_merge (src/ragged_attn.py:1619-1653) at cfg4's verify shape:
    # two [B, H, Nq, D] blocks and their LSEs merged into one output
    "merge4": dict(B=4, b=4, d=3, H=32, Hkv=32, D=128, L=0, sigma=1.0, layout="merge"),
    # cfg4's prefix pass alone (prefix_attention: the same queries and prefix,
    # no tree keys), the denominator of the cfg4 verify/prefix-only ratio
    "cfg4_prefix": dict(B=4, b=4, d=3, H=32, Hkv=8, D=128, L=10240, sigma=1.0, layout="prefix_only"),
    # cfg2 and cfg4 in bfloat16 (the reference takes fp16 or bf16,
    # src/ragged_attn.py:1113-1116)
    "cfg2_bf16": dict(B=4, b=4, d=5, H=32, Hkv=32, D=128, L=0, sigma=1.0, dtype="bf16"),
    "cfg4_bf16": dict(B=4, b=4, d=3, H=32, Hkv=8, D=128, L=10240, sigma=1.0, dtype="bf16"),
    # cfg4 with one prefix shared by the batch ([L, Hkv, D], the first
    # sequence's prefix for all four), as the reference's micro-benchmark
    # shares K_sh/V_sh across its branches (scripts/benchmark_micro.py:318-331)
    "cfg4_shared": dict(B=4, b=4, d=3, H=32, Hkv=8, D=128, L=10240, sigma=1.0, layout="shared_prefix"),
    # The reference's published kernel rows for this path, its balanced
    # micro-benchmark (scripts/benchmark_micro.py --balanced-trees, budgeted
    # N): a b=28 heap tree capped at N=672 nodes (depth 2, max_depth 2),
    # H=32, D=128, fp16, B = 1, 4, 8 (results/balanced_micro/aggregate.csv:
    # 17, 81, 113: 22.3, 272.9, 553.1 us), and B=8 over a 4096-token prefix
    # shared by the batch (:129, 6454.2 us; scripts/benchmark_micro.py:
    # 568-593: shared-prefix pass + tree pass + fused_lse_merge), other hardware
    "micro28_B1": dict(B=1, b=28, d=2, H=32, Hkv=32, D=128, L=0, sigma=1.0, N=672),
    "micro28_B4": dict(B=4, b=28, d=2, H=32, Hkv=32, D=128, L=0, sigma=1.0, N=672),
    "micro28_B8": dict(B=8, b=28, d=2, H=32, Hkv=32, D=128, L=0, sigma=1.0, N=672),
    "micro28_B8_L4096": dict(B=8, b=28, d=2, H=32, Hkv=32, D=128, L=4096, sigma=1.0, N=672,
                             layout="shared_prefix"),
}
# the reference's published time for each micro config (us per call, other hardware)
PUBLISHED_US = {"micro28_B1": 22.3, "micro28_B4": 272.9, "micro28_B8": 553.1, "micro28_B8_L4096": 6454.2}


def torch_dtype(c):
    """The config's element type (fp16 unless it names bf16)."""
    import torch
    return torch.bfloat16 if c.get("dtype") == "bf16" else torch.float16


def num_tree_nodes(b, d):
    return d + 1 if b == 1 else (b ** (d + 1) - 1) // (b - 1)


def tree_size(c):
    """Nodes per sequence: the complete tree, or the config's cap."""
    return c.get("N", num_tree_nodes(c["b"], c["d"]))


def heap_parents(b, n):
    """Sequence-local parent array of a heap-indexed tree, the root its own parent."""
    return [0] + [(i - 1) // b for i in range(1, n)]


def eagle_parents(n, depth):
    """A draft tree of n nodes in BFS order, depth levels below the root,
    levels as even as n allows; node j of a level hangs under node j mod
    (previous level size) of the level above.  The root is its own parent."""
    sizes = [1] + [(n - 1) // depth + (1 if i < (n - 1) % depth else 0) for i in range(depth)]
    par, first = [0], 0
    for lv in range(1, len(sizes)):
        prev = sizes[lv - 1]
        par += [first + j % prev for j in range(sizes[lv])]
        first += prev
    return par


def tree_parents(c):
    """Parent array of one sequence of the config's tree."""
    n = tree_size(c)
    return eagle_parents(n, c["d"]) if c.get("walk") == "eagle" else heap_parents(c["b"], n)


def make_set(c, seed, dtype):
    """Q, tree K, tree V (packed) and prefix K/V [B, L, Hkv, D], drawn in that order."""
    import torch
    N = tree_size(c)
    T = c["B"] * N
    g = torch.Generator().manual_seed(seed)
    s = c["sigma"]
    Q = (torch.randn(T, c["H"], c["D"], generator=g) * s).to(dtype)
    K = (torch.randn(T, c["Hkv"], c["D"], generator=g) * s).to(dtype)
    V = (torch.randn(T, c["Hkv"], c["D"], generator=g) * s).to(dtype)
    Kp = Vp = None
    if c["L"]:
        Kp = (torch.randn(c["B"], c["L"], c["Hkv"], c["D"], generator=g) * s).to(dtype)
        Vp = (torch.randn(c["B"], c["L"], c["Hkv"], c["D"], generator=g) * s).to(dtype)
    return Q, K, V, Kp, Vp


def model_costs(c):
    """Algorithmic HBM bytes and FLOPs of one call."""
    B, b, d, H, Hkv, D, L = (c[k] for k in ("B", "b", "d", "H", "Hkv", "D", "L"))
    N = tree_size(c)
    T = B * N
    if c.get("layout") == "merge":
        # read two O blocks and two fp32 LSEs, write one O; ~6 FLOP per element
        return 3 * 2 * T * H * D + 2 * 4 * T * H, 6 * T * H * D, 0
    tree_bytes = 2 * T * D * (2 * H + 2 * Hkv)          # Q + O at H, tree K + V at Hkv
    prefix_bytes = 2 * 2 * B * L * Hkv * D                 # prefix K + V at Hkv
    if c.get("layout") == "shared_prefix":
        prefix_bytes //= B                                 # one prefix for the batch
    prefix_flops = 4 * B * N * H * L * D
    if c.get("layout") == "prefix_only":
        return 2 * T * D * 2 * H + prefix_bytes, prefix_flops, prefix_flops
    # attended (query, key) pairs per sequence: min(depth, d) + 1 per node
    par = tree_parents(c)
    depth = [0] * N
    for i in range(1, N):
        depth[i] = depth[par[i]] + 1 if (b > 1 or c.get("walk") == "eagle") else i
    steps = sum(min(x, d) + 1 for x in depth)
    tree_flops = 4 * D * H * B * steps
    return tree_bytes + prefix_bytes, tree_flops + prefix_flops, prefix_flops


def measured_traffic(config):
    """HBM bytes per dispatch of the dominant kernel, from the committed counter
    summary profiles/<kernel>_<config>_traffic.md (line 'hbm_bytes_per_dispatch: N'),
    or None when no summary exists for this config."""
    import glob
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", f"*_{config}_traffic.md"))):
        try:
            for line in open(path):
                if line.strip().startswith("hbm_bytes_per_dispatch:"):
                    return int(float(line.split(":", 1)[1].strip().strip("`")))
        except (OSError, ValueError):
            pass
    return None


def copy_calibration(mib):
    """A plain device copy of `mib` MiB (read mib, write mib): the reference
    kernel for scaling FETCH_SIZE / WRITE_SIZE counters to bytes."""
    import torch
    n = mib << 20
    x = torch.empty(n // 2, dtype=torch.float16, device="cuda").normal_()
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "copies": 3}), flush=True)


def cpu_baseline(c, budget_s=12.0):
    """Reference CPU path on a bounded sample: padded SDPA (fp32, MATH) with
    the tree mask (prefix columns all-attend), repeated until ~budget_s."""
    import numpy as np
    import torch
    from oracle import sdpa, tree

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    B, b, d = c["B"], c["b"], c["d"]
    N = tree_size(c)
    Q, K, V, Kp, Vp = make_set(c, B * 10000 + b * 100 + d, torch_dtype(c))
    nseq = B
    if c["L"] and B * N * (N + c["L"]) * c["H"] > 4e9:
        nseq = 1  # sample: one sequence of the batch (the full score tensor would not fit)
    Q, K, V = (t[:nseq * N].float() for t in (Q, K, V))
    if c.get("layout") == "shared_prefix":  # the first sequence's prefix for every sequence
        Kp, Vp = (t[:1].expand(nseq, -1, -1, -1) for t in (Kp, Vp))
    Kp = Kp[:nseq].float() if Kp is not None else None
    Vp = Vp[:nseq].float() if Vp is not None else None
    cu = torch.arange(0, (nseq + 1) * N, N, dtype=torch.int32)
    if c.get("walk") in ("parents", "eagle"):
        # the walk's tree: every node attends its ancestors (the root holds -1 here)
        pa = [-1] + tree_parents(c)[1:]
        m = np.zeros((N, N), dtype=bool)
        for i in range(N):
            for a in tree.ancestors(i, pa):
                m[i, a] = True
        masks = [m] * nseq
    else:
        masks = [tree.tree_attention_mask_n(b, N)] * nseq

    def run():
        sdpa.packed_tree_attention(Q, K, V, cu, masks, Kp=Kp, Vp=Vp)

    t0 = time.perf_counter()
    run()  # warmup
    first = time.perf_counter() - t0
    iters = max(3, min(60, int(budget_s / max(first, 1e-3))))
    times = []
    for _ in range(iters):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times)) * (B / nseq)
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    what = f"{nseq} of {B} sequences, scaled x{B // nseq} to the full batch" if nseq < B else "the full config"
    return {
        "value": round(med * 1e6, 1),
        "unit": "us/call",
        "cores": cores,
        "kind": "port",
        "sample": (f"{what} (B={B} b={b} d={d} N={N} H={c['H']} Hkv={c['Hkv']} D={c['D']} L={c['L']}): "
                   f"padded SDPA fp32 MATH with the ancestor mask (oracle/sdpa.py), median of {iters} calls "
                   f"after 1 warmup; CPU {model}"),
    }


def n_sets(alg_bytes, forced=0):
    """Input sets to rotate: two when one set alone exceeds 512 MB, else at
    least 4 and enough for 600 MB (at most 64)."""
    if forced:
        return forced
    if alg_bytes > 512_000_000:
        return 2
    return min(64, max(4, -(-600_000_000 // alg_bytes)))


def rotation_chunks(start, n):
    """Calls start .. start+n-1 as graphs of up to CALLS_PER_GRAPH consecutive
    calls: a list of (first call, calls); call k reads set k mod nsets."""
    out = []
    while n > 0:
        m = min(CALLS_PER_GRAPH, n)
        out.append((start, m))
        start, n = start + m, n - m
    return out


def time_rotating(call, nsets, steps, warmup):
    """Time `steps` calls, call k reading input set k mod nsets.

    call(i) launches one call on set i on torch's current stream.  Every set
    is run eagerly first (on the current stream and on a side stream, as
    graph capture needs), then the calls are captured in graphs of up to
    CALLS_PER_GRAPH consecutive calls (one graph per distinct run of sets),
    replayed untimed for SETTLE_S seconds, then for exactly `warmup` calls and
    exactly `steps` timed calls that continue the rotation.  Returns
    (µs per call from HIP events on the stream the graphs replay on,
     µs per call of host wall time)."""
    import torch
    for i in range(nsets):
        call(i)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(nsets):
            call(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graphs = {}

    def graph(start, n):
        key = (start % nsets, n)
        if key not in graphs:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for k in range(n):
                    call((start + k) % nsets)
            graphs[key] = g
        return graphs[key]

    def plan(start, n):
        return [graph(s0, m) for s0, m in rotation_chunks(start, n)]

    settle = plan(0, CALLS_PER_GRAPH * nsets)
    warm = plan(0, warmup)
    timed = plan(warmup, steps)
    torch.cuda.synchronize()
    t_settle = time.perf_counter()
    k = 0
    while time.perf_counter() - t_settle < SETTLE_S:
        settle[k % len(settle)].replay()
        k += 1
        if k % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    for g in warm:
        g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for g in timed:
        g.replay()
    ev1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    del graphs, settle, warm, timed
    return ev0.elapsed_time(ev1) * 1e3 / steps, (t1 - t0) / steps * 1e6


def build_workload(name, algo, forced_sets=0):
    """Device input sets of a config and call(i) running one call on set i."""
    import torch
    from qattention_amd import ragged_attn as ra

    c = CONFIGS[name]
    B, b, d, H, Hkv, D, L = (c[k] for k in ("B", "b", "d", "H", "Hkv", "D", "L"))
    N = tree_size(c)
    parents_walk = c.get("walk") in ("parents", "eagle")
    dev = torch.device("cuda:0")
    alg_bytes, _, _ = model_costs(c)
    nsets = n_sets(alg_bytes, forced_sets)
    seed = B * 10000 + b * 100 + d
    layout = c.get("layout")
    sets = []
    for i in range(nsets):
        Q, K, V, Kp, Vp = make_set(c, seed + i, torch_dtype(c))
        if layout == "bhnd":
            # the same values in the E2E layout: prefix rows then tree rows per sequence
            Q = Q.view(B, N, H, D).permute(0, 2, 1, 3).contiguous()
            K = torch.cat([Kp, K.view(B, N, Hkv, D)], 1).permute(0, 2, 1, 3).contiguous()
            V = torch.cat([Vp, V.view(B, N, Hkv, D)], 1).permute(0, 2, 1, 3).contiguous()
            Kp = Vp = None
        if layout == "paged":
            Kc, Vc, pt = ra.build_paged_kv(list(K.view(B, N, Hkv, D)), list(V.view(B, N, Hkv, D)), 16)
            perm = torch.randperm(Kc.shape[0], generator=torch.Generator().manual_seed(seed + i))
            K, V = torch.empty_like(Kc), torch.empty_like(Vc)
            K[perm], V[perm] = Kc, Vc
            Kp = perm.to(torch.int32)[pt.long()]  # the page table rides in the prefix slot
        if layout == "merge":
            # out_pre, out_tree [B, H, Nq, D]; the LSEs ride in the prefix slots
            g = torch.Generator().manual_seed(seed + i)
            Q = Q.view(B, N, H, D).permute(0, 2, 1, 3).contiguous()
            K = K.view(B, N, H, D).permute(0, 2, 1, 3).contiguous()
            Kp = torch.randn(B, H, N, generator=g) * 3
            Vp = torch.randn(B, H, N, generator=g) * 3
        if layout == "prefix_only":
            K = V = None  # no tree keys
        if layout == "shared_prefix":
            Kp, Vp = Kp[0], Vp[0]  # [L, Hkv, D]: sequence stride 0
        sets.append([t.to(dev) if t is not None else None for t in (Q, K, V, Kp, Vp)])
    cu = torch.arange(0, (B + 1) * N, N, dtype=torch.int32, device=dev)
    parents = torch.tensor(tree_parents(c) * B, dtype=torch.int32, device=dev) if parents_walk else None
    torch.cuda.synchronize()

    def call(i):
        Q, K, V, Kp, Vp = sets[i]
        if layout == "bhnd":
            return ra.ragged_tree_attn(Q, K, V, b, d, parents[:N] if parents_walk else None)
        if layout == "paged":
            return ra._paged_forward(Q, K, V, Kp, cu, b, d, N, False, algo)[0]
        if layout == "merge":
            return ra.fused_lse_merge(Kp, Vp, Q, K)
        if layout == "prefix_only":
            return ra.prefix_attention(Q, Kp, Vp, cu, max_seqlen=N)
        if L:
            return ra.ragged_attention_prefix(Q, K, V, cu, Kp, Vp, b, d, max_seqlen=N)
        if parents_walk:
            return ra.ragged_attention_with_parents(Q, K, V, cu, parents, d, max_seqlen=N)[0]
        return ra._tree_forward(Q, K, V, cu, b, d, N, False, algo)[0]

    return call, nsets


def roofline_of(c, t_us):
    alg_bytes, flops, prefix_flops = model_costs(c)
    t_s = t_us * 1e-6
    achieved_bw = alg_bytes / t_s
    if c["L"]:
        t_min = max(alg_bytes / PEAK_HBM, flops / PEAK_MFMA)
        bound = "mfma" if flops / PEAK_MFMA >= alg_bytes / PEAK_HBM else "hbm"
        return {"bound": bound, "achieved": round(flops / t_s / 1e12, 1) if bound == "mfma"
                else round(achieved_bw / 1e9, 1),
                "peak": PEAK_MFMA / 1e12 if bound == "mfma" else PEAK_HBM / 1e9,
                "unit": "TFLOP/s" if bound == "mfma" else "GB/s",
                "frac": round(t_min / t_s, 4), "t_min_us": round(t_min * 1e6, 2),
                "hbm_frac": round(achieved_bw / PEAK_HBM, 4),
                "mfma_frac": round(flops / t_s / PEAK_MFMA, 4)}
    return {"bound": "hbm", "achieved": round(achieved_bw / 1e9, 1), "peak": PEAK_HBM / 1e9,
            "unit": "GB/s", "frac": round(achieved_bw / PEAK_HBM, 4)}


def hbm_ceiling(alg_bytes, steps, warmup):
    """torch.addcmul(a, b, c) -> o over rotating sets, 4 tensors of alg_bytes/4
    each (3 reads, 1 write, the tree workloads' Q+K+V read and O write):
    a plain streaming kernel's rate under the same cache conditions."""
    import torch
    n = alg_bytes // 4 // 2
    nsets = n_sets(alg_bytes)
    dev = torch.device("cuda:0")
    sets = [[torch.empty(n, dtype=torch.float16, device=dev).normal_() for _ in range(4)] for _ in range(nsets)]

    def call(i):
        a, b, c, o = sets[i]
        torch.addcmul(a, b, c, out=o)

    us, _ = time_rotating(call, nsets, steps, warmup)
    del sets
    torch.cuda.empty_cache()
    return {"kernel": "torch.addcmul fp16, 3 reads + 1 write of the workload's bytes, rotating sets",
            "us": round(us, 2), "GBps": round(alg_bytes / us / 1e3, 1),
            "frac": round(alg_bytes / (us * 1e-6) / PEAK_HBM, 4)}


def eager_calls(name, algo, n, forced_sets=0):
    """n eager calls of a config on rotating input sets (call k reads set k
    mod nsets, as in the timed runs), synchronised at the end: the workload a
    rocprofv3 --pmc counter pass collects from, one dispatch group per call."""
    import torch
    call, nsets = build_workload(name, algo, forced_sets)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(n):
        call(k % nsets)
    torch.cuda.synchronize()
    print(json.dumps({"eager_calls": n, "config": name, "sets": nsets,
                      "wall_us_per_call": round((time.perf_counter() - t0) / n * 1e6, 2)}), flush=True)


def measure(name, algo, steps, warmup, forced_sets=0):
    """(µs per call from events, µs per call of wall time, input sets)."""
    import torch
    call, nsets = build_workload(name, algo, forced_sets)
    us, wall = time_rotating(call, nsets, steps, warmup)
    del call
    torch.cuda.empty_cache()
    return us, wall, nsets


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--config", default="cfg2", choices=sorted(CONFIGS))
    ap.add_argument("--algo", default="auto", choices=["auto", "gather", "subtree"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="cfg2 only: skip the extra timings (cfg3, cfg4 verify / prefix-only, the EAGLE-3 "
                         "step, cfg5, the reference's published micro shapes, HBM ceiling)")
    ap.add_argument("--sets", type=int, default=0, help="rotating input sets (0: see n_sets)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain MIB-MiB device copy (counter calibration) and exit")
    ap.add_argument("--eager-calls", type=int, default=0, metavar="N",
                    help="only run N eager calls of --config on rotating input sets (no graphs, no "
                         "timing) and exit: the workload of a rocprofv3 --pmc counter pass")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the tree path shards over sequences/heads with no exchange between GPUs", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        print("bench.py: --steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        sys.exit(2)

    import torch
    from qattention_amd import _lib

    torch.cuda.set_device(torch.device("cuda:0"))
    algo = {"auto": _lib.ALGO_AUTO, "gather": _lib.ALGO_GATHER, "subtree": _lib.ALGO_SUBTREE}[args.algo]
    if args.eager_calls:
        eager_calls(args.config, algo, args.eager_calls, args.sets)
        return
    c = CONFIGS[args.config]
    B, b, d, H, Hkv, D, L = (c[k] for k in ("B", "b", "d", "H", "Hkv", "D", "L"))
    N = tree_size(c)
    T = B * N
    layout = c.get("layout")
    parents_walk = c.get("walk") in ("parents", "eagle")
    alg_bytes, flops, _ = model_costs(c)

    event_us, wall_us, nsets = measure(args.config, algo, args.steps, args.warmup, args.sets)
    roofline = roofline_of(c, event_us)
    roofline.update({"traffic": measured_traffic(args.config), "algorithmic_bytes": alg_bytes, "flops": flops})

    extra = None
    ceiling = None
    if not L and layout != "merge":
        ceiling = hbm_ceiling(alg_bytes, args.steps, args.warmup)
    if args.config == "cfg2" and not args.no_extra:
        extra = {}
        us3, _, _ = measure("cfg3", algo, args.steps, args.warmup)
        extra.update({"cfg3_us": round(us3, 2), "cfg3_hbm_frac": roofline_of(CONFIGS["cfg3"], us3)["frac"]})
        us4, _, _ = measure("cfg4", _lib.ALGO_AUTO, args.steps, args.warmup)
        us4p, _, _ = measure("cfg4_prefix", _lib.ALGO_AUTO, args.steps, args.warmup)
        extra.update({"cfg4_verify_us": round(us4, 2), "cfg4_prefix_only_us": round(us4p, 2),
                      "cfg4_ratio": round(us4 / us4p, 3),
                      "cfg4_frac": roofline_of(CONFIGS["cfg4"], us4)["frac"],
                      "cfg4_prefix_only_frac": roofline_of(CONFIGS["cfg4_prefix"], us4p)["frac"]})
        # one EAGLE-3 verify step (latency-bound: a decode step of a small draft tree)
        use3, _, _ = measure("eagle3", _lib.ALGO_AUTO, args.steps, args.warmup)
        extra.update({"eagle3_us": round(use3, 2)})
        # cfg5: the MFMA prefix (L=2048) and a 74,896-token tree walk in one call
        us5, _, _ = measure("cfg5", _lib.ALGO_AUTO, args.steps, args.warmup)
        r5 = roofline_of(CONFIGS["cfg5"], us5)
        extra.update({"cfg5_us": round(us5, 2), "cfg5_frac": r5["frac"], "cfg5_mfma_frac": r5["mfma_frac"],
                      "cfg5_hbm_frac": r5["hbm_frac"]})
        # the reference's published balanced micro-benchmark rows (other hardware)
        micro = {}
        for name in ("micro28_B1", "micro28_B4", "micro28_B8", "micro28_B8_L4096"):
            usm, _, _ = measure(name, _lib.ALGO_AUTO, args.steps, args.warmup)
            micro[name] = {"us": round(usm, 2), "frac": roofline_of(CONFIGS[name], usm)["frac"],
                           "reference_us": PUBLISHED_US[name]}
        extra["micro28"] = micro

    cpu = None
    if not args.no_cpu_baseline and layout not in ("merge", "prefix_only"):
        # (the merge and the prefix pass alone have no padded-SDPA tree counterpart)
        cpu = cpu_baseline(c)

    achieved_bw = alg_bytes / (event_us * 1e-6)
    out = {
        "metric": METRIC,
        "value": round(event_us, 2),
        "unit": "us/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_s": SETTLE_S,
        "ms_per_step": round(wall_us / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": c.get("dtype", "f16"),
        "data": (f"synthetic N(0,{c['sigma']}^2), CPU-seeded (seed B*10000+b*100+d + set), {nsets} input sets "
                 "rotated call by call"),
        "config": {"workload": f"{args.config}: verify attention B={B} b={b} d={d} N={N} H={H} Hkv={Hkv} "
                               f"D={D} L={L} {c.get('dtype', 'fp16')}" + (", explicit parents" if parents_walk else "")
                               + (", [B, H, N, D] views" if layout == "bhnd" else "")
                               + (", paged K/V (16-token pages, shuffled)" if layout == "paged" else "")
                               + (", fused_lse_merge of two [B, H, Nq, D] blocks" if layout == "merge" else "")
                               + (", prefix pass only (no tree keys)" if layout == "prefix_only" else ""),
                   "B": B, "b": b, "d": d, "N": N, "H": H, "Hkv": Hkv,
                   "D": D, "L": L, "tokens": T, "algo": args.algo},
        "achieved_GBps": round(achieved_bw / 1e9, 1),
        "wall_us_per_call": round(wall_us, 2),
        "roofline": roofline,
        "hbm_ceiling": ceiling,
        "extra": extra,
        "cpu_baseline": cpu,
        "sched_static_launches": _lib.sched_info()["static_launches"],
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
