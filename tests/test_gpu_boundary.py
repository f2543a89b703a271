"""GPU checks of the C-ABI contract around the kernels: the prefix-only pass
(prefix_attention / qattn_prefix_fwd) against the oracle and composed into
the reference's three-step verify pipeline; any finite scale through both
tree kernels; and schedule-counter slots that never serve two launches that
may overlap (many streams at once, more streams than slots).

Tolerances: fp16 max |o - o_ref| <= 2e-3 plus allclose(atol=rtol=1e-2);
bf16 2^-7 max(1, |o_ref|) + 1e-3 (the prefix path rounds P to bf16, as the
reference hybrid kernel does, src/ragged_attn.py:1797); LSE 1e-4 (fp16) /
2e-3 (bf16).  Stream and graph checks are bit-exact against a solo run.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import make_inputs, num_tree_nodes, oracle_tree, tree_case
from oracle import clib

pytestmark = pytest.mark.gpu

DEV = "cuda"


def say(*a):
    print(*a, flush=True)


def _ra():
    from qattention_amd import _lib, ragged_attn
    return ragged_attn, _lib


def check_fp16(o, o_ref, what=""):
    err = float(np.abs(o - o_ref).max()) if o.size else 0.0
    assert err <= 2e-3, f"{what}: max abs err {err:.3e}"
    assert np.allclose(o, o_ref, atol=1e-2, rtol=1e-2), what


def check_bf16(o, o_ref, what=""):
    bound = 2.0 ** -7 * np.maximum(1.0, np.abs(o_ref)) + 1e-3
    err = np.abs(o - o_ref)
    assert (err <= bound).all(), f"{what}: bf16 err {err.max():.3e}"


def _prefix(B, L, Hkv, D, seed, dtype=torch.float16, sigma=1.0):
    g = torch.Generator().manual_seed(seed)
    Kp = (torch.randn(B, L, Hkv, D, generator=g) * sigma).to(dtype)
    Vp = (torch.randn(B, L, Hkv, D, generator=g) * sigma).to(dtype)
    return Kp, Vp


def _prefix_oracle(Q, cu, Kp, Vp):
    """Prefix-only attention: the oracle with no tree ancestor attended."""
    T, Hq, D = Q.shape
    Hkv = Kp.shape[2]
    anc = np.full((T, 1), -1, dtype=np.int32)
    zk = np.zeros((T, Hkv, D), dtype=np.float32)
    return clib.tree_attn(Q.float().numpy(), zk, zk, cu.numpy(), anc, 1.0 / math.sqrt(D),
                          Kp.float().numpy(), Vp.float().numpy())


# ---------------------------------------------------------------------------
# prefix-only pass
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("lens,Hq,Hkv,D,L,ns,dtype", [
    ([85, 85, 85, 85], 32, 8, 128, 2000, 0, torch.float16),   # cfg4-like, automatic (several) splits
    ([85, 85], 32, 8, 128, 700, 1, torch.float16),            # one split: normalised in the prefix kernel
    ([40, 1, 13], 6, 3, 64, 333, 3, torch.float16),           # ragged, forced splits + merge kernel
    ([31, 7], 4, 1, 32, 130, 0, torch.float16),
    ([63], 2, 2, 128, 1, 0, torch.float16),                   # a one-row prefix
    ([85, 40], 8, 2, 128, 500, 0, torch.bfloat16),
    ([85, 40], 8, 2, 128, 500, 1, torch.bfloat16),
])
def test_prefix_attention_oracle(lens, Hq, Hkv, D, L, ns, dtype):
    ra, _ = _ra()
    say("prefix only", lens, Hq, Hkv, D, L, ns, dtype)
    Q, _, _, cu = make_inputs(lens, Hq, D, 8100 + L, dtype=dtype, Hkv=Hkv)
    Kp, Vp = _prefix(len(lens), L, Hkv, D, 8101 + L, dtype=dtype)
    O, LSE = ra.prefix_attention(Q.to(DEV), Kp.to(DEV), Vp.to(DEV), cu, num_splits=ns)
    o_ref, lse_ref = _prefix_oracle(Q, cu, Kp, Vp)
    o = O.double().cpu().numpy()
    if dtype == torch.float16:
        check_fp16(o, o_ref, "prefix only")
        assert np.abs(LSE.double().cpu().numpy() - lse_ref).max() <= 1e-4
    else:
        check_bf16(o, o_ref, "prefix only bf16")
        assert np.abs(LSE.double().cpu().numpy() - lse_ref).max() <= 2e-3


def test_prefix_attention_shared_prefix():
    """The reference benchmark's prefix pass: every query of the batch attends
    one shared prefix [L, H, D] (flashinfer single_prefill over Q [B*N, H, D],
    scripts/benchmark_micro.py:574-580), cu_seqlens None."""
    ra, _ = _ra()
    T, H, D, L = 4 * 85, 8, 128, 1024
    Q, _, _, _ = make_inputs([T], H, D, 8200)
    Kp, Vp = _prefix(1, L, H, D, 8201)
    O, LSE = ra.prefix_attention(Q.to(DEV), Kp[0].to(DEV), Vp[0].to(DEV))
    o_ref, lse_ref = _prefix_oracle(Q, torch.tensor([0, T], dtype=torch.int32), Kp, Vp)
    check_fp16(O.double().cpu().numpy(), o_ref, "shared prefix")
    assert np.abs(LSE.double().cpu().numpy() - lse_ref).max() <= 1e-4


def test_prefix_attention_shared_prefix_graph_capture():
    """The shared-prefix call (cu_seqlens None) records into a HIP graph: no
    host copy inside the call.  A fresh query length (no cached cu) is
    captured first, then replayed several times with eager calls and
    synchronisations in between; every replay bit-equals the eager call."""
    ra, _ = _ra()
    T, H, D, L = 3 * 85 + 7, 8, 128, 1000
    Q, _, _, _ = make_inputs([T], H, D, 8210)
    Kp, Vp = _prefix(1, L, H, D, 8211)
    Qd, Kd, Vd = Q.to(DEV), Kp[0].to(DEV), Vp[0].to(DEV)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        Og, LSEg = ra.prefix_attention(Qd, Kd, Vd)
    O, LSE = ra.prefix_attention(Qd, Kd, Vd)
    torch.cuda.synchronize()
    for rep in range(3):
        Og.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(Og, O) and torch.equal(LSEg, LSE), f"replay {rep}"
        ra.prefix_attention(Qd, Kd, Vd)
    o_ref, _ = _prefix_oracle(Q, torch.tensor([0, T], dtype=torch.int32), Kp, Vp)
    check_fp16(O.double().cpu().numpy(), o_ref, "shared prefix, captured")


@pytest.mark.parametrize("ns", [0, 1])
def test_reference_pipeline_equals_verify(ns):
    """The reference's verify pipeline (scripts/benchmark_micro.py:568-593):
    prefix pass with LSE + ragged_attention_with_lse + fused_lse_merge, all on
    the GPU, equals the one-call verify (ragged_attention_prefix) -- the FA2
    merge identity -- and both equal the oracle."""
    ra, _ = _ra()
    B, b, d, H, D, L = 2, 4, 3, 8, 128, 640
    N = num_tree_nodes(b, d)
    say("pipeline", ns)
    Q, K, V, cu = tree_case(B, b, d, H, D)
    Kp, Vp = _prefix(B, L, H, D, 12)
    Qd, Kd, Vd, Kpd, Vpd = Q.to(DEV), K.to(DEV), V.to(DEV), Kp.to(DEV), Vp.to(DEV)
    fused = ra.ragged_attention_prefix(Qd, Kd, Vd, cu, Kpd, Vpd, b, d, num_splits=ns)
    o_p, lse_p = ra.prefix_attention(Qd, Kpd, Vpd, cu, num_splits=ns)
    o_t, lse_t = ra.ragged_attention_with_lse(Qd, Kd, Vd, cu, b, d)
    to_bhn = lambda x: x.view(B, N, H, -1).permute(0, 2, 1, 3)
    merged = ra.fused_lse_merge(lse_p.view(B, N, H).permute(0, 2, 1), lse_t.view(B, N, H).permute(0, 2, 1),
                                to_bhn(o_p), to_bhn(o_t))
    merged = merged.permute(0, 2, 1, 3).reshape(B * N, H, D)
    o_ref, _, _ = oracle_tree(Q, K, V, cu, b, d, Kp=Kp, Vp=Vp)
    check_fp16(fused.double().cpu().numpy(), o_ref, "one-call verify")
    # the pipeline rounds O_pre and O_tree to fp16 before merging: one more rounding
    assert float((fused.float() - merged.float()).abs().max()) <= 4e-3


# ---------------------------------------------------------------------------
# any finite scale, both tree kernels
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("scale", [0.0, -0.1, -1.0 / math.sqrt(128), 0.5])
def test_tree_scale_any_sign(scale):
    """qattn_tree_fwd with scale <= 0: the subtree kernel masks and takes its
    running max after scaling, so it agrees with the gather kernel and the
    oracle (scale 0 is a plain average over the ancestors)."""
    ra, _lib = _ra()
    B, b, d, H, D = 4, 4, 5, 8, 128
    say("scale", scale)
    Q, K, V, cu = tree_case(B, b, d, H, D)
    T = Q.shape[0]
    anc = clib.ancestor_table_heap(cu.numpy(), b, d)
    o_ref, lse_ref = clib.tree_attn(Q.float().numpy(), K.float().numpy(), V.float().numpy(), cu.numpy(), anc,
                                    scale)
    L = _lib.lib()
    Qd, Kd, Vd, cud = Q.to(DEV), K.to(DEV), V.to(DEV), cu.to(DEV)
    for algo in (_lib.ALGO_GATHER, _lib.ALGO_SUBTREE):
        O = torch.empty_like(Qd)
        LSE = torch.empty(T, H, dtype=torch.float32, device=DEV)
        st = _lib.i64arr(Qd.stride())
        rc = L.qattn_tree_fwd(Qd.data_ptr(), st, Kd.data_ptr(), st, Vd.data_ptr(), st, O.data_ptr(), st,
                              LSE.data_ptr(), _lib.i64arr(LSE.stride()), cud.data_ptr(), B,
                              num_tree_nodes(b, d), T, H, H, D, b, d, scale, _lib.DTYPE_F16, algo,
                              torch.cuda.current_stream().cuda_stream)
        _lib.check(rc, "qattn_tree_fwd")
        torch.cuda.synchronize()
        check_fp16(O.double().cpu().numpy(), o_ref, f"scale={scale} algo={algo}")
        assert np.abs(LSE.double().cpu().numpy() - lse_ref).max() <= 1e-4, f"LSE scale={scale} algo={algo}"


# ---------------------------------------------------------------------------
# schedule-counter slots
# ---------------------------------------------------------------------------

def _hip_runtime():
    """The HIP runtime torch has loaded (ctypes handle of the same mapping)."""
    import ctypes
    import os
    maps = open(f"/proc/{os.getpid()}/maps").read()
    paths = {l.split()[-1] for l in maps.splitlines() if "libamdhip64" in l}
    assert len(paths) == 1, paths
    hip = ctypes.CDLL(paths.pop())
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    return hip


def test_many_streams_match_solo():
    """Subtree-kernel launches (cfg2 shape: more tiles than workgroups, so
    the counters are used) queued on 72 distinct HIP streams at once (made
    with hipStreamCreate: torch's own stream pool hands out at most 32
    handles) -- more than the 64 stream slots, so the last ones run the
    static schedule, which qattn_sched_info must count -- with several
    launches queued on the first stream before the others start, each
    bit-equal to a solo run of its inputs."""
    import ctypes
    ra, _lib = _ra()
    B, b, d, H, D = 4, 4, 5, 32, 128
    N = num_tree_nodes(b, d)
    nstreams, nsets = 72, 3
    say("streams", nstreams)
    sets = []
    for i in range(nsets):
        Q, K, V, cu = tree_case(B, b, d, H, D, seed=9000 + i)
        sets.append((Q.to(DEV), K.to(DEV), V.to(DEV), cu.to(DEV)))
    solo = [ra._tree_forward(*s, b, d, N, False, _lib.ALGO_SUBTREE)[0] for s in sets]
    torch.cuda.synchronize()
    hip = _hip_runtime()
    handles = []
    for _ in range(nstreams):
        h = ctypes.c_void_p()
        assert hip.hipStreamCreate(ctypes.byref(h)) == 0
        handles.append(h.value)
    assert len(set(handles)) == nstreams
    before = _lib.sched_info()
    try:
        outs = []
        for i, h in enumerate(handles):
            s = torch.cuda.ExternalStream(h)
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                reps = 6 if i == 0 else 1
                for r in range(reps):
                    k = (i + r) % nsets
                    outs.append((k, ra._tree_forward(*sets[k], b, d, N, False, _lib.ALGO_SUBTREE)[0]))
        torch.cuda.synchronize()
        for k, o in outs:
            assert torch.equal(o, solo[k]), f"set {k}"
        after = _lib.sched_info()
        say("sched_info", before, after)
        assert after["stream_slots"] == after["stream_capacity"] == 64
        # at least the streams beyond the 64 slots ran the static schedule
        assert after["static_launches"] - before["static_launches"] >= nstreams - 64
    finally:
        torch.cuda.synchronize()
        for h in handles:
            hip.hipStreamDestroy(h)


def test_graph_slots_per_capture_and_released():
    """Launches recorded into graphs share one counter slot per capture: 10
    graphs of 30 subtree launches (300 recorded launches, past the 192
    captured slots the library holds) all run with counters, every replay
    bit-equal to solo runs; destroying the graphs hands their slots back, so
    200 more graphs captured and destroyed one after another still get
    counters."""
    import gc
    import time
    ra, _lib = _ra()
    B, b, d, H, D = 4, 4, 5, 8, 128
    N = num_tree_nodes(b, d)
    ngraphs, per_graph, nsets = 10, 30, 3
    say("graph slots", ngraphs, per_graph)
    sets = []
    for i in range(nsets):
        Q, K, V, cu = tree_case(B, b, d, H, D, seed=9300 + i)
        sets.append((Q.to(DEV), K.to(DEV), V.to(DEV), cu.to(DEV)))
    solo = [ra._tree_forward(*s, b, d, N, False, _lib.ALGO_SUBTREE)[0].clone() for s in sets]
    torch.cuda.synchronize()
    before = _lib.sched_info()
    graphs, outs = [], []
    for gi in range(ngraphs):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            og = [ra._tree_forward(*sets[(gi + r) % nsets], b, d, N, False, _lib.ALGO_SUBTREE)[0]
                  for r in range(per_graph)]
        graphs.append(g)
        outs.append(og)
    mid = _lib.sched_info()
    say("sched_info", before, mid)
    assert mid["static_launches"] == before["static_launches"]
    assert mid["dynamic_launches"] - before["dynamic_launches"] == ngraphs * per_graph
    assert mid["capture_slots"] - before["capture_slots"] == ngraphs
    for rep in range(3):
        for g in graphs:
            g.replay()
        torch.cuda.synchronize()
        for gi, og in enumerate(outs):
            for r, o in enumerate(og):
                assert torch.equal(o, solo[(gi + r) % nsets]), f"replay {rep} graph {gi} launch {r}"
    del graphs, outs, og, g
    gc.collect()
    torch.cuda.synchronize()

    def held():
        return _lib.sched_info()["capture_slots"]

    t0 = time.time()
    while held() > before["capture_slots"] and time.time() - t0 < 5.0:
        time.sleep(0.01)
    assert held() == before["capture_slots"], _lib.sched_info()
    # churn: more captures than slots, each graph destroyed after one replay
    for gi in range(200):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            o = ra._tree_forward(*sets[gi % nsets], b, d, N, False, _lib.ALGO_SUBTREE)[0]
        g.replay()
        torch.cuda.synchronize()
        if gi % 50 == 0:
            assert torch.equal(o, solo[gi % nsets]), f"churn graph {gi}"
        del g, o
        gc.collect()
    torch.cuda.synchronize()
    end = _lib.sched_info()
    say("sched_info after churn", end)
    assert end["static_launches"] == before["static_launches"]


def test_graph_replays_and_eager_launches_interleaved():
    """A captured subtree launch (its own slot) replayed on one stream while
    eager launches of other inputs run on another: every result bit-equals a
    solo run."""
    ra, _lib = _ra()
    B, b, d, H, D = 4, 4, 5, 32, 128
    N = num_tree_nodes(b, d)
    say("graph + eager")
    sets = []
    for i in range(2):
        Q, K, V, cu = tree_case(B, b, d, H, D, seed=9100 + i)
        sets.append((Q.to(DEV), K.to(DEV), V.to(DEV), cu.to(DEV)))
    solo = [ra._tree_forward(*s, b, d, N, False, _lib.ALGO_SUBTREE)[0].clone() for s in sets]
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s1):
        ra._tree_forward(*sets[0], b, d, N, False, _lib.ALGO_SUBTREE)
    torch.cuda.current_stream().wait_stream(s1)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        og = ra._tree_forward(*sets[0], b, d, N, False, _lib.ALGO_SUBTREE)[0]
    eager = []
    for rep in range(4):
        s1.wait_stream(torch.cuda.current_stream())
        s2.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s1):
            graph.replay()
        with torch.cuda.stream(s2):
            eager.append(ra._tree_forward(*sets[1], b, d, N, False, _lib.ALGO_SUBTREE)[0])
        torch.cuda.current_stream().wait_stream(s1)
        torch.cuda.current_stream().wait_stream(s2)
        torch.cuda.synchronize()
        assert torch.equal(og, solo[0]), f"replay {rep}"
    for o in eager:
        assert torch.equal(o, solo[1])
