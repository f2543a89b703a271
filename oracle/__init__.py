"""CPU oracle for ancestor-sparse tree-verify attention.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this package, and only as the checker or the
reported CPU baseline -- never as the thing measured or shipped.  The product
path (qattention_amd/, src/) must not import it.

Contents
--------
tree.py  complete-tree helpers restated from the reference's src/tree_mask.py
         (num_tree_nodes, build_tree, ancestors, tree_attention_mask,
         tree_attention_mask_n, verify_tree_mask) plus walk-derived masks.
sdpa.py  the reference's own oracle: padded SDPA (MATH backend, fp32) with an
         additive tree-mask bias (tests/test_correctness.py:50-124), its
         prefix variant (:444-469), GQA by repeat-interleave, LSE and merge.
clib.py  ctypes binding of qattn_oracle.c: exact integer ancestor tables and a
         double-precision sparse ancestor walk (src/ragged_attn.py:262-497).

Pinning status (each function's checks are in tests/test_oracle.py):
  ancestor tables (heap, parents)   pinned: closed form + build_tree KAT +
                                     mask invariants + dense-mask agreement
  tree masks                        pinned: KAT b=2 d=2, invariants of
                                     verify_tree_mask, walk agreement
  sparse attention (C, fp64)        pinned: agreement with padded SDPA (MATH),
                                     b=1 == causal SDPA, d=0 == V, brute force
  padded SDPA oracle                pinned: library routine + brute force
  LSE                               pinned: torch.logsumexp over masked scores
  LSE merge                         pinned: FA2 identity (merge of two disjoint
                                     key sets == softmax over their union)
  prefix (hybrid) oracle            pinned: all-attend prefix == SDPA with
                                     prefix columns unmasked; L=0 == tree-only
  GQA                               pinned: Hkv == Hq reduces to the reference;
                                     repeat_interleave equivalence
  paged layout                      pinned: gather through the page table ==
                                     dense rows (build_paged_kv restatement)
"""
