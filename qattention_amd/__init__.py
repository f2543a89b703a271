"""qattention_amd -- MI355X-native ancestor-sparse tree-verify attention.

Public API mirrors the reference module src.ragged_attn (saifmb0/QAttention):
see qattention_amd.ragged_attn.  Kernels are hand-written gfx950 HIP in
csrc/, exposed through the C ABI of include/qattn.h (libqattn.so).
"""
from .ragged_attn import (  # noqa: F401
    ancestor_table,
    build_paged_kv,
    fused_lse_merge,
    pack_inputs,
    ragged_attention,
    ragged_attention_hybrid,
    ragged_attention_paged,
    ragged_attention_prefix,
    ragged_attention_sibling,
    ragged_attention_sibling_with_lse,
    ragged_attention_with_lse,
    ragged_attention_with_parents,
    set_layout_copies,
)

__version__ = "0.1.0"
