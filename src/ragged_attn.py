"""`src.ragged_attn` drop-in: re-exports qattention_amd.ragged_attn."""
from qattention_amd.ragged_attn import *  # noqa: F401,F403
from qattention_amd.ragged_attn import (  # noqa: F401
    ancestor_table,
    build_paged_kv,
    fused_lse_merge,
    pack_inputs,
    prefix_attention,
    ragged_attention,
    ragged_attention_hybrid,
    ragged_attention_paged,
    ragged_attention_prefix,
    ragged_attention_sibling,
    ragged_attention_sibling_with_lse,
    ragged_attention_with_lse,
    ragged_attention_with_parents,
    ragged_tree_attn,
    set_layout_copies,
)
