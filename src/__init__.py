"""Drop-in import path of the reference (`from src.ragged_attn import ...`).

The modules here re-export qattention_amd so code written against the
reference's src package runs unchanged on MI355X.
"""
