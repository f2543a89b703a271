"""`src.tree_mask` drop-in: re-exports qattention_amd.tree_mask."""
from qattention_amd.tree_mask import *  # noqa: F401,F403
