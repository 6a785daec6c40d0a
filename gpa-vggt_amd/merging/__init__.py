"""GPA-VGGT token-merging hot path on MI355X (gfx950).

Drop-in replacement for the reference package `merging/`: put
`gpa-vggt_amd/` on `sys.path` ahead of the reference and
`from merging.merge import token_merge_bipartite2d`,
`from merging.fused_attention import attention_keybias`,
`from merging.fused_similarity import fused_similarity_argmax` resolve here.
"""
from . import merge

__all__ = ["merge"]
