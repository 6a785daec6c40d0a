"""Fused similarity + argmax for bipartite token matching, on gfx950.

Drop-in for the reference's `merging/fused_similarity.py`: same function
name, arguments, dtype contract and return types
(`fused_similarity_argmax`, reference :81-112).  The kernel itself is the
hand-written HIP kernel `sim_argmax_kernel` in `csrc/sim_argmax.hip`,
reached through the `gpa::sim_argmax` custom op.

Any feature dim up to 4096 (the projected 128-d metric, and the unprojected
1024-d metric of `metric_dim=0`, eval/eval_co3d.py:121-122).
Numerics: fp32 accumulation of bf16 (or fp16) products; the max is taken over the fp32
scores (not bf16-rounded scores as in the chunked torch path), and ties
resolve to the lowest destination index, as the reference kernel's strict
`>` across tiles plus `tl.argmax`'s first index do
(merging/fused_similarity.py:71-75).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _native

__all__ = ["fused_similarity_argmax"]


def fused_similarity_argmax(a: torch.Tensor, b: torch.Tensor):
    """node_max, node_idx = (a @ b.transpose(-1,-2)).max(dim=-1), fused.

    a: [B, M, D] src metric, b: [B, N, D] dst metric (GPU, fp16, bf16 or
    fp32).  Returns node_max [B, M] (a.dtype) and node_idx [B, M] (int64).
    Follows merging/fused_similarity.py:81-112: an fp32 `a` rounds both
    operands to bf16 first (:90-95); fp16 operands run the fp16 MFMA; the max
    comes back in a's dtype (:112).
    """
    if not (a.is_cuda and b.is_cuda and a.dim() == 3 and b.dim() == 3):
        raise AssertionError(
            "fused_similarity_argmax expects 3-D GPU tensors "
            f"(got a {tuple(a.shape)} on {a.device}, b {tuple(b.shape)} on {b.device})")
    out_dtype = a.dtype
    if a.dtype == torch.float32:
        a = a.to(torch.bfloat16)
        b = b.to(torch.bfloat16)
    if a.dtype != b.dtype or a.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"fused_similarity_argmax: a is {a.dtype}, b is {b.dtype}; the kernel "
                         "takes two bf16 or two fp16 operands (fp32 a casts both to bf16)")
    D = a.shape[-1]
    if b.shape[-1] != D:
        raise ValueError(f"feature dims differ: {D} vs {b.shape[-1]}")
    if D % 32:
        # Zero features add nothing to any dot product, so padding is exact.
        pad = 32 - D % 32
        a = F.pad(a, (0, pad))
        b = F.pad(b, (0, pad))
    # The kernel writes the max in a's 16-bit dtype itself when that is the
    # output dtype (fp32 inputs keep the fp32 max).
    node_max, node_idx = torch.ops.gpa.sim_argmax(a, b, out_dtype == a.dtype)
    return node_max.to(out_dtype), node_idx
