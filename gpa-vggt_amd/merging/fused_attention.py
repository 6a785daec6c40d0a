"""Flash attention with a per-key additive bias, on gfx950.

Drop-in for the reference's `merging/fused_attention.py`: same function name,
arguments, dtype contract and return types (`attention_keybias`, reference
:130-180) and the same `LOG2E` constant (:40).  The kernel is the
hand-written HIP kernel `attn_keybias_kernel` in `csrc/attn_keybias.hip`,
reached through the `gpa::attn_keybias` custom op.

Math matches SDPA(q, k, v, attn_mask=bias): scores = q@k^T * scale + bias,
softmax over keys in fp32, P rounded to the operand format (bf16 or fp16)
for the P@V product, fp32 accumulation.  With return_lse the log2 softmax
denominators come back as well, so callers can split the key set and
recombine exactly (reference :123-127); `combine_by_lse` is that recombination for the
frame-special split path of vggt/layers/attention.py:148-176.
"""
from __future__ import annotations

import torch

from . import _native  # noqa: F401  (registers torch.ops.gpa.*)

__all__ = ["attention_keybias", "combine_by_lse", "LOG2E"]

LOG2E = 1.4426950408889634


def _autocast_dtype() -> torch.dtype:
    if torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return torch.bfloat16


def attention_keybias(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      bias: torch.Tensor, sm_scale: float, return_lse: bool = False):
    """SDPA(q, k, v, attn_mask=bias) where bias is per-key: [B, H, 1, N].

    q [B, H, M, D], k/v [B, H, N, D] (GPU, bf16 or fp16; fp32 inputs are cast
    to the autocast dtype or bf16 first, as at merging/fused_attention.py:
    139-144).  Returns [B, H, M, D] in q's dtype; with return_lse also
    [B, H, M] fp32 log2 softmax denominators.  `bias` may be None (plain
    attention).
    """
    if q.dtype == torch.float32:
        dt = _autocast_dtype()
        q, k, v = q.to(dt), k.to(dt), v.to(dt)
        bias = None if bias is None else bias.to(dt)
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise NotImplementedError(
            f"attention_keybias: {q.dtype} is not supported; the gfx950 kernels run bf16 and fp16")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("attention_keybias expects [B, H, T, D] q/k/v")
    v = v.to(q.dtype)
    k = k.to(q.dtype)
    o, lse = torch.ops.gpa.attn_keybias(q, k, v, bias, float(sm_scale), bool(return_lse))
    return (o, lse) if return_lse else o


def combine_by_lse(out_a: torch.Tensor, lse_a: torch.Tensor, out_b: torch.Tensor,
                   lse_b: torch.Tensor, frames: int) -> torch.Tensor:
    """Merge the two halves of the frame-special split attention.

    out_a [B*S, H, P, D], lse_a [B*S, H, P]: attention of every frame's P
    queries over the frame's own keys (frame-major, as the own-frame call of
    vggt/layers/attention.py:157 returns it); out_b [B, H, S*P, D], lse_b
    [B, H, S*P]: attention of all queries over the shared keys (:162).  The
    log2 LSEs weight the two (:166-176); returns [B, S*P, H*D] in the
    outputs' dtype (bf16 or fp16), the layout the output projection takes.
    The weights and the sum are fp32 (the reference rounds the weights to the
    activation dtype first).
    """
    return torch.ops.gpa.lse_combine(out_a, lse_a, out_b, lse_b, int(frames))
