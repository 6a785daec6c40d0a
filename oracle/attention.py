"""Oracle for the per-key-biased attention (test infrastructure only).

`attention_reference` is the reference's fallback path
(vggt/layers/attention.py:270-276, `F.scaled_dot_product_attention(q, k, v,
attn_mask=bias)`) evaluated on the CPU in fp32 on the same bf16 inputs the
kernel sees, after the dtype contract of `attention_keybias`
(merging/fused_attention.py:139-144: fp32 q/k/v/bias are rounded to bf16).
The log2 LSE follows merging/fused_attention.py:123-127 (exp2-domain
max + log2 of the denominator), i.e. logsumexp of the natural-log scores
times log2(e).  `attention_fp64` is the numpy closed form that pins it, and
`lse_combine` restates the exact two-partition merge of
vggt/layers/attention.py:166-176.
"""
from __future__ import annotations

from typing import Optional, Tuple

import numpy as np
import torch
import torch.nn.functional as F

LOG2E = 1.4426950408889634


def kernel_inputs(q, k, v, bias):
    """The bf16 tensors the kernel computes on (fused_attention.py:139-157)."""
    if q.dtype == torch.float32:
        q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
        bias = None if bias is None else bias.to(torch.bfloat16)
    v = v.to(q.dtype)
    return q, k, v, bias


def attention_reference(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        bias: Optional[torch.Tensor], sm_scale: float,
                        q_chunk: int = 2048) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp32 SDPA with an additive per-key bias, chunked over queries.

    q [B,H,M,D], k/v [B,H,N,D], bias broadcastable to [B,H,1,N] or None.
    Returns (o [B,H,M,D] fp32, lse2 [B,H,M] fp32 log2 denominators).
    """
    q32, k32, v32 = q.float().cpu(), k.float().cpu(), v.float().cpu()
    bsz, nh, m, d = q32.shape
    n = k32.shape[2]
    b32 = None if bias is None else bias.float().cpu().expand(bsz, nh, 1, n)
    out = torch.empty(bsz, nh, m, d, dtype=torch.float32)
    lse = torch.empty(bsz, nh, m, dtype=torch.float32)
    kt = k32.transpose(-1, -2).contiguous()
    for lo in range(0, m, q_chunk):
        hi = min(lo + q_chunk, m)
        s = torch.matmul(q32[:, :, lo:hi], kt) * sm_scale
        if b32 is not None:
            s = s + b32
        lse[:, :, lo:hi] = torch.logsumexp(s, dim=-1) * LOG2E
        out[:, :, lo:hi] = torch.matmul(torch.softmax(s, dim=-1), v32)
    return out, lse


def sdpa_reference(q, k, v, bias, sm_scale):
    """The reference's literal fallback call (attention.py:270-276).

    Used for the CPU baseline timing; numerically the same as
    `attention_reference` up to fp32 rounding.
    """
    return F.scaled_dot_product_attention(q, k, v, attn_mask=bias, scale=sm_scale)


def attention_fp64(q, k, v, bias, sm_scale):
    """numpy fp64 closed form: (o [B,H,M,D], lse2 [B,H,M])."""
    q64 = q.double().cpu().numpy()
    k64 = k.double().cpu().numpy()
    v64 = v.double().cpu().numpy()
    s = np.einsum("bhmd,bhnd->bhmn", q64, k64) * sm_scale
    if bias is not None:
        s = s + np.broadcast_to(bias.double().cpu().numpy(), (q64.shape[0], q64.shape[1], 1, k64.shape[2]))
    mx = s.max(axis=-1, keepdims=True)
    e = np.exp(s - mx)
    den = e.sum(axis=-1, keepdims=True)
    o = np.einsum("bhmn,bhnd->bhmd", e / den, v64)
    lse2 = (mx[..., 0] + np.log(den[..., 0])) / np.log(2.0)
    return o, lse2


def lse_combine(out_a: torch.Tensor, lse_a: torch.Tensor,
                out_b: torch.Tensor, lse_b: torch.Tensor) -> torch.Tensor:
    """Exact merge of two key partitions by their log2 LSE (attention.py:166-176)."""
    mx = torch.maximum(lse_a, lse_b)
    wa, wb = torch.exp2(lse_a - mx), torch.exp2(lse_b - mx)
    den = wa + wb
    return out_a * (wa / den).unsqueeze(-1) + out_b * (wb / den).unsqueeze(-1)
