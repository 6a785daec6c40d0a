"""Seeded synthetic inputs for the merging hot-path workloads.

Shapes follow a VGGT-1B aggregator at 518x518: 1374 tokens per frame
(1 camera + 4 register + 37x37 patches), width 1024, 16 heads of 64.

  shifted_basis_tokens   frames of tokens x[f,p] = B[(p + o_f) mod 1369]
                         + 0.3 N(0,1), B a 1369 x 1024 N(0,1) basis and o_f a
                         per-frame offset in [0, 37): frames are shifted
                         copies of one texture, so cross-frame matches exist.
  sim_inputs             source/destination metrics for the similarity
                         kernel: tokens projected 1024 -> 128 by N(0,1)/sqrt(128),
                         L2-normalised, bf16; destinations are evenly spaced
                         (token floor(i*(m+n)/n)), i.e. every 4th token at
                         75,000 x 25,000.
  attn_inputs            biased-attention operands: Q/K/V ~ N(0,1)/sqrt(64)
                         bf16 and per-key bias log(c), c the counts of a
                         uniform multinomial assignment of M tokens to N keys
                         with every key given at least one.
  merge_inputs           a K/V merge of the same shape: [1,H,M,64] rows and
                         the slot lists (offsets, tokens) of a random
                         assignment of M tokens to N slots with those counts.
"""
from __future__ import annotations

import math
from typing import Tuple

import torch

TOKENS_PER_FRAME = 1374
PATCH_PERIOD = 1369
WIDTH = 1024
HEADS = 16
HEAD_DIM = 64


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def shifted_basis_tokens(frames: int, dim: int = WIDTH, seed: int = 0, device="cpu",
                         noise: float = 0.3, dtype=torch.float32) -> torch.Tensor:
    """[1, frames*1374, dim] tokens from one shifted basis plus noise."""
    g = _gen(device, seed)
    basis = torch.randn(PATCH_PERIOD, dim, generator=g, device=device)
    offsets = torch.randint(0, 37, (frames,), generator=g, device=device)
    p = torch.arange(TOKENS_PER_FRAME, device=device)
    rows = (p[None, :] + offsets[:, None]) % PATCH_PERIOD
    x = basis[rows]
    x.add_(torch.randn(x.shape, generator=g, device=device), alpha=noise)
    return x.reshape(1, frames * TOKENS_PER_FRAME, dim).to(dtype)


def projection(dim: int = WIDTH, out_dim: int = 128, seed: int = 1, device="cpu") -> torch.Tensor:
    """Gaussian projection dim -> out_dim scaled by 1/sqrt(out_dim)."""
    g = _gen(device, seed)
    return torch.randn(dim, out_dim, generator=g, device=device) / math.sqrt(out_dim)


def sim_inputs(m: int = 75_000, n: int = 25_000, out_dim: int = 128, seed: int = 0,
               device="cpu", dtype=torch.bfloat16) -> Tuple[torch.Tensor, torch.Tensor]:
    """(src [1, m, out_dim], dst [1, n, out_dim]) in `dtype` (bf16 or fp16),
    unit rows.

    m + n tokens come from `shifted_basis_tokens`, are projected and
    normalised in fp32, then rounded once to `dtype`; token
    floor(i * (m + n) / n) is destination i.
    """
    total = m + n
    frames = -(-total // TOKENS_PER_FRAME)
    x = shifted_basis_tokens(frames, seed=seed, device=device)[0, :total]
    y = x @ projection(x.shape[-1], out_dim, seed=seed + 1, device=device)
    del x
    y = y / y.norm(dim=-1, keepdim=True)
    is_dst = torch.zeros(total, dtype=torch.bool, device=device)
    is_dst[torch.arange(n, device=device) * total // n] = True
    dst = y[is_dst]
    src = y[~is_dst]
    return src.to(dtype).unsqueeze(0), dst.to(dtype).unsqueeze(0)


def merge_counts(m: int, n: int, seed: int = 0, device="cpu") -> torch.Tensor:
    """[n] float32 counts: 1 per key plus a uniform multinomial of m - n tokens."""
    if m < n:
        raise ValueError("merge_counts: need m >= n")
    g = _gen(device, seed + 7)
    extra = torch.randint(0, n, (m - n,), generator=g, device=device)
    return (torch.bincount(extra, minlength=n) + 1).to(torch.float32)


def attn_inputs(m: int = 274_800, n: int = 68_700, heads: int = HEADS, d: int = HEAD_DIM,
                seed: int = 0, device="cpu", bias_dtype=torch.bfloat16, dtype=torch.bfloat16):
    """(q [1,H,m,d], k [1,H,n,d], v [1,H,n,d], bias [1,H,1,n]) for the biased attention.

    q, k and v are N(0, 1/d) rounded once to `dtype` (bf16 or fp16); bias =
    log(counts) cast to `bias_dtype` (the q dtype in the model) and
    expanded to every head, the layout vggt/layers/attention.py:259-260
    hands to the kernel.
    """
    g = _gen(device, seed)
    s = 1.0 / math.sqrt(d)
    q = (torch.randn(1, heads, m, d, generator=g, device=device) * s).to(dtype)
    k = (torch.randn(1, heads, n, d, generator=g, device=device) * s).to(dtype)
    v = (torch.randn(1, heads, n, d, generator=g, device=device) * s).to(dtype)
    counts = merge_counts(m, n, seed=seed, device=device)
    bias = counts.log().to(bias_dtype).reshape(1, 1, 1, n).expand(1, heads, 1, n).contiguous()
    return q, k, v, bias


def attn_flops(bh: int, m: int, n: int, d: int = HEAD_DIM) -> float:
    """Algorithmic FLOPs of one biased attention call: QK^T plus PV."""
    return 4.0 * bh * m * n * d


def sim_flops(b: int, m: int, n: int, d: int) -> float:
    """Algorithmic FLOPs of one similarity-argmax call."""
    return 2.0 * b * m * n * d


def merge_inputs(m: int = 274_800, n: int = 66_845, heads: int = HEADS, d: int = HEAD_DIM,
                 dtype=torch.float32, seed: int = 0, device="cpu"):
    """(t [1,H,m,d], offsets [n+1] int64, tokens [m] int64): every token in
    exactly one of n slot lists, list lengths from `merge_counts`."""
    g = _gen(device, seed + 11)
    t = torch.randn(1, heads, m, d, generator=g, device=device).to(dtype)
    counts = merge_counts(m, n, seed=seed, device=device).to(torch.int64)
    offsets = torch.zeros(n + 1, dtype=torch.int64, device=device)
    offsets[1:] = torch.cumsum(counts, 0)
    tokens = torch.randperm(m, generator=g, device=device)
    return t, offsets, tokens


def merge_bytes(m: int, n: int, heads: int, d: int, elem: int) -> int:
    """Algorithmic HBM bytes of one merge: every row read once, every slot
    written once, the lists read once."""
    return (m + n) * heads * d * elem + 8 * (m + n + 1)
