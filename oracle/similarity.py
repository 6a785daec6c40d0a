"""Oracle for the fused similarity-argmax (test infrastructure only).

`fast_similarity_chunks` restates the reference's torch path
(merging/merge.py:13-36): bf16 inputs, a bf16 `bmm` per chunk of source rows
(so scores are rounded to bf16), then `torch.max(dim=2)`, whose index is the
first occurrence of the maximum.  `sim_argmax_fp64` is the brute-force fp64
check on the same bf16-rounded inputs: products of bf16 values are exact in
fp64, so the only error left is the fp64 summation.
"""
from __future__ import annotations

from typing import Tuple

import numpy as np
import torch


def bf16_round(x: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (nearest even) and return in fp32."""
    return x.to(torch.bfloat16).to(torch.float32)


def fast_similarity_chunks(a: torch.Tensor, b_transposed: torch.Tensor,
                           chunk_size: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Reference torch path of merging/merge.py:13-36, on the CPU.

    a [B, M, C], b_transposed [B, C, N].  Returns node_max [B, M] in a.dtype
    (the bf16 max cast back, :33) and node_idx [B, M] int64.
    """
    bsz, m, _ = a.shape
    out_dtype = a.dtype
    a16 = a.to(torch.bfloat16)
    # A transposed bf16 right operand of bmm is made contiguous first.
    b16 = b_transposed.to(torch.bfloat16).contiguous()
    node_max = torch.empty(bsz, m, dtype=out_dtype, device=a.device)
    node_idx = torch.empty(bsz, m, dtype=torch.int64, device=a.device)
    for lo in range(0, m, chunk_size):
        hi = min(lo + chunk_size, m)
        scores = torch.bmm(a16[:, lo:hi], b16)          # bf16 scores
        vmax, vidx = torch.max(scores, dim=2)
        node_max[:, lo:hi] = vmax.to(out_dtype)
        node_idx[:, lo:hi] = vidx
    return node_max, node_idx


def scores_fp64(a: torch.Tensor, b: torch.Tensor) -> np.ndarray:
    """fp64 a @ b^T per batch on bf16-rounded inputs: [B, M, N]."""
    a64 = bf16_round(a).double().numpy()
    b64 = bf16_round(b).double().numpy()
    return np.einsum("bmd,bnd->bmn", a64, b64, optimize=True)


def sim_argmax_fp64(a: torch.Tensor, b: torch.Tensor, row_chunk: int = 4096):
    """Exact-ish row max, first argmax and top-2 gap of a @ b^T in fp64.

    Returns (max [B,M] f64, idx [B,M] i64, gap [B,M] f64) where gap is the
    difference between the largest and second-largest score of the row
    (0 for exact ties; +inf when N == 1).
    """
    a64 = bf16_round(a).double().numpy()
    b64 = bf16_round(b).double().numpy()
    bsz, m, _ = a64.shape
    n = b64.shape[1]
    vmax = np.empty((bsz, m))
    vidx = np.empty((bsz, m), dtype=np.int64)
    gap = np.full((bsz, m), np.inf)
    for bi in range(bsz):
        bt = np.ascontiguousarray(b64[bi].T)
        for lo in range(0, m, row_chunk):
            s = a64[bi, lo:lo + row_chunk] @ bt
            idx = np.argmax(s, axis=1)          # first occurrence of the max
            top = s[np.arange(s.shape[0]), idx]
            vmax[bi, lo:lo + row_chunk] = top
            vidx[bi, lo:lo + row_chunk] = idx
            if n > 1:
                s[np.arange(s.shape[0]), idx] = -np.inf
                gap[bi, lo:lo + row_chunk] = top - s.max(axis=1)
    return vmax, vidx, gap


def bf16_top2_gap(a: torch.Tensor, b: torch.Tensor, chunk_size: int = 5000) -> torch.Tensor:
    """Top-2 gap of the bf16-rounded score rows the torch path compares.

    This is "the reference's top-2 similarity gap" of the parity rule: rows
    where it is below 1e-3 may legitimately pick a different index.
    """
    bsz, m, _ = a.shape
    a16 = a.to(torch.bfloat16)
    b16 = b.to(torch.bfloat16).transpose(1, 2).contiguous()
    out = torch.empty(bsz, m, dtype=torch.float32, device=a.device)
    for lo in range(0, m, chunk_size):
        hi = min(lo + chunk_size, m)
        s = torch.bmm(a16[:, lo:hi], b16).float()
        if s.shape[-1] == 1:
            out[:, lo:hi] = float("inf")
            continue
        top2 = torch.topk(s, 2, dim=2).values
        out[:, lo:hi] = top2[..., 0] - top2[..., 1]
    return out
