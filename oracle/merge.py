"""Oracle for token_merge_bipartite2d (test infrastructure only).

`token_merge_reference` restates merging/merge.py:39-256 on the CPU, step for
step: the window pattern is built the way the reference builds it (one-hot
cell per window, then the (frames, h//sy, w//sx, sy, sx) -> (frames,
h//sy*sy, w//sx*sx) relayout, :119-163), then dst/src order, projection,
normalisation, similarity, top-r, index bookkeeping and slot sizes.  The two
things the reference draws from its device's generator -- the window cells
(:121-126) and the projection basis (:181-184) -- can be injected so that a
GPU run and this CPU restatement see the same draws.

Two orderings the reference delegates to torch's unstable sort (dst/src
split :165, merge order :199) are implementation-defined: torch's CPU sort
scrambles ties.  With `stable=False` the restatement makes the reference's
literal unstable calls (so it reproduces a CPU run of the reference
exactly); with `stable=True` (default) it uses stable sorts -- dst and src
tokens in position order, merge order by descending node_max with ties by
source position -- the canonical order the GPU product implements.

`merge_heads_fp64` is the brute-force K/V mean that pins `merge.heads`.
"""
from __future__ import annotations

from types import SimpleNamespace
from typing import Callable, Optional

import numpy as np
import torch

from .similarity import fast_similarity_chunks

PROJ_SEED = 1234


def window_draw(num_imgs, w, h, sx, sy, generator=None, device="cpu"):
    """The reference's window-cell draw (merging/merge.py:121-126)."""
    return torch.randint(sy * sx, size=(num_imgs - 1, h // sy, w // sx), device=device,
                         generator=generator)


def projection_basis(c: int, metric_dim: int, device="cpu", dtype=torch.float32):
    """The reference's seeded Gaussian basis (merging/merge.py:181-184)."""
    g = torch.Generator(device=device)
    g.manual_seed(PROJ_SEED)
    return torch.randn(c, metric_dim, device=device, dtype=torch.float32, generator=g).to(dtype)


def build_dst_mask(num_imgs, w, h, sx, sy, num_special, no_rand, cell):
    """[N] int64, -1 = dst, 0 = src, built as merging/merge.py:85-163 does."""
    tpi = w * h + num_special
    mask = torch.zeros(num_imgs * tpi, dtype=torch.int64)
    hsy, wsx = h // sy, w // sx
    if num_imgs > 0:
        mask[:tpi] = -1
    if num_imgs > 1:
        for f in range(1, num_imgs):
            mask[f * tpi: f * tpi + num_special] = -1
        eff_h, eff_w = min(hsy * sy, h), min(wsx * sx, w)
        if not no_rand:
            onehot = torch.zeros(num_imgs - 1, hsy, wsx, sy * sx, dtype=torch.int64)
            onehot.scatter_(3, cell.cpu().unsqueeze(-1), -1)
            grid = (onehot.view(num_imgs - 1, hsy, wsx, sy, sx).transpose(2, 3)
                    .reshape(num_imgs - 1, hsy * sy, wsx * sx))
            flat = grid[:, :eff_h, :eff_w].reshape(num_imgs - 1, -1)
            for f in range(1, num_imgs):
                lo = f * tpi + num_special
                mask[lo: lo + eff_h * eff_w] = flat[f - 1]
    return mask


def token_merge_reference(metric: torch.Tensor, w: int, h: int, sx: int, sy: int, r: int,
                          no_rand: bool = False, generator=None, metric_dim: int = 0,
                          num_special: int = 5, *, cell: Optional[torch.Tensor] = None,
                          proj: Optional[torch.Tensor] = None,
                          sim: Optional[Callable] = None,
                          stable: bool = True) -> SimpleNamespace:
    """CPU restatement of merging/merge.py:39-256.

    cell: window draw [frames-1, h//sy, w//sx] (default: drawn here with
    `generator`, as the reference does); proj: projection basis [C,
    metric_dim] (default: seeded CPU basis); sim(a, b) -> (node_max,
    node_idx) replaces the chunked similarity (default: fast_similarity_chunks
    with chunk min(5000, num_src), as at :191, :198).
    """
    metric = metric.cpu()
    bsz, n, c = metric.shape
    if r <= 0:
        raise ValueError("r must be positive")
    tpi = w * h + num_special
    num_imgs = n // tpi
    assert tpi * num_imgs == n
    if cell is None and num_imgs > 1 and not no_rand:
        cell = window_draw(num_imgs, w, h, sx, sy, generator)
    mask = build_dst_mask(num_imgs, w, h, sx, sy, num_special, no_rand, cell)
    if stable:
        order = torch.argsort(mask, stable=True)
    else:
        order = mask.reshape(1, -1, 1).argsort(dim=1).reshape(-1)
    num_dst = int((mask == -1).sum())
    a_idx = order[num_dst:]
    b_idx = order[:num_dst]
    num_src = a_idx.numel()

    if metric_dim and metric_dim < c:
        if proj is None:
            proj = projection_basis(c, metric_dim, dtype=metric.dtype)
        metric = metric @ proj.cpu().to(metric.dtype)
    metric = metric / metric.norm(dim=-1, keepdim=True)
    a = metric[:, a_idx]
    b = metric[:, b_idx]
    r = min(num_src, r)
    if sim is None:
        node_max, node_idx = fast_similarity_chunks(a, b.transpose(-1, -2), min(5000, num_src))
    else:
        node_max, node_idx = sim(a, b)
        node_max, node_idx = node_max.cpu(), node_idx.cpu()
    if stable:
        edge = torch.argsort(node_max, dim=-1, descending=True, stable=True)
    else:
        edge = node_max.argsort(dim=-1, descending=True)
    src_rows = edge[:, :r]
    unm_rows = edge[:, r:]
    dst_idx = torch.gather(node_idx, 1, src_rows)
    unm_abs = a_idx[unm_rows]
    src_abs = a_idx[src_rows]
    unm_len = unm_rows.shape[1]
    size = torch.ones(bsz, unm_len + num_dst, dtype=torch.float32)
    size[:, unm_len:].scatter_add_(1, dst_idx, torch.ones(bsz, r, dtype=torch.float32))

    def heads(t: torch.Tensor, mode: str = "mean") -> torch.Tensor:
        t = t.cpu()
        nb, nh, _, d = t.shape
        out = torch.empty(nb, nh, unm_len + num_dst, d, dtype=t.dtype)
        out[:, :, :unm_len] = torch.gather(t, 2, unm_abs[:, None, :, None].expand(nb, nh, unm_len, d))
        out[:, :, unm_len:] = t[:, :, b_idx]
        moved = torch.gather(t, 2, src_abs[:, None, :, None].expand(nb, nh, r, d))
        out[:, :, unm_len:].scatter_reduce_(2, dst_idx[:, None, :, None].expand(nb, nh, r, d),
                                            moved, reduce=mode)
        return out

    def merge(x: torch.Tensor, mode: str = "mean") -> torch.Tensor:
        return heads(x.cpu().unsqueeze(1), mode).squeeze(1)

    return SimpleNamespace(a_idx=a_idx, b_idx=b_idx, node_max=node_max, node_idx=node_idx,
                           edge_idx=edge, dst_idx=dst_idx, unm_abs_idx=unm_abs,
                           src_abs_idx=src_abs, size=size, num_dst=num_dst, num_src=num_src,
                           r=r, unm_len=unm_len, mask=mask, merge=merge, heads=heads)


def merge_heads_fp64(t: np.ndarray, unm_abs: np.ndarray, b_idx: np.ndarray,
                     src_abs: np.ndarray, dst_idx: np.ndarray) -> np.ndarray:
    """Brute-force fp64 mean merge for one batch element: t [H, N, D]."""
    t = np.asarray(t, dtype=np.float64)
    nh, _, d = t.shape
    unm_len, num_dst = len(unm_abs), len(b_idx)
    out = np.empty((nh, unm_len + num_dst, d))
    out[:, :unm_len] = t[:, unm_abs]
    acc = t[:, b_idx].copy()
    cnt = np.ones(num_dst)
    np.add.at(acc, (slice(None), dst_idx), t[:, src_abs])
    np.add.at(cnt, dst_idx, 1.0)
    out[:, unm_len:] = acc / cnt[None, :, None]
    return out
