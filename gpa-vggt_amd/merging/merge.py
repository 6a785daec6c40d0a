"""Bipartite K/V token merge for GPA-VGGT, on gfx950.

Drop-in for the reference's `merging/merge.py`: `token_merge_bipartite2d`
keeps its signature and returns the same closure (`merge(x, mode)`,
`merge.heads(t, mode)`, `merge.size`), and `PROJ_SEED` keeps its value.
The similarity step always runs the gfx950 kernel (`fused_similarity_argmax`);
there is no chunked-bmm fallback.  `fast_similarity_chunks` keeps the
reference's name and arguments (reference :13-36) and runs the same kernel.

Orderings the reference leaves to torch's sort are fixed here:
  * dst / src order (reference :165): tokens in increasing position within
    each class -- a stable sort of the -1/0 mask;
  * merge order (reference :199): descending node_max, ties by increasing
    source position -- a stable descending sort.
On the GPU the reference's own calls (`reshape(1, -1, 1).argsort(dim=1)`
and `argsort(dim=-1, descending=True)`, torch's default sort) give exactly
these orders, for masks of 1 to 200 frames and node_max rows of 1,045 to
207,955 entries with tied values (tests/test_gpu_sort_order.py), so the
stable sorts change no result while making the order a documented property.
`merge.index` exposes the index tensors for inspection.

Under bf16 or fp16 autocast (the model's and the evaluation stack's
cases), or on a bf16 metric, the metric projection, normalisation, dst/src
split and bf16 cast (reference :180-187 and fused_similarity.py:90-95) run
as one gfx950 kernel
(`gpa::merge_metric`) that writes the similarity operands [dst | src]
directly; node_max keeps the dtype the reference's division yields (fp32
under autocast).  Other chains (fp32 arithmetic without autocast, no
projection) keep the torch ops on the device.

`merge` and `merge.heads` in "sum" / "mean" mode (fp32, bf16, fp16 rows)
run the deterministic gfx950 merge kernel (`gpa::merge_heads`): every
output slot lists its own token and the tokens merged into it once per
merge, and the sum runs over that list in fp32 in a fixed order.  The
reference's scatter_reduce_ (reference :246-249) sums with atomics in a
run-dependent order, in the rows' own precision; other modes keep that
gather + scatter_reduce_ on the device.
"""
from __future__ import annotations

from types import SimpleNamespace
from typing import Callable, Optional

import torch

from . import _native
from .fused_similarity import fused_similarity_argmax

__all__ = ["token_merge_bipartite2d", "fast_similarity_chunks", "PROJ_SEED", "dst_mask",
           "num_dst_tokens"]

# Seed of the fixed Gaussian basis used by the metric_dim random projection
# (reference merging/merge.py:10).
PROJ_SEED = 1234


def num_dst_tokens(num_imgs: int, w: int, h: int, sx: int, sy: int, num_special: int,
                   no_rand: bool) -> int:
    """Destination count implied by the mask rules of `dst_mask` (closed form)."""
    tpi = w * h + num_special
    if num_imgs <= 0:
        return 0
    if num_imgs == 1:
        return tpi
    per_frame = num_special + (0 if no_rand else (h // sy) * (w // sx))
    return tpi + (num_imgs - 1) * per_frame


def dst_mask(num_imgs: int, w: int, h: int, sx: int, sy: int, num_special: int,
             no_rand: bool, generator: Optional[torch.Generator],
             device: torch.device) -> torch.Tensor:
    """[num_imgs * (w*h + num_special)] int64 mask: -1 = dst, 0 = src.

    Rules of merging/merge.py:85-163: every token of frame 0 and the special
    tokens of every frame are dst; for frames >= 1 one cell of each sy x sx
    window is dst, drawn with one `torch.randint(sy*sx, (frames-1, h//sy,
    w//sx), generator=...)` call.  As in the reference, the window grid is
    laid out with row length (w//sx)*sx over the first (h//sy)*sy*(w//sx)*sx
    patch positions of the frame; `no_rand=True` marks no patch of frames
    >= 1 (reference :105-118 writes an all-zero pattern).
    """
    tpi = w * h + num_special
    n = num_imgs * tpi
    mask = torch.zeros(n, device=device, dtype=torch.int64)
    if num_imgs <= 0:
        return mask
    mask[:tpi] = -1
    if num_imgs == 1:
        return mask
    starts = torch.arange(1, num_imgs, device=device) * tpi
    mask[(starts[:, None] + torch.arange(num_special, device=device)).reshape(-1)] = -1
    if no_rand:
        return mask
    hsy, wsx = h // sy, w // sx
    cell = torch.randint(sy * sx, size=(num_imgs - 1, hsy, wsx), device=device,
                         generator=generator)
    row_len = wsx * sx
    ys = torch.arange(hsy, device=device).view(1, hsy, 1) * sy + cell // sx
    xs = torch.arange(wsx, device=device).view(1, 1, wsx) * sx + cell % sx
    pos = starts.view(-1, 1, 1) + num_special + ys * row_len + xs
    mask[pos.reshape(-1)] = -1
    return mask


def fast_similarity_chunks(a: torch.Tensor, b_transposed: torch.Tensor,
                           chunk_size: int):
    """node_max, node_idx of a @ b_transposed, under the reference's name
    and arguments (merging/merge.py:13-36), on the fused gfx950 kernel.

    a [B, M, C], b_transposed [B, C, N] on the GPU (fp32, bf16 or fp16).
    Like the reference, both operands are cast to bf16 whatever their dtype
    (:22-23) and node_max comes back as a bf16 value in a's dtype (:31-33);
    node_idx is int64.  No chunk of scores is materialised, so `chunk_size`
    (which must be positive, as the reference's `range` step) does not change
    the result.  The reference takes the max over bf16-rounded scores, this
    kernel over the fp32 scores and rounds the max once: rounding is
    monotonic, so the two maxima agree up to the order in which each sums a
    score's products, and node_idx differs from the reference's only where
    two destinations round to the same bf16 score
    (merging/fused_similarity.py:86 states the same of its own kernel).
    """
    if chunk_size <= 0:
        raise ValueError(f"fast_similarity_chunks: chunk_size must be positive, got {chunk_size}")
    if not (a.dim() == 3 and b_transposed.dim() == 3):
        raise AssertionError(
            "fast_similarity_chunks expects a [B, M, C] and b_transposed [B, C, N] "
            f"(got {tuple(a.shape)} and {tuple(b_transposed.shape)})")
    out_dtype = a.dtype
    node_max, node_idx = fused_similarity_argmax(
        a.to(torch.bfloat16), b_transposed.transpose(-1, -2).to(torch.bfloat16).contiguous())
    return node_max.to(out_dtype), node_idx


_PROJ_CACHE: dict = {}


def _projection(dev: torch.device, C: int, metric_dim: int,
                dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """The fixed Gaussian basis of the metric projection (reference
    merging/merge.py:181-184: `randn(C, metric_dim)` from a device generator
    seeded with PROJ_SEED), drawn once per device and shape and kept."""
    key = (dev, C, metric_dim, dtype)
    proj = _PROJ_CACHE.get(key)
    if proj is None:
        g_proj = torch.Generator(device=dev)
        g_proj.manual_seed(PROJ_SEED)
        proj = torch.randn(C, metric_dim, device=dev, dtype=torch.float32,
                           generator=g_proj).to(dtype)
        _PROJ_CACHE[key] = proj
    return proj


def _front_end_mode(metric: torch.Tensor, C: int, metric_dim: int) -> Optional[str]:
    """Which rounding chain the fused front end reproduces, or None when the
    reference's chain is one the kernel does not compute (no projection, a
    projection other than C -> 128, fp32 arithmetic without autocast, a
    non-fp32 metric under fp16 autocast)."""
    if metric_dim != 128 or C not in (256, 512, 768, 1024):
        return None
    if torch.is_autocast_enabled("cuda"):
        dt = torch.get_autocast_dtype("cuda")
        if dt == torch.bfloat16:
            return "autocast" if metric.dtype in (torch.float32, torch.bfloat16) else None
        if dt == torch.float16:
            return "autocast16" if metric.dtype == torch.float32 else None
        return None
    return "bf16" if metric.dtype == torch.bfloat16 else None


def token_merge_bipartite2d(
    metric: torch.Tensor,
    w: int,
    h: int,
    sx: int,
    sy: int,
    r: int,
    no_rand: bool = False,
    generator: Optional[torch.Generator] = None,
    metric_dim: int = 0,
    num_special: int = 5,
) -> Callable:
    """Bipartite token merging over the multi-frame token sequence.

    Same contract as merging/merge.py:39-256.  Tokens are split into dst (one
    random token per (sx, sy) window, every token of the first frame, every
    special token) and src; the r src tokens most similar to a dst token are
    merged into it.

    Returns merge(x [B, N, C], mode) -> [B, N - r, C] laid out as
    [unmerged src | dst]; merge.heads(t [B, H, N, D], mode) merges in
    head-major layout; merge.size [B, N - r] (B == 1, else None) holds the
    number of tokens behind each output slot.
    """
    B, N, C = metric.shape
    if r <= 0:
        raise ValueError("token_merge_bipartite2d: r must be positive")
    tpi = w * h + num_special
    num_imgs = N // tpi
    if tpi * num_imgs != N:
        raise AssertionError(
            f"Token count doesn't match (w*h+{num_special})*num_imgs: N={N} w={w} h={h}")
    if not metric.is_cuda:
        raise ValueError("token_merge_bipartite2d runs on the GPU; got a tensor on "
                         f"{metric.device}")
    dev = metric.device

    with torch.no_grad():
        mask = dst_mask(num_imgs, w, h, sx, sy, num_special, no_rand, generator, dev)
        num_dst = num_dst_tokens(num_imgs, w, h, sx, sy, num_special, no_rand)
        order = torch.argsort(mask, stable=True)  # dst positions first, then src
        b_pos = order[:num_dst]
        a_pos = order[num_dst:]
        num_src = N - num_dst

        front = _front_end_mode(metric, C, metric_dim)
        if front is not None:
            # One kernel: projection, normalisation, [dst | src] split and
            # bf16 cast (reference :180-187 plus the cast of
            # fused_similarity.py:90-95); node_max keeps the dtype the
            # reference's division produces.
            mode = {"autocast": 0, "bf16": 1, "autocast16": 2}[front]
            ab = _native.merge_metric(
                metric, _projection(dev, C, metric_dim,
                                    torch.float16 if mode == 2 else torch.bfloat16),
                order, mode)
            max_dtype = torch.bfloat16 if front == "bf16" else torch.float32
            a = ab[:, num_dst:]
            b = ab[:, :num_dst]
        else:
            if metric_dim and metric_dim < C:
                proj = _projection(dev, C, metric_dim, torch.float32).to(metric.dtype)
                metric = metric @ proj
            metric = metric / metric.norm(dim=-1, keepdim=True)
            a = metric.index_select(1, a_pos)
            b = metric.index_select(1, b_pos)
            max_dtype = metric.dtype

        r = min(num_src, r)
        if num_src > 0 and front is not None:
            node_max, node_idx = torch.ops.gpa.sim_argmax(a, b)     # fp32 row max
            node_max = node_max.to(max_dtype)
        elif num_src > 0:
            node_max, node_idx = fused_similarity_argmax(a, b)
        else:
            node_max = torch.empty(B, 0, device=dev, dtype=max_dtype)
            node_idx = torch.empty(B, 0, device=dev, dtype=torch.int64)
        edge = torch.argsort(node_max, dim=-1, descending=True, stable=True)
        src_rank = edge[:, :r]          # merged source rows (rows of `a`)
        unm_rank = edge[:, r:]          # kept source rows
        dst_slot = torch.gather(node_idx, 1, src_rank)        # [B, r] dst slot per merged row
        unm_abs = a_pos[unm_rank]                             # [B, unm_len] token positions
        src_abs = a_pos[src_rank]                             # [B, r]
        unm_len = unm_rank.shape[1]

        size = torch.ones(B, unm_len + num_dst, device=dev, dtype=torch.float32)
        size[:, unm_len:].scatter_add_(1, dst_slot, torch.ones(B, r, device=dev,
                                                                dtype=torch.float32))

        # Token list of every output slot, for the deterministic merge
        # kernel: slot i < unm_len holds kept source token unm_abs[i]; dst
        # slot unm_len + j holds dst token b_pos[j] first, then the source
        # tokens merged into it in increasing position.  Every input token
        # appears exactly once, so each batch element lists N tokens.
        slots = unm_len + num_dst
        key = torch.cat([torch.arange(unm_len, device=dev).expand(B, unm_len),
                         (unm_len + torch.arange(num_dst, device=dev)).expand(B, num_dst),
                         unm_len + dst_slot], dim=1)
        tok = torch.cat([unm_abs, b_pos.expand(B, num_dst), src_abs], dim=1)
        sub = torch.cat([torch.zeros(B, unm_len + num_dst, device=dev, dtype=torch.int64),
                         src_abs + 1], dim=1)      # the slot's own token sorts first
        order = torch.argsort(key * (N + 1) + sub, dim=1)
        csr_tokens = torch.gather(tok, 1, order).reshape(-1)
        csr_offsets = torch.zeros(B * slots + 1, device=dev, dtype=torch.int64)
        csr_offsets[1:] = torch.cumsum(size.reshape(-1).to(torch.int64), 0)

    def kernel_merge(t: torch.Tensor, mode: str) -> Optional[torch.Tensor]:
        """The deterministic gfx950 merge for sum / mean of fp32, bf16 and
        fp16 rows that split into 16-byte runs; None when it does not apply."""
        if (mode not in ("mean", "sum") or t.dtype not in (torch.float32, torch.bfloat16,
                                                           torch.float16)
                or t.shape[-1] % (16 // t.element_size()) != 0 or not t.is_cuda):
            return None
        out, _, _ = _native.merge_heads(t, csr_offsets, csr_tokens, slots, mode == "mean")
        return out

    def merge(x: torch.Tensor, mode: str = "mean") -> torch.Tensor:
        """[B, N, C] -> [B, unm_len + num_dst, C]: unmerged src, then dst."""
        if x.shape[0] != B or x.shape[1] != N:
            raise ValueError("merge input does not match the merge mapping")
        out = kernel_merge(x.unsqueeze(1), mode)
        if out is not None:
            return out.squeeze(1)
        nb, _, c = x.shape
        out = torch.empty(nb, unm_len + num_dst, c, device=x.device, dtype=x.dtype)
        torch.gather(x, 1, unm_abs[..., None].expand(nb, unm_len, c), out=out[:, :unm_len])
        torch.gather(x, 1, b_pos.view(1, -1, 1).expand(nb, num_dst, c), out=out[:, unm_len:])
        moved = torch.gather(x, 1, src_abs[..., None].expand(nb, r, c))
        out[:, unm_len:].scatter_reduce_(1, dst_slot[..., None].expand(nb, r, c), moved,
                                         reduce=mode)
        return out

    def merge_heads(t: torch.Tensor, mode: str = "mean") -> torch.Tensor:
        """Merge [B, H, N, D] K/V directly in the attention-kernel layout."""
        nb, nh, ntok, d = t.shape
        if nb != B or ntok != N:
            raise ValueError("merge_heads input does not match the merge mapping")
        out = kernel_merge(t, mode)
        if out is not None:
            return out
        out = torch.empty(nb, nh, unm_len + num_dst, d, device=t.device, dtype=t.dtype)
        torch.gather(t, 2, unm_abs[:, None, :, None].expand(nb, nh, unm_len, d),
                     out=out[:, :, :unm_len])
        torch.gather(t, 2, b_pos.view(1, 1, -1, 1).expand(nb, nh, num_dst, d),
                     out=out[:, :, unm_len:])
        moved = torch.gather(t, 2, src_abs[:, None, :, None].expand(nb, nh, r, d))
        out[:, :, unm_len:].scatter_reduce_(
            2, dst_slot[:, None, :, None].expand(nb, nh, r, d), moved, reduce=mode)
        return out

    merge.size = size if B == 1 else None
    merge.heads = merge_heads
    merge.index = SimpleNamespace(
        a_idx=a_pos, b_idx=b_pos, node_max=node_max, node_idx=node_idx, edge_idx=edge,
        dst_idx=dst_slot, unm_abs_idx=unm_abs, src_abs_idx=src_abs,
        num_dst=num_dst, num_src=num_src, r=r, unm_len=unm_len, mask=mask,
        slot_offsets=csr_offsets, slot_tokens=csr_tokens)
    return merge
