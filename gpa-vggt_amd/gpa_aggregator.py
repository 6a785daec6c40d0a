"""GPA aggregator harness: a random-init VGGT-1B aggregator with the GPA block
schedule, running the merging package's gfx950 kernels, for end-to-end latency.

This is the measurement harness around the hot path, not a model port.  It
restates, in plain torch modules, the layer sequence whose latency the
merging kernels sit in:

  * DINOv2 ViT-L/14 with 4 registers as the patch embedder
    (vggt/layers/vision_transformer.py:57-310; 24 blocks, LayerNorm eps 1e-6,
    LayerScale 1.0, plain attention over each frame's 1374 tokens);
  * camera + register tokens prepended per frame, 2D RoPE positions with the
    special tokens at 0 (vggt/models/aggregator.py:249-291);
  * 24 frame blocks alternating with 24 global blocks
    (aggregator.py:299-347), pre-LN blocks with LayerScale 0.01
    (vggt/layers/block.py:84-96), qk LayerNorm and RoPE (frequency 100,
    vggt/layers/rope.py:167-209);
  * the GPA schedule of aggregator.py:133-150 and :317-325: global blocks
    below `early_frame_split` run frame attention plus the shared K/V set
    (vggt/layers/attention.py:73-176, split path; the pooled summaries by
    the `gpa::pool_shared` kernel), global blocks in
    [merging, merge_end] merge K/V (attention.py:233-268) at `merge_ratio`,
    the core blocks at `core_merge_ratio`.

Everything on the merging path goes through the drop-in package:
`token_merge_bipartite2d` (similarity-argmax kernel + deterministic merge
kernel), `attention_keybias` (biased flash attention), `combine_by_lse`.
Frame attention (no bias) runs the same attention kernel with bias=None by
default; `frame_attn="sdpa"` switches the plain frame attention to torch's
SDPA, the reference's choice at attention.py:270-276, for comparison.

Weights are random (no checkpoint is available offline): Linear weights
N(0, 0.02^2), biases 0, LayerNorm weight 1 / bias 0, LayerScale gammas at the
reference's init values.  Run under `torch.autocast("cuda", bf16)` on a
bf16 model, as eval/bench_e2e.py:76-92 does.

The qk LayerNorm, RoPE and bf16 cast of every aggregator block run as one
fused kernel (`gpa::qk_norm_rope`) instead of the reference's separate torch
ops; K stays fp32 for the merge in merged blocks, as in the reference.

Known departure: RoPE angles are evaluated in fp64 and rounded once (a
table of cos/sin of p * f); the reference builds them through an einsum
that autocast may run in bf16.
"""
from __future__ import annotations

import time
from dataclasses import dataclass
from typing import Dict, List, NamedTuple, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from merging.fused_attention import attention_keybias, combine_by_lse
from merging.merge import token_merge_bipartite2d

RESNET_MEAN = (0.485, 0.456, 0.406)
RESNET_STD = (0.229, 0.224, 0.225)
MERGE_GENERATOR_SEED = 33              # attention.py:238-239


@dataclass
class GpaConfig:
    """Aggregator shape and GPA schedule; defaults are the paper's
    (aggregator.py:53-79, eval/eval_co3d.py:100-123)."""
    img_size: int = 518
    patch_size: int = 14
    embed_dim: int = 1024
    depth: int = 24
    num_heads: int = 16
    mlp_ratio: float = 4.0
    num_register_tokens: int = 4
    rope_freq: float = 100.0
    init_values: float = 0.01
    merging: Optional[int] = 9
    merge_end: int = 23
    merge_ratio: float = 0.98
    early_frame_split: int = 9
    broadcast_pool: int = 8
    core_blocks: Tuple[int, ...] = (13, 14, 15, 16)
    core_merge_ratio: float = 0.2
    merge_metric_dim: int = 128
    merge_grid: int = 2
    frame_attn: str = "gpa"            # "gpa" (attention kernel, bias=None) or "sdpa"
    fused_norms: bool = True           # residual + LayerScale + LayerNorm kernel (bf16 blocks)
    vit_depth: int = 24                # DINOv2 ViT-L/14 blocks
    dpt_blocks: Tuple[int, ...] = (4, 11, 17, 23)   # outputs kept (aggregator.py:296)
    img_width: Optional[int] = None    # image width; None: square (img_size x img_size)

    @property
    def grid_h(self) -> int:
        """Patch rows (ph, `patch_height` of attention.py:42)."""
        return self.img_size // self.patch_size

    @property
    def grid_w(self) -> int:
        """Patch columns (pw, `patch_width` of attention.py:41)."""
        return (self.img_width or self.img_size) // self.patch_size

    @property
    def grid(self) -> int:
        """Side of a square patch grid."""
        if self.grid_h != self.grid_w:
            raise ValueError(f"{self.grid_h} x {self.grid_w} patch grid is not square")
        return self.grid_h

    @property
    def num_special(self) -> int:
        return 1 + self.num_register_tokens

    @property
    def tokens_per_frame(self) -> int:
        return self.grid_h * self.grid_w + self.num_special

    def global_merging(self, block: int) -> Optional[int]:
        """The block index if global block `block` merges K/V (aggregator.py:317-325)."""
        if self.merging is None:
            return None
        in_window = (block >= self.merging
                     and (self.merge_end < 0 or block <= self.merge_end)
                     and block >= self.early_frame_split
                     and (block not in self.core_blocks or self.core_merge_ratio > 0))
        return block if in_window else None

    def block_kind(self, block: int) -> str:
        """'frame_special', 'merged' or 'global' for global block `block`."""
        if block < min(self.early_frame_split, self.depth):
            return "frame_special"
        return "merged" if self.global_merging(block) is not None else "global"

    def block_merge_ratio(self, block: int) -> float:
        return self.core_merge_ratio if block in self.core_blocks else self.merge_ratio


def vanilla_config(**kw) -> GpaConfig:
    """VGGT without GPA: plain global attention everywhere (eval_co3d.py:127-128)."""
    return GpaConfig(merging=None, early_frame_split=0, **kw)


# ---------------------------------------------------------------------------
# building blocks
# ---------------------------------------------------------------------------

class RopeTable(NamedTuple):
    """Positions [P, 2] int32 of one frame's tokens (token n uses row
    n mod P) and the (cos, sin) table [npos, head_dim/4, 2] fp32."""
    pos: torch.Tensor
    cs: torch.Tensor


class Rope2D:
    """2D rotary embedding: the first half of each head's features rotates
    with the row coordinate, the second half with the column coordinate, each
    half as [x1, x2] -> [x1 cos - x2 sin, x2 cos + x1 sin] with frequencies
    freq^(-2i/half) (rope.py:92-209).  The rotation itself runs fused with
    the qk LayerNorm in the `gpa::qk_norm_rope` kernel."""

    def __init__(self, freq: float):
        self.freq = freq

    def cs_table(self, npos: int, head_dim: int, device="cpu") -> torch.Tensor:
        """[npos, head_dim/4, 2] fp32: (cos, sin) of p * freq^(-2j/(head_dim/2)),
        evaluated in fp64 and rounded once."""
        half = head_dim // 2
        inv = self.freq ** (-torch.arange(0, half, 2, dtype=torch.float64) / half)
        ang = torch.arange(npos, dtype=torch.float64)[:, None] * inv
        return torch.stack((ang.cos(), ang.sin()), dim=-1).float().to(device)

    def table(self, pos: torch.Tensor, head_dim: int) -> RopeTable:
        npos = int(pos.max()) + 1
        return RopeTable(pos.to(torch.int32).contiguous(),
                         self.cs_table(npos, head_dim, pos.device))


class LayerScale(nn.Module):
    def __init__(self, dim: int, init: float):
        super().__init__()
        self.gamma = nn.Parameter(torch.full((dim,), float(init)))

    def forward(self, x):
        return x * self.gamma


class Mlp(nn.Module):
    def __init__(self, dim: int, hidden: int):
        super().__init__()
        self.fc1 = nn.Linear(dim, hidden)
        self.fc2 = nn.Linear(hidden, dim)

    def forward(self, x):
        return self.fc2(F.gelu(self.fc1(x)))


def _frame_attention(q, k, v, scale: float, backend: str) -> torch.Tensor:
    """Plain attention, [b, H, T, D] -> [b, H, T, D] bf16."""
    if backend == "sdpa":
        return F.scaled_dot_product_attention(q, k, v)
    return attention_keybias(q, k, v, None, scale)


class GpaAttention(nn.Module):
    """Attention of a VGGT block with the GPA global paths (attention.py:17-282)."""

    def __init__(self, dim: int, heads: int, qk_norm: bool, norm_eps: float, cfg: GpaConfig):
        super().__init__()
        self.heads, self.head_dim = heads, dim // heads
        self.scale = self.head_dim ** -0.5
        self.qkv = nn.Linear(dim, 3 * dim)
        self.q_norm = nn.LayerNorm(self.head_dim, eps=norm_eps) if qk_norm else nn.Identity()
        self.k_norm = nn.LayerNorm(self.head_dim, eps=norm_eps) if qk_norm else nn.Identity()
        self.proj = nn.Linear(dim, dim)
        self.cfg = cfg
        self.frame_special = False
        self.merge_ratio = cfg.merge_ratio
        self.tracer: Optional["StageTimer"] = None
        # When a list: every merge / pooling of this module appends a record
        # (device tensors, no host synchronisation inside the forward).
        self.merge_log: Optional[list] = None

    def _mark(self, name: str) -> None:
        if self.tracer is not None:
            self.tracer.mark(name)

    def qk(self, x: torch.Tensor, rope: Optional[RopeTable], k_f32: bool = False):
        """q, k, v [B, H, N, D] from the block input (attention.py:210-220).

        With qk LayerNorm the normalisation, the rotation and the cast run
        as one `gpa::qk_norm_rope` kernel over the bf16 (or, under fp16
        autocast, fp16) projection (q in the projection's format; k fp32
        when `k_f32`, for the K merge, else the projection's format); v
        stays a view of the projection.  Without it (the patch embedder's blocks) q, k, v
        are all views of the projection.
        """
        B, N, C = x.shape
        H, D = self.heads, self.head_dim
        qkv = self.qkv(x)
        v = qkv.view(B, N, 3, H, D)[:, :, 2].transpose(1, 2)
        if isinstance(self.q_norm, nn.LayerNorm):
            if qkv.dtype not in (torch.bfloat16, torch.float16):
                raise ValueError("the fused qk-norm/RoPE kernel takes a bf16 or fp16 "
                                 "projection (run the model under bf16 or fp16 autocast)")
            ln_w = torch.stack((self.q_norm.weight, self.k_norm.weight))
            ln_b = torch.stack((self.q_norm.bias, self.k_norm.bias))
            q, k = torch.ops.gpa.qk_norm_rope(
                qkv, ln_w, ln_b, self.q_norm.eps, None if rope is None else rope.pos,
                None if rope is None else rope.cs, H, False, k_f32)
            return q, k, v
        if rope is not None:
            raise ValueError("RoPE without qk LayerNorm is not implemented")
        t = qkv.view(B, N, 3, H, D)
        return t[:, :, 0].transpose(1, 2), t[:, :, 1].transpose(1, 2), v

    def forward(self, x: torch.Tensor, rope: Optional[RopeTable] = None,
                global_merging: Optional[int] = None):
        B, N, C = x.shape
        H, D = self.heads, self.head_dim
        q, k, v = self.qk(x, rope, k_f32=global_merging is not None and not self.frame_special)
        self._mark("qkv")

        if self.frame_special:
            out = self._frame_special(q, k, v, B, N, C)
            self._mark("frame_special_attn")
            return self.proj(out)

        if global_merging is not None:
            gen = torch.Generator(device=x.device)
            gen.manual_seed(MERGE_GENERATOR_SEED)
            r = int(N * self.merge_ratio)
            m = token_merge_bipartite2d(x, self.cfg.grid_w, self.cfg.grid_h, self.cfg.merge_grid,
                                        self.cfg.merge_grid, r,
                                        False, gen, metric_dim=self.cfg.merge_metric_dim,
                                        num_special=self.cfg.num_special)
            k = m.heads(k, "mean")
            v = m.heads(v, "mean")
            if self.merge_log is not None:
                self.merge_log.append({"kind": "merged", "block": global_merging, "tokens": N,
                                       "num_dst": m.index.num_dst, "r": m.index.r,
                                       "size": m.size, "slot_offsets": m.index.slot_offsets,
                                       "keys": k.shape[2]})
            size = m.size
            if size is None:
                # More than one scene: the sizes as the reference forms them
                # (vggt/layers/attention.py:250-253), summed ones.
                size = m(torch.ones(B, N, 1, device=x.device, dtype=torch.float32), "sum")
            bias = size.reshape(B, 1, 1, -1).log().to(q.dtype).expand(B, H, 1, k.shape[2])
            self._mark("merge")
            out = attention_keybias(q, k, v, bias, self.scale)
            self._mark("merged_attn")
        elif N > self.cfg.tokens_per_frame:
            out = attention_keybias(q, k, v, None, self.scale)
            self._mark("global_attn")
        else:
            out = _frame_attention(q, k, v, self.scale, self.cfg.frame_attn)
            self._mark("frame_attn")
        return self.proj(out.transpose(1, 2).reshape(B, N, C))

    def _frame_special(self, q, k, v, B, N, C) -> torch.Tensor:
        """Frame attention + shared K/V set, split path (attention.py:148-176)."""
        if q.dtype == torch.float32:
            dt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") \
                else torch.bfloat16
            q, k, v = q.to(dt), k.to(dt), v.to(dt)
        H, D = self.heads, self.head_dim
        pts, gh, gw = self.cfg.num_special, self.cfg.grid_h, self.cfg.grid_w
        P = gh * gw + pts
        S = N // P
        if S * P != N:
            raise ValueError(f"frame_special: {N} tokens is not a multiple of {P}")
        q_f = q.view(B, H, S, P, D).permute(0, 2, 1, 3, 4).reshape(B * S, H, P, D)
        k5, v5 = k.view(B, H, S, P, D), v.view(B, H, S, P, D)
        kp = self.cfg.broadcast_pool
        if kp < 0:
            # No shared set: plain attention over each frame's own tokens
            # (attention.py:178-182).
            k_f = k5.permute(0, 2, 1, 3, 4).reshape(B * S, H, P, D)
            v_f = v5.permute(0, 2, 1, 3, 4).reshape(B * S, H, P, D)
            out = attention_keybias(q_f, k_f, v_f, None, self.scale)
            return out.reshape(B, S, H, P, D).permute(0, 1, 3, 2, 4).reshape(B, N, C)
        own_k = k5[:, :, :, pts:].permute(0, 2, 1, 3, 4).reshape(B * S, H, P - pts, D)
        own_v = v5[:, :, :, pts:].permute(0, 2, 1, 3, 4).reshape(B * S, H, P - pts, D)
        out_a, lse_a = attention_keybias(q_f, own_k, own_v, None, self.scale, return_lse=True)
        del own_k, own_v
        self._mark("frame_special_attn")
        if kp > 0:
            pooled_k, pooled_v, pool_size, _ = pool_shared_set(k, v, S, pts, gh, gw, kp)
            if self.merge_log is not None:
                self.merge_log.append({"kind": "pool", "frames": S, "pool_size": pool_size})
            sh_k = torch.cat([k5[:, :, :, :pts].reshape(B, H, S * pts, D), pooled_k], dim=2)
            sh_v = torch.cat([v5[:, :, :, :pts].reshape(B, H, S * pts, D), pooled_v], dim=2)
            bias = torch.zeros(B, H, 1, sh_k.shape[2], device=q.device, dtype=torch.float32)
            bias[:, :, 0, S * pts:] = pool_size.log().reshape(B, H, -1)
            bias = bias.to(q.dtype)
        else:
            sh_k = k5[:, :, :, :pts].reshape(B, H, S * pts, D)
            sh_v = v5[:, :, :, :pts].reshape(B, H, S * pts, D)
            bias = None
        self._mark("pool")
        out_b, lse_b = attention_keybias(q, sh_k, sh_v, bias, self.scale, return_lse=True)
        return combine_by_lse(out_a, lse_a, out_b, lse_b, S)


POOL_KERNEL_MAX_PATCHES = 4096   # patches per frame the gpa::pool_shared kernels hold


def pool_shared_set(k: torch.Tensor, v: torch.Tensor, frames: int, pts: int, grid_h: int,
                    grid_w: int, kp: int, want_assign: bool = False):
    """The pooled summaries of the shared set (attention.py:113-140) from
    k, v [B, H, S*P, D] on a grid_h x grid_w patch grid (ph x pw there): the
    `gpa::pool_shared` kernels for bf16/fp16 k and v of head dim 64 and up
    to 4,096 patches per frame, any pool stride (seeds held in registers up
    to 64 per frame, in super-chunks of 64 above); otherwise the
    reference's own torch ops on the device (`pool_shared_torch`).
    Returns (pooled_k, pooled_v [B, H, S*npool, D], size [B, H, S, npool]
    fp32, assign [B, H, S, grid_h*grid_w] or an empty tensor)."""
    if (grid_h * grid_w <= POOL_KERNEL_MAX_PATCHES and k.shape[-1] == 64
            and k.dtype in (torch.bfloat16, torch.float16)):
        return torch.ops.gpa.pool_shared(k, v, frames, pts, grid_h, grid_w, kp, want_assign)
    B, H, N, D = k.shape
    P = N // frames
    pk, pv, size, assign = pool_shared_torch(k.view(B, H, frames, P, D),
                                             v.view(B, H, frames, P, D), pts, grid_h, grid_w, kp)
    return pk, pv, size, assign if want_assign else assign.new_empty(0)


def pool_shared_torch(k5: torch.Tensor, v5: torch.Tensor, pts: int, grid_h: int, grid_w: int,
                      kp: int):
    """Content-adaptive pooled summaries of the shared K/V set (attention.py:113-140),
    restated with torch ops.  The harness runs the `gpa::pool_shared`
    kernels wherever they apply (bf16/fp16, head dim 64, <= 4,096 patches)
    and this restatement otherwise; the tests pin the kernels against it.

    k5/v5 [B, H, S, P, D], patches row-major on a grid_h x grid_w grid.
    Seeds are the stride-kp lattice patches; every patch joins the seed whose
    key it matches best by cosine (per head), and a summary is the mean of
    its group, for keys and values alike.  Returns (pooled_k, pooled_v
    [B, H, S*npool, D] in the input dtype, size [B, H, S, npool] fp32,
    assign [B, H, S, grid_h*grid_w] int64).
    """
    B, H, S, P, D = k5.shape
    npatch = grid_h * grid_w
    npool = -(-grid_h // kp) * -(-grid_w // kp)
    xk = k5[:, :, :, pts:].reshape(B, H, S, grid_h, grid_w, D)
    seeds = xk[:, :, :, ::kp, ::kp].reshape(B, H, S, npool, D).float()
    a = xk.reshape(B, H, S, npatch, D).float()
    a = a / a.norm(dim=-1, keepdim=True).clamp_min(1e-6)
    seeds = seeds / seeds.norm(dim=-1, keepdim=True).clamp_min(1e-6)
    assign = torch.matmul(a, seeds.transpose(-1, -2).contiguous()).argmax(-1)
    del a, seeds
    size = torch.zeros(B, H, S, npool, device=k5.device, dtype=torch.float32)
    size.scatter_add_(3, assign, torch.ones_like(assign, dtype=torch.float32))
    idx = assign[..., None].expand(B, H, S, npatch, D)
    out = []
    for t5 in (k5, v5):
        acc = torch.zeros(B, H, S, npool, D, device=k5.device, dtype=torch.float32)
        acc.scatter_add_(3, idx, t5[:, :, :, pts:].reshape(B, H, S, npatch, D).float())
        acc /= size.clamp_min(1.0).unsqueeze(-1)
        out.append(acc.reshape(B, H, S * npool, D).to(t5.dtype))
    return out[0], out[1], size, assign


class Block(nn.Module):
    """Pre-LN transformer block with LayerScale (block.py:84-96)."""

    def __init__(self, dim: int, heads: int, mlp_ratio: float, ls_init: float,
                 qk_norm: bool, norm_eps: float, cfg: GpaConfig):
        super().__init__()
        self.norm1 = nn.LayerNorm(dim, eps=norm_eps)
        self.attn = GpaAttention(dim, heads, qk_norm, 1e-5, cfg)
        self.ls1 = LayerScale(dim, ls_init)
        self.norm2 = nn.LayerNorm(dim, eps=norm_eps)
        self.mlp = Mlp(dim, int(dim * mlp_ratio))
        self.ls2 = LayerScale(dim, ls_init)

    def _fused_ok(self, x: torch.Tensor) -> bool:
        """The fused kernel reproduces the 16-bit chain: a bf16 (fp16) block
        on a bf16 (fp16) stream, under autocast to that format or none."""
        dt = x.dtype
        if not (self.attn.cfg.fused_norms and x.is_cuda and dt in (torch.bfloat16, torch.float16)
                and x.shape[-1] % 512 == 0 and self.norm1.weight.dtype == dt
                and self.ls1.gamma.dtype == dt):
            return False
        return not torch.is_autocast_enabled("cuda") or torch.get_autocast_dtype("cuda") == dt

    def forward(self, x, rope: Optional[RopeTable] = None, global_merging=None):
        if self._fused_ok(x):
            # block.py:84-96 with the elementwise steps fused: LayerNorm 1 to
            # the 16-bit format; x + ls1(attn) with LayerNorm 2 in one pass;
            # x + ls2(mlp).
            rl = torch.ops.gpa.residual_layernorm
            _, ln1 = rl(x, None, None, self.norm1.weight, self.norm1.bias, self.norm1.eps, False)
            a = self.attn(ln1, rope, global_merging)
            h, ln2 = rl(x, a, self.ls1.gamma, self.norm2.weight, self.norm2.bias,
                        self.norm2.eps, True)
            out, _ = rl(h, self.mlp(ln2), self.ls2.gamma, None, None, 0.0, True)
            return out
        x = x + self.ls1(self.attn(self.norm1(x), rope, global_merging))
        return x + self.ls2(self.mlp(self.norm2(x)))


class DinoV2Reg(nn.Module):
    """DINOv2 ViT-L/14 with register tokens as the patch embedder
    (vision_transformer.py:259-310): conv patchify, cls + position
    embedding, registers after cls, 24 blocks, final LayerNorm; returns the
    normalised patch tokens."""

    def __init__(self, cfg: GpaConfig):
        super().__init__()
        dim = cfg.embed_dim
        self.patch = nn.Conv2d(3, dim, cfg.patch_size, cfg.patch_size)
        self.cls_token = nn.Parameter(torch.zeros(1, 1, dim))
        self.pos_embed = nn.Parameter(torch.zeros(1, cfg.grid_h * cfg.grid_w + 1, dim))
        self.register_tokens = nn.Parameter(torch.zeros(1, cfg.num_register_tokens, dim))
        self.blocks = nn.ModuleList(
            Block(dim, cfg.num_heads, cfg.mlp_ratio, 1.0, False, 1e-6, cfg)
            for _ in range(cfg.vit_depth))
        self.norm = nn.LayerNorm(dim, eps=1e-6)
        self.nreg = cfg.num_register_tokens

    def patchify(self, img: torch.Tensor) -> torch.Tensor:
        """The stride-14 14x14 convolution as what it is, one GEMM over the
        non-overlapping patches (MIOpen runs this conv shape with its naive
        direct kernel, ~120 ms at 200 frames).  [B, 3, H, W] -> [B, P, D]."""
        B, C, H, W = img.shape
        ps = self.patch.kernel_size[0]
        gh, gw = H // ps, W // ps
        cols = (img[:, :, :gh * ps, :gw * ps].reshape(B, C, gh, ps, gw, ps)
                .permute(0, 2, 4, 1, 3, 5).reshape(B * gh * gw, C * ps * ps))
        w = self.patch.weight.reshape(self.patch.out_channels, C * ps * ps)
        return F.linear(cols, w, self.patch.bias).view(B, gh * gw, -1)

    def forward(self, img: torch.Tensor) -> torch.Tensor:
        x = self.patchify(img)
        x = torch.cat((self.cls_token.expand(x.shape[0], -1, -1).to(x.dtype), x), dim=1)
        x = x + self.pos_embed.to(x.dtype)
        x = torch.cat((x[:, :1], self.register_tokens.expand(x.shape[0], -1, -1).to(x.dtype),
                       x[:, 1:]), dim=1)
        for blk in self.blocks:
            x = blk(x)
        return self.norm(x)[:, 1 + self.nreg:]


class StageTimer:
    """Device-time marks on the current stream, summed per stage name."""

    def __init__(self):
        self.events: List[Tuple[str, torch.cuda.Event]] = []

    def start(self) -> None:
        self.events = []
        self.mark("start")

    def mark(self, name: str) -> None:
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        self.events.append((name, e))

    def totals(self) -> Dict[str, float]:
        torch.cuda.synchronize()
        out: Dict[str, float] = {}
        for (_, e0), (name, e1) in zip(self.events, self.events[1:]):
            out[name] = out.get(name, 0.0) + e0.elapsed_time(e1)
        return out


class GpaAggregator(nn.Module):
    """The VGGT aggregator with the GPA schedule (aggregator.py:26-357)."""

    def __init__(self, cfg: GpaConfig):
        super().__init__()
        self.cfg = cfg
        dim = cfg.embed_dim
        self.patch_embed = DinoV2Reg(cfg)
        self.camera_token = nn.Parameter(torch.randn(1, 2, 1, dim) * 1e-6)
        self.register_token = nn.Parameter(torch.randn(1, 2, cfg.num_register_tokens, dim) * 1e-6)
        mk = lambda: Block(dim, cfg.num_heads, cfg.mlp_ratio, cfg.init_values, True, 1e-5, cfg)  # noqa: E731
        self.frame_blocks = nn.ModuleList(mk() for _ in range(cfg.depth))
        self.global_blocks = nn.ModuleList(mk() for _ in range(cfg.depth))
        for i, blk in enumerate(self.global_blocks):
            blk.attn.frame_special = cfg.block_kind(i) == "frame_special"
            blk.attn.merge_ratio = cfg.block_merge_ratio(i)
        self.rope = Rope2D(cfg.rope_freq)
        self.register_buffer("mean", torch.tensor(RESNET_MEAN).view(1, 1, 3, 1, 1), persistent=False)
        self.register_buffer("std", torch.tensor(RESNET_STD).view(1, 1, 3, 1, 1), persistent=False)
        self.tracer: Optional[StageTimer] = None

    def set_tracer(self, tracer: Optional[StageTimer]) -> None:
        self.tracer = tracer
        for blk in list(self.frame_blocks) + list(self.global_blocks):
            blk.attn.tracer = tracer

    def set_merge_log(self, log: Optional[list]) -> None:
        """Collect one record per merge and per shared-set pooling of the
        global blocks into `log` (None stops collecting)."""
        for blk in self.global_blocks:
            blk.attn.merge_log = log

    def _mark(self, name: str) -> None:
        if self.tracer is not None:
            self.tracer.mark(name)

    def positions(self, device) -> torch.Tensor:
        return frame_positions(self.cfg.grid_h, self.cfg.num_special, device,
                               grid_w=self.cfg.grid_w)

    def embed(self, images: torch.Tensor) -> torch.Tensor:
        """[B, S, 3, H, W] in [0, 1] -> tokens [B*S, P, C] in the model dtype."""
        B, S, C_in, Hh, Ww = images.shape
        dt = self.camera_token.dtype
        x = ((images - self.mean) / self.std).to(dt).view(B * S, C_in, Hh, Ww)
        patches = self.patch_embed(x).to(dt)
        cam = _first_vs_rest(self.camera_token, B, S)
        reg = _first_vs_rest(self.register_token, B, S)
        return torch.cat((cam, reg, patches), dim=1).to(dt)

    def rope_table(self, device) -> RopeTable:
        return self.rope.table(self.positions(device), self.cfg.embed_dim // self.cfg.num_heads)

    def forward(self, images: torch.Tensor) -> List[torch.Tensor]:
        B, S = images.shape[:2]
        tokens = self.embed(images)
        self._mark("patch_embed")
        P, C = tokens.shape[1], tokens.shape[2]
        rope = self.rope_table(images.device)
        outputs = []
        for i in range(self.cfg.depth):
            tokens = self.frame_blocks[i](tokens.view(B * S, P, C), rope)
            self._mark("frame_block")
            frame_out = tokens.view(B, S, P, C)
            tokens = self.global_blocks[i](tokens.view(B, S * P, C), rope,
                                           self.cfg.global_merging(i))
            self._mark(f"global_block_{self.cfg.block_kind(i)}")
            if i in self.cfg.dpt_blocks:
                outputs.append(torch.cat((frame_out, tokens.view(B, S, P, C)), dim=-1))
        return outputs


def frame_positions(grid: int, num_special: int, device="cpu",
                    grid_w: Optional[int] = None) -> torch.Tensor:
    """[P, 2] RoPE positions of one frame on a grid x grid_w patch grid
    (grid_w None: square): specials at (0, 0), patch (y, x) at (y + 1, x + 1),
    row-major (aggregator.py:279-288, rope.py:54-65)."""
    gw = grid if grid_w is None else grid_w
    yx = torch.cartesian_prod(torch.arange(grid, device=device), torch.arange(gw, device=device))
    return torch.cat((torch.zeros(num_special, 2, dtype=yx.dtype, device=device), yx + 1))


def _first_vs_rest(tok: torch.Tensor, B: int, S: int) -> torch.Tensor:
    """(1, 2, X, C) -> (B*S, X, C): slot 0 for frame 0, slot 1 for the others
    (aggregator.py:420-442)."""
    first = tok[:, :1].expand(B, 1, *tok.shape[2:])
    rest = tok[:, 1:].expand(B, S - 1, *tok.shape[2:])
    return torch.cat((first, rest), dim=1).reshape(B * S, *tok.shape[2:])


def init_random_(model: nn.Module, seed: int = 0) -> nn.Module:
    """Random init in place: Linear/Conv weights N(0, 0.02^2), biases 0,
    LayerNorm 1/0, position embedding N(0, 0.02^2); LayerScale and the
    special tokens keep their constructor values."""
    g = torch.Generator(device=next(model.parameters()).device)
    g.manual_seed(seed)
    with torch.no_grad():
        for mod in model.modules():
            if isinstance(mod, (nn.Linear, nn.Conv2d)):
                mod.weight.normal_(0.0, 0.02, generator=g)
                if mod.bias is not None:
                    mod.bias.zero_()
            elif isinstance(mod, nn.LayerNorm):
                mod.weight.fill_(1.0)
                mod.bias.zero_()
            elif isinstance(mod, DinoV2Reg):
                mod.pos_embed.normal_(0.0, 0.02, generator=g)
                mod.cls_token.normal_(0.0, 1e-6, generator=g)
                mod.register_tokens.normal_(0.0, 1e-6, generator=g)
    return model


def build_aggregator(cfg: Optional[GpaConfig] = None, device="cuda", dtype=torch.bfloat16,
                     seed: int = 0) -> GpaAggregator:
    """A random-init aggregator on `device` in `dtype`, in eval mode."""
    cfg = cfg or GpaConfig()
    with torch.device(device):
        model = GpaAggregator(cfg)
    init_random_(model, seed)
    return model.to(dtype).eval()


def shifted_texture_images(frames: int, size=518, shift: int = 64, seed: int = 0,
                           device="cpu", dtype=torch.float32) -> torch.Tensor:
    """[1, frames, 3, h, w] (size = h = w, or size = (h, w)) i.i.d. U[0,1]
    RGB crops of one shared random texture at per-frame random offsets in
    [0, shift)^2: every frame is a translated view of the same content."""
    h, w = (size, size) if isinstance(size, int) else size
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    tex = torch.rand(3, h + shift, w + shift, generator=g, device=device)
    off = torch.randint(0, shift, (frames, 2), generator=g, device=device).tolist()
    imgs = torch.stack([tex[:, y:y + h, x:x + w] for y, x in off])
    return imgs.unsqueeze(0).to(dtype)


def timed(fn, warmup: int = 2, iters: int = 3) -> Tuple[float, float]:
    """(mean ms, peak GiB) with the protocol of eval/bench_e2e.py:49-71:
    warm-up calls, synchronize, reset the peak, `iters` calls, synchronize."""
    out = None
    for _ in range(warmup):
        out = fn()
    torch.cuda.synchronize()
    del out
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats()
    t0 = time.perf_counter()
    out = None
    for _ in range(iters):
        del out
        out = fn()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / iters * 1e3
    peak = torch.cuda.max_memory_allocated() / 2 ** 30
    del out
    torch.cuda.empty_cache()
    return ms, peak


def aggregator_flops(cfg: GpaConfig, frames: int) -> Dict[str, float]:
    """Algorithmic FLOPs of one aggregator forward, by part (dense GEMMs,
    attention contractions, similarity); elementwise work is not counted."""
    C, P, Hd = cfg.embed_dim, cfg.tokens_per_frame, cfg.embed_dim // cfg.num_heads
    T = frames * P
    hid = int(C * cfg.mlp_ratio)
    dense_block = 2.0 * T * (3 * C * C + C * C + 2 * C * hid)
    frame_attn = 4.0 * frames * cfg.num_heads * P * P * Hd
    out = {"dense": dense_block * (cfg.vit_depth + 2 * cfg.depth)
           + 2.0 * frames * cfg.grid_h * cfg.grid_w * 3 * cfg.patch_size ** 2 * C,
           "frame_attn": frame_attn * (cfg.vit_depth + cfg.depth),
           "global_attn": 0.0, "similarity": 0.0}
    pts, gh, gw = cfg.num_special, cfg.grid_h, cfg.grid_w
    from merging.merge import num_dst_tokens
    for i in range(cfg.depth):
        kind = cfg.block_kind(i)
        if kind == "frame_special":
            kp = cfg.broadcast_pool
            if kp < 0:      # plain attention over each frame's own tokens
                out["global_attn"] += 4.0 * frames * cfg.num_heads * P * P * Hd
                continue
            npool = (-(-gh // kp)) * (-(-gw // kp)) if kp > 0 else 0
            out["global_attn"] += 4.0 * frames * cfg.num_heads * P * (P - pts) * Hd
            out["global_attn"] += 4.0 * cfg.num_heads * T * frames * (pts + npool) * Hd
        elif kind == "merged":
            nd = num_dst_tokens(frames, gw, gh, cfg.merge_grid, cfg.merge_grid, pts, False)
            ns = T - nd
            r = min(ns, int(T * cfg.block_merge_ratio(i)))
            out["global_attn"] += 4.0 * cfg.num_heads * T * (T - r) * Hd
            # The metric is projected to merge_metric_dim features only when
            # that is a reduction (merge.py:180); else the C-d cosine runs.
            projected = 0 < cfg.merge_metric_dim < C
            out["similarity"] += 2.0 * ns * nd * (cfg.merge_metric_dim if projected else C)
            if projected:
                out["dense"] += 2.0 * T * C * cfg.merge_metric_dim
        else:
            out["global_attn"] += 4.0 * cfg.num_heads * T * T * Hd
    return out
