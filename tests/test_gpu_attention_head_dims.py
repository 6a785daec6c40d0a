"""Biased attention at head dims other than 64 (16, 32, 128, 256): the
reference kernel takes HEAD_DIM as a constexpr and its wrapper reads it
from q (merging/fused_attention.py:82, 89, 97, 146, 177).  Checked against
the fp32 oracle on the same 16-bit inputs, output and log2 LSE, for both
operand formats, every bias kind, ragged query and key counts (partial
tiles, one key), sharp logits, a late key that moves the softmax offset of
the tiled kernel, and strided views (the allocation-free entry point at head
dim 128: test_zz_no_alloc.py); head dim 64 keeps the tuned kernel, so a
64-d slice of the same data must agree with the oracle to the same bar.

Bar: max-abs <= 2e-2 and mean-abs <= 2e-3 on unit-scale values; the LSE
within 2^-8 / ln 2 (the 16-bit P of the P.V product is not in the row sum
here, which follows the reference's fp32 sum, so the LSE bar is loose).
"""
import math

import pytest
import torch

from merging.fused_attention import attention_keybias
from oracle.attention import attention_reference

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3
LSE_TOL = 2.0 ** -8 / math.log(2.0) + 1e-5


def _inputs(B, H, M, N, D, seed, dtype, qk_scale=None, bias="bf16"):
    g = torch.Generator().manual_seed(seed)
    s = (0.5 if qk_scale is None else qk_scale) * (64.0 / D) ** 0.25   # logits of a similar spread
    q = (torch.randn(B, H, M, D, generator=g) * s).to(dtype)
    k = (torch.randn(B, H, N, D, generator=g) * s).to(dtype)
    v = torch.randn(B, H, N, D, generator=g).to(dtype)
    counts = torch.randint(1, 9, (B, 1, 1, N), generator=g).float()
    b = counts.log().expand(B, H, 1, N)
    if bias == "bf16":
        b = b.to(dtype).contiguous()
    elif bias == "f32":
        b = b.contiguous()
    elif bias == "none":
        b = None
    return q, k, v, b


def _check(dev, q, k, v, b, D, tight=True):
    o, lse = attention_keybias(q.to(dev), k.to(dev), v.to(dev), None if b is None else b.to(dev),
                               D ** -0.5, return_lse=True)
    assert o.shape == q.shape and o.dtype == q.dtype and lse.dtype == torch.float32
    ref, ref_lse = attention_reference(q, k, v, b, D ** -0.5)
    err = (o.float().cpu() - ref).abs()
    assert err.max().item() <= MAX_ABS, err.max().item()
    assert err.mean().item() <= (MEAN_ABS if tight else 5e-3), err.mean().item()
    # each row at its own scale too: |o - ref|_2 / |ref|_2 (16-bit P and output)
    rel = ((o.float().cpu() - ref).norm(dim=-1) / ref.norm(dim=-1)).max().item()
    assert rel <= 2e-2, rel
    assert (lse.cpu() - ref_lse).abs().max().item() < LSE_TOL
    return o


@pytest.mark.parametrize("D", [16, 32, 128, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,H,M,N,bias", [
    (1, 2, 300, 77, "bf16"), (2, 3, 129, 1000, "f32"), (1, 1, 5, 1, "none"), (1, 4, 1000, 333, "bf16"),
])
def test_head_dims_match_oracle(dev, D, dtype, B, H, M, N, bias):
    q, k, v, b = _inputs(B, H, M, N, D, seed=D + M + N, dtype=dtype, bias=bias)
    if b is not None and b.dtype != torch.float32:
        b = b.to(dtype)
    _check(dev, q, k, v, b, D)


@pytest.mark.parametrize("D", [32, 128])
def test_head_dims_sharp_logits(dev, D):
    """Logits spread over ~100 log2 units: the running max (16, 32) or the
    lazily moved offset (128) moves on late tiles and the rescale path
    carries the result."""
    q, k, v, b = _inputs(1, 2, 400, 2000, D, seed=5, dtype=torch.bfloat16, qk_scale=3.0)
    _check(dev, q, k, v, b, D)


@pytest.mark.parametrize("D", [16, 128])
def test_head_dims_strided_views(dev, D):
    """q, k, v as head-major views of one fused [B, N, 3, H, D] projection."""
    B, H, N = 1, 4, 700
    g = torch.Generator().manual_seed(D)
    qkv = (torch.randn(B, N, 3, H, D, generator=g) * 0.5).bfloat16()
    q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
    assert not q.is_contiguous()
    b = torch.randint(1, 5, (B, 1, 1, N), generator=g).float().log().expand(B, H, 1, N)
    _check(dev, q, k, v, b, D)


def test_head_dim_64_slice_agrees(dev):
    """The same data sliced to 64 features runs the tuned kernel: both meet
    the same bar against the oracle, so the two kernels share one contract."""
    q, k, v, b = _inputs(1, 2, 600, 900, 128, seed=9, dtype=torch.bfloat16)
    _check(dev, q, k, v, b, 128)
    _check(dev, q[..., :64].contiguous(), k[..., :64].contiguous(), v[..., :64].contiguous(), b, 64)


def test_head_dim_fp32_inputs_follow_the_cast_contract(dev):
    """fp32 q/k/v/bias are cast to bf16 first (fused_attention.py:139-144)."""
    q, k, v, b = _inputs(1, 2, 200, 300, 32, seed=3, dtype=torch.float32, bias="f32")
    o32 = attention_keybias(q.to(dev), k.to(dev), v.to(dev), b.to(dev), 32 ** -0.5)
    o16 = attention_keybias(q.to(dev).bfloat16(), k.to(dev).bfloat16(), v.to(dev).bfloat16(),
                            b.to(dev).bfloat16(), 32 ** -0.5)
    assert o32.dtype == torch.bfloat16
    assert torch.equal(o32, o16)


@pytest.mark.parametrize("D", [128, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rise", [20.0, 90.0])
def test_late_key_moves_the_offset(dev, D, dtype, rise):
    """Head dims 128 and 256 keep a softmax offset that moves only when a
    tile's row max rises more than 15 (fp16 P) or 64 (bf16 P) log2 units
    above it.  A key in the last tile aligned with every query lifts the row
    max ~`rise` log2 units above the earlier tiles, so the offset moves on a
    late tile (for fp16 at both rises, for bf16 at 90) and the output
    accumulated so far is rescaled; rows then concentrate on that key."""
    B, H, M, N = 1, 2, 256, 1000
    q, k, v, b = _inputs(B, H, M, N, D, seed=int(rise) + D, dtype=torch.float32, bias="f32")
    g = torch.Generator().manual_seed(D)
    u = torch.randn(D, generator=g)
    u /= u.norm()
    q = q + 2.0 * u                                   # every query has q.u ~ 2
    alpha = rise * D ** 0.5 / (2.0 * math.log2(math.e))
    k[:, :, N - 7] = alpha * u                        # score ~ rise log2 units
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    _check(dev, q, k, v, b, D, tight=False)


@pytest.mark.parametrize("D", [128, 256])
def test_rows_past_n_never_reach_the_output(dev, D):
    """k and v are views of longer buffers whose rows past N hold NaN: the
    tiled kernel's range-checked DMA must read zeros there (the last tile is
    partial, N = 1000 = 31 x 32 + 8), so the output equals that of
    contiguous copies bit for bit and matches the oracle."""
    B, H, M, N = 1, 2, 300, 1000
    q, k, v, b = _inputs(B, H, M, N, D, seed=D + 1, dtype=torch.bfloat16)
    kf = torch.full((B, H, N + 96, D), float("nan"), dtype=torch.bfloat16)
    vf = torch.full((B, H, N + 96, D), float("nan"), dtype=torch.bfloat16)
    kf[:, :, :N] = k
    vf[:, :, :N] = v
    kd, vd = kf.to(dev), vf.to(dev)
    o_view, lse_view = attention_keybias(q.to(dev), kd[:, :, :N], vd[:, :, :N], b.to(dev),
                                         D ** -0.5, return_lse=True)
    o_copy = _check(dev, q, k, v, b, D)
    assert torch.isfinite(o_view.float()).all() and torch.isfinite(lse_view).all()
    assert torch.equal(o_view.view(torch.int16), o_copy.view(torch.int16))
