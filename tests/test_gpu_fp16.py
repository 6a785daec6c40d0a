"""The fp16 twins of the similarity and attention kernels.

The reference's accuracy evaluation runs the model under fp16 autocast
(eval_co3d.py:226): attention_keybias then receives fp16 q, k, v
(fused_attention.py:139-144), and fused_similarity_argmax passes fp16
operands to its kernel as they are (fused_similarity.py:81-112 casts only an
fp32 `a`).

Similarity: max within 1e-5 of fp64 on the same fp16 values, index equal to
the fp64 argmax wherever the top-2 gap exceeds 1e-5, ties to the lowest
index.

Attention: against the fp32 reference on the same fp16 values, the parity
bars (max-abs 2e-2, mean-abs 5e-3); and, since P is rounded to fp16 (11
significant bits) instead of bf16 (8), an error well below the bf16
kernel's on inputs both formats hold exactly -- which a path that silently
ran bf16 would not show.  The log2 LSE sums fp16-rounded probabilities:
within 2^-10 / ln 2 of the fp32 one.  Edge cases: waves routed to the
lazily moved offset, logits that raise the row max on every tile (lazy
rescale at 2^15), a
row whose max meets the score bound (largest P = 2^15, no overflow), an
fp16 bias, the fp32-input cast under fp16 autocast.
"""
import numpy as np
import pytest
import torch

from merging import _native
from merging.fused_attention import attention_keybias
from merging.fused_similarity import fused_similarity_argmax
from oracle.attention import attention_reference

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 5e-3


def _worst_row_rel(o, ref):
    """Largest |o - ref|_2 / |ref|_2 over the rows: each row at its own scale."""
    got = o.float().cpu()
    return ((got - ref).norm(dim=-1) / ref.norm(dim=-1)).max().item()
LSE_TOL16 = 2.0 ** -10 / 0.6931471805599453 + 1e-5


def _unit_f16(shape, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    return (x / x.norm(dim=-1, keepdim=True)).half()


def _fp64_argmax(a, b):
    a64, b64 = a.double().numpy(), b.double().numpy()
    s = np.einsum("bmd,bnd->bmn", a64, b64)
    idx = s.argmax(-1)
    top = np.take_along_axis(s, idx[..., None], -1)[..., 0]
    if s.shape[-1] > 1:
        np.put_along_axis(s, idx[..., None], -np.inf, -1)
        gap = top - s.max(-1)
    else:
        gap = np.full(top.shape, np.inf)
    return top, idx, gap


@pytest.mark.parametrize("B,M,N,D", [
    (1, 5, 17, 64), (2, 257, 100, 128), (1, 1000, 513, 256), (1, 3000, 4000, 128),
    (1, 700, 20_000, 128),
])
def test_similarity_f16_matches_fp64(dev, B, M, N, D):
    a = _unit_f16((B, M, D), seed=M + N)
    b = _unit_f16((B, N, D), seed=M + N + 1)
    vmax, vidx = torch.ops.gpa.sim_argmax(a.to(dev), b.to(dev))      # fp32 max
    fmax, fidx, gap = _fp64_argmax(a, b)
    assert np.abs(vmax.cpu().numpy() - fmax).max() < 1e-5
    sure = gap > 1e-5
    assert sure.mean() > 0.9
    assert np.array_equal(vidx.cpu().numpy()[sure], fidx[sure])
    # the wrapper's contract: max in a's dtype, int64 indices
    wmax, widx = fused_similarity_argmax(a.to(dev), b.to(dev))
    assert wmax.dtype == torch.float16 and widx.dtype == torch.int64
    assert torch.equal(widx, vidx)


def test_similarity_f16_ties_and_dtype_errors(dev):
    base = _unit_f16((1, 40, 128), seed=3)
    b = _unit_f16((1, 3000, 128), seed=4)
    slots = torch.randperm(3000, generator=torch.Generator().manual_seed(5))[:120].view(3, 40)
    slots = slots.sort(dim=0).values
    for c in range(3):
        b[0, slots[c]] = base[0]
    _, vidx = fused_similarity_argmax(base.to(dev), b.to(dev))
    assert torch.equal(vidx[0].cpu(), slots[0])
    with pytest.raises(ValueError):
        fused_similarity_argmax(base.to(dev), b.to(dev).bfloat16())


def _common_values(shape, seed, scale):
    """Values exactly representable in both bf16 and fp16."""
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(*shape, generator=g) * scale).bfloat16().float()
    x[x.abs() < 2.0 ** -14] = 0.0
    assert torch.equal(x.half().float(), x)
    return x


def _attn_inputs(B, H, M, N, seed, qk_scale=0.5):
    q = _common_values((B, H, M, 64), seed, qk_scale)
    k = _common_values((B, H, N, 64), seed + 1, qk_scale)
    v = _common_values((B, H, N, 64), seed + 2, 1.0)
    counts = torch.randint(1, 9, (B, 1, 1, N), generator=torch.Generator().manual_seed(seed))
    bias = counts.float().log().half().float().expand(B, H, 1, N).contiguous()
    return q, k, v, bias


def _run(q, k, v, bias, dtype, dev, scale=0.125, lse=True):
    b = None if bias is None else bias.to(dev, dtype)
    return attention_keybias(q.to(dev, dtype), k.to(dev, dtype), v.to(dev, dtype), b, scale,
                             return_lse=lse)


@pytest.mark.parametrize("B,H,M,N", [
    (1, 1, 1, 1), (1, 2, 37, 31), (2, 3, 257, 100), (1, 2, 1000, 1000), (1, 16, 513, 2049),
])
@pytest.mark.parametrize("with_bias", [True, False])
def test_attention_f16_matches_reference_and_beats_bf16(dev, B, H, M, N, with_bias):
    q, k, v, bias = _attn_inputs(B, H, M, N, seed=M + N + H)
    if not with_bias:
        bias = None
    ref, ref_lse = attention_reference(q, k, v, bias, 0.125)
    o16, l16 = _run(q, k, v, bias, torch.float16, dev)
    assert o16.dtype == torch.float16 and l16.dtype == torch.float32
    err16 = (o16.float().cpu() - ref).abs()
    assert err16.max().item() <= MAX_ABS and err16.mean().item() <= MEAN_ABS
    assert _worst_row_rel(o16, ref) <= 2e-2
    assert (l16.cpu() - ref_lse).abs().max().item() < LSE_TOL16
    obf, _ = _run(q, k, v, bias, torch.bfloat16, dev)
    errbf = (obf.float().cpu() - ref).abs()
    print(f"\n[fp16 attention {B}x{H}x{M}x{N}] mean err fp16 {err16.mean().item():.2e} "
          f"bf16 {errbf.mean().item():.2e}")
    if M * N > 1000:
        assert err16.mean().item() < 0.5 * errbf.mean().item()


@pytest.mark.parametrize("lse", [False, True])
def test_attention_f16_fixed_and_lazy_offset_waves_mix(dev, lse):
    """Rows whose score bound sits far above their scores cannot keep the
    bound-certified offset (with fp16's 16-unit window more rows do): their
    waves take the tile-0 offset (verified after the loop) or the lazily
    moved one.  The flags name the waves; the outputs match either way."""
    g = torch.Generator().manual_seed(11)
    M, N = 600, 1000
    q = torch.randn(1, 2, M, 64, generator=g) * 0.3
    k = torch.randn(1, 2, N, 64, generator=g) * 0.3
    k[:, :, :32] *= -1.0
    boost = torch.zeros(M, dtype=torch.bool)
    boost[32:64] = True
    boost[[5, 300, 555]] = True
    q[:, :, boost] = k[:, :, 40:41].expand(-1, -1, int(boost.sum()), -1) * 20.0
    q, k = q.half().float(), k.half().float()
    v = torch.randn(1, 2, N, 64, generator=g).half().float()
    bias = torch.randn(1, 1, 1, N, generator=g).half().float()
    out = _run(q, k, v, bias, torch.float16, dev, lse=lse)
    o = out[0] if lse else out
    ref, ref_lse = attention_reference(q, k, v, bias, 0.125)
    err = (o.float().cpu() - ref).abs()
    assert err.max().item() <= MAX_ABS and err.mean().item() <= MEAN_ABS
    assert _worst_row_rel(o, ref) <= 2e-2
    if lse:
        assert (out[1].cpu() - ref_lse).abs().max().item() < LSE_TOL16
    _, _, flags = _native.attn_keybias_offset_flags(
        q.to(dev, torch.float16), k.to(dev, torch.float16), v.to(dev, torch.float16),
        bias.to(dev, torch.float16), 0.125)
    for wg, row in ((0, 32), (1, 300 - 256), (2, 555 - 512)):       # the boosted rows' waves
        assert ((flags[:, wg, row // 64] &
                 (_native.ATTN_FLAG_LAZY | _native.ATTN_FLAG_TILE0)) != 0).all()


def test_attention_f16_increasing_logits_rescale(dev):
    """Each tile raises the row max (logits over ~46 log2 units): the bound is
    far above tile 0, so the wave runs the lazily moved offset and rescales
    whenever a tile's max passes m + 15."""
    g = torch.Generator().manual_seed(4)
    n = 1024
    q = torch.ones(1, 1, 64, 64)
    k = torch.zeros(1, 1, n, 64)
    k[..., 0] = torch.linspace(-4, 4, n)
    k = k.half().float()
    v = torch.randn(1, 1, n, 64, generator=g).half().float()
    o, lse = _run(q, k, v, None, torch.float16, dev, scale=4.0)
    ref, ref_lse = attention_reference(q, k, v, None, 4.0)
    err = (o.float().cpu() - ref).abs()
    assert torch.isfinite(o).all()
    assert err.max().item() <= MAX_ABS and err.mean().item() <= MEAN_ABS
    assert _worst_row_rel(o, ref) <= 2e-2
    assert (lse.cpu() - ref_lse).abs().max().item() < LSE_TOL16


def test_attention_f16_row_max_at_the_bound(dev):
    """q parallel to the longest key: its score equals the Cauchy-Schwarz
    bound, so the largest probability is 2^15 in fp16 -- finite, and the
    output follows the reference."""
    g = torch.Generator().manual_seed(6)
    n = 500
    k = torch.randn(1, 1, n, 64, generator=g) * 0.5
    k[0, 0, 123] = k[0, 0, 123] / k[0, 0, 123].norm() * 6.0     # the longest key
    q = k[:, :, 123:124].expand(1, 1, 256, 64) * torch.linspace(0.1, 1.5, 256).view(1, 1, 256, 1)
    q, k = q.half().float(), k.half().float()
    v = torch.randn(1, 1, n, 64, generator=g).half().float()
    o, lse = _run(q, k, v, None, torch.float16, dev)
    ref, ref_lse = attention_reference(q, k, v, None, 0.125)
    assert torch.isfinite(o).all() and torch.isfinite(lse).all()
    err = (o.float().cpu() - ref).abs()
    assert err.max().item() <= MAX_ABS and err.mean().item() <= MEAN_ABS
    assert _worst_row_rel(o, ref) <= 2e-2
    assert (lse.cpu() - ref_lse).abs().max().item() < LSE_TOL16


def test_attention_f16_bias_kinds_and_autocast_cast(dev):
    q, k, v, bias = _attn_inputs(1, 2, 300, 400, seed=7)
    qd, kd, vd = q.to(dev, torch.float16), k.to(dev, torch.float16), v.to(dev, torch.float16)
    o32b = attention_keybias(qd, kd, vd, bias.to(dev), 0.125)                  # fp32 bias
    o16b = attention_keybias(qd, kd, vd, bias.to(dev, torch.float16), 0.125)   # fp16 bias
    assert torch.equal(o32b, o16b)
    # fp32 q/k/v under fp16 autocast take the fp16 kernel (fused_attention.py:139-144)
    with torch.autocast("cuda", dtype=torch.float16):
        oa = attention_keybias(q.to(dev), k.to(dev), v.to(dev), bias.to(dev), 0.125)
    assert oa.dtype == torch.float16 and torch.equal(oa, o16b)
