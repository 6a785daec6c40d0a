"""The fused residual + LayerScale + LayerNorm kernel (gpa::residual_layernorm)
against the torch op sequence of vggt/layers/block.py:84-96 under bf16
autocast on a bf16 block (and the same under fp16 autocast on an fp16
block, in fp16 ulps): `x + ls(y)` in bf16 (bit-identical: the same two
roundings), and `layer_norm` in fp32 cast to bf16 (almost every element
bit-identical, the rest one bf16 ulp apart -- or 1e-5 where the bias cancels
the normalised value -- from the order of the moment sums; and within 2^-8
relative of fp64 LayerNorm of the same h).  Widths
512..4096, ragged row counts, strided rows; and a whole harness block with
the fused path against the torch path.
"""
import pytest
import torch
import torch.nn.functional as F

import gpa_aggregator as A

pytestmark = pytest.mark.gpu


def _ordered(t):
    v = t.contiguous().view(torch.int16).int()
    return torch.where(v < 0, -(v & 0x7FFF), v)


def _params(C, dev, seed, dt=torch.bfloat16):
    g = torch.Generator(device=dev).manual_seed(seed)
    gamma = (torch.randn(C, generator=g, device=dev) * 0.1).to(dt)
    w = (1 + 0.3 * torch.randn(C, generator=g, device=dev)).to(dt)
    b = (0.2 * torch.randn(C, generator=g, device=dev)).to(dt)
    return gamma, w, b


# ulp of the 16-bit format, relative: bf16 2^-7, fp16 2^-10
_ULP = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,C,stride", [(1, 512, 512), (7, 1024, 1024), (4099, 1024, 1152),
                                           (301, 1536, 1536), (65, 4096, 4096)])
def test_matches_the_autocast_chain(dev, rows, C, stride, dt):
    """bf16 rows under bf16 autocast, and fp16 rows under fp16 autocast (the
    accuracy-evaluation stack)."""
    g = torch.Generator(device=dev).manual_seed(rows + C)
    xs = (torch.randn(rows, stride, generator=g, device=dev) * 2 + 0.5).to(dt)
    ys = torch.randn(rows, stride, generator=g, device=dev).to(dt)
    x, y = xs[:, :C], ys[:, :C]
    gamma, w, b = _params(C, dev, rows, dt)
    eps = 1e-6
    h, ln = torch.ops.gpa.residual_layernorm(x, y, gamma, w, b, eps, True)
    with torch.autocast("cuda", dtype=dt):
        h_ref = x + y * gamma
        ln_ref = F.layer_norm(h_ref, (C,), w, b, eps)           # fp32 under autocast
    assert h_ref.dtype == dt and ln_ref.dtype == torch.float32
    assert h.dtype == ln.dtype == dt
    assert torch.equal(h, h_ref)
    ln_ref16 = ln_ref.to(dt)
    ulps = (_ordered(ln) - _ordered(ln_ref16)).abs()
    print(f"\n[ln {rows}x{C}] max ulps {ulps.max().item()} differing "
          f"{(ulps > 0).float().mean().item():.2e}")
    # one ulp of the format, or 1e-5 absolute where b cancels the normalised
    # value and fp32 last-bit differences exceed a tiny result's ulp
    diff = (ln.float() - ln_ref16.float()).abs()
    assert (diff <= _ULP[dt] * ln_ref16.float().abs() + 1e-5).all()
    assert (ulps > 0).float().mean().item() <= 1e-2
    h64 = h.double()
    mu = h64.mean(-1, keepdim=True)
    var = ((h64 - mu) ** 2).mean(-1, keepdim=True)
    ref64 = (h64 - mu) / torch.sqrt(var + eps) * w.double() + b.double()
    assert ((ln.double() - ref64).abs() <= _ULP[dt] / 2 * ref64.abs() + 1e-3).all()
    # the other two modes: LayerNorm alone, residual alone
    _, ln1 = torch.ops.gpa.residual_layernorm(x, None, None, w, b, eps, False)
    with torch.autocast("cuda", dtype=dt):
        ln1_ref = F.layer_norm(x, (C,), w, b, eps).to(dt)
    assert ((ln1.float() - ln1_ref.float()).abs() <= _ULP[dt] * ln1_ref.float().abs() + 1e-5).all()
    h2, empty = torch.ops.gpa.residual_layernorm(x, y, gamma, None, None, 0.0, True)
    assert torch.equal(h2, h_ref) and empty.numel() == 0


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_harness_block_fused_equals_torch_path(dev, dt):
    """One frame block at VGGT width, 3 frames: the fused block against the
    torch-op block (same weights), both under autocast to the block's dtype."""
    cfg = A.GpaConfig(vit_depth=0, depth=1)
    blk = A.Block(1024, 16, 4.0, 0.01, True, 1e-6, cfg).to(dev)
    A.init_random_(blk, seed=3)
    with torch.no_grad():
        blk.ls1.gamma.normal_(0.0, 0.5)
        blk.ls2.gamma.normal_(0.0, 0.5)
    blk = blk.to(dt).eval()
    S, P = 3, cfg.tokens_per_frame
    x = (torch.randn(S, P, 1024, device=dev) * 0.7).to(dt)
    rope = A.Rope2D(100.0).table(A.frame_positions(cfg.grid, cfg.num_special, dev), 64)
    with torch.no_grad(), torch.autocast("cuda", dtype=dt):
        fused = blk(x, rope)
        cfg.fused_norms = False
        plain = blk(x, rope)
        cfg.fused_norms = True
    assert fused.dtype == plain.dtype == dt
    d = (fused.float() - plain.float()).abs()
    rel = d.max().item() / plain.float().abs().max().item()
    print(f"\n[block] max |fused - torch| {d.max().item():.3e} (rel {rel:.2e}), "
          f"mean {d.mean().item():.3e}")
    assert rel < 2e-2 and d.mean().item() < 2e-3 * plain.float().abs().mean().item() + 1e-4
