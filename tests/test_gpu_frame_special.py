"""The frame-special split path on the gfx950 kernels (row f2).

vggt/layers/attention.py:148-176 attends every frame's queries to the
frame's own patch keys (bias None, return_lse) and all queries to a shared
key set (the special tokens of every frame plus pooled patch summaries, with
bias log(pool size), return_lse), then merges the two by their log2 LSE.
Checks:
  * `combine_by_lse` against the oracle's restatement of the merge
    (oracle.attention.lse_combine) on fp32 math, from arbitrary LSEs;
  * the whole split path against one fp32 attention per frame over the
    frame's full key set [own | specials | pooled] with the same bias (the
    reference's non-split fallback, :178-203) -- within the attention bar;
  * the 200-frame shapes (200 frames x 1374 tokens, 16 heads; 6,000 shared
    keys), on a sample of queries.
The pooling itself (the `_pool` assignment) is not on this path: the test
draws pooled keys and pool sizes directly.
"""
import math

import pytest
import torch

from merging.fused_attention import attention_keybias, combine_by_lse
from oracle.attention import attention_reference, lse_combine

pytestmark = pytest.mark.gpu

SCALE = 0.125


def _split_inputs(B, S, H, P, pts, npool, seed, scale=0.5, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    N = S * P
    q = (torch.randn(B, H, N, 64, generator=g) * scale).to(dtype)
    k = (torch.randn(B, H, N, 64, generator=g) * scale).to(dtype)
    v = torch.randn(B, H, N, 64, generator=g).to(dtype)
    pk = (torch.randn(B, H, S * npool, 64, generator=g) * scale).to(dtype)
    pv = torch.randn(B, H, S * npool, 64, generator=g).to(dtype)
    psize = torch.randint(1, 9, (B, H, S * npool), generator=g).float()
    return q, k, v, pk, pv, psize


def _split_path(q, k, v, pk, pv, psize, S, P, pts):
    """The split path of vggt/layers/attention.py:148-176 on the kernels."""
    B, H, N, D = q.shape
    q_f = q.view(B, H, S, P, D).permute(0, 2, 1, 3, 4).reshape(B * S, H, P, D)
    k5, v5 = k.view(B, H, S, P, D), v.view(B, H, S, P, D)
    own_k = k5[:, :, :, pts:].permute(0, 2, 1, 3, 4).reshape(B * S, H, P - pts, D)
    own_v = v5[:, :, :, pts:].permute(0, 2, 1, 3, 4).reshape(B * S, H, P - pts, D)
    out_a, lse_a = attention_keybias(q_f, own_k, own_v, None, SCALE, return_lse=True)
    sh_k = torch.cat([k5[:, :, :, :pts].reshape(B, H, S * pts, D), pk], dim=2)
    sh_v = torch.cat([v5[:, :, :, :pts].reshape(B, H, S * pts, D), pv], dim=2)
    sh_bias = torch.zeros(B, H, 1, sh_k.shape[2], device=q.device)
    sh_bias[:, :, 0, S * pts:] = psize.log()
    out_b, lse_b = attention_keybias(q, sh_k, sh_v, sh_bias.to(q.dtype), SCALE, return_lse=True)
    return combine_by_lse(out_a, lse_a, out_b, lse_b, S), (out_a, lse_a, out_b, lse_b)


def _full_reference(q, k, v, pk, pv, psize, S, P, pts, frames=None, rows=None):
    """fp32 attention per frame over [own | all specials | pooled] keys."""
    B, H, N, D = q.shape
    k5, v5 = k.view(B, H, S, P, D), v.view(B, H, S, P, D)
    sp_k = k5[:, :, :, :pts].reshape(B, H, S * pts, D)
    sp_v = v5[:, :, :, :pts].reshape(B, H, S * pts, D)
    outs = {}
    for f in (range(S) if frames is None else frames):
        qf = q.view(B, H, S, P, D)[:, :, f]
        if rows is not None:
            qf = qf[:, :, rows]
        kf = torch.cat([k5[:, :, f, pts:], sp_k, pk], dim=2)
        vf = torch.cat([v5[:, :, f, pts:], sp_v, pv], dim=2)
        bias = torch.zeros(B, H, 1, kf.shape[2])
        bias[:, :, 0, kf.shape[2] - pk.shape[2]:] = psize.log()
        o, _ = attention_reference(qf, kf, vf, bias.to(q.dtype), SCALE)
        outs[f] = o                                  # [B, H, rows, D]
    return outs


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,S,H,P,pts,npool", [(1, 4, 2, 41, 5, 9), (2, 3, 3, 70, 5, 16),
                                                (1, 6, 4, 1374, 5, 25)])
def test_split_path_matches_full_attention(dev, B, S, H, P, pts, npool, dtype):
    """bf16, and fp16 as under the fp16-autocast evaluation stack (the
    attention kernels and the combine all in fp16)."""
    q, k, v, pk, pv, psize = _split_inputs(B, S, H, P, pts, npool, seed=S * P + H, dtype=dtype)
    y, _ = _split_path(q.to(dev), k.to(dev), v.to(dev), pk.to(dev), pv.to(dev), psize.to(dev),
                       S, P, pts)
    assert y.shape == (B, S * P, H * 64) and y.dtype == dtype
    ref = _full_reference(q, k, v, pk, pv, psize, S, P, pts)
    yc = y.float().cpu().view(B, S, P, H, 64)
    errs = [(yc[:, f].permute(0, 2, 1, 3) - ref[f]).abs() for f in range(S)]
    err = torch.stack(errs)
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3, (err.max(), err.mean())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_combine_matches_oracle(dev, dtype):
    g = torch.Generator().manual_seed(9)
    B, S, H, P, D = 2, 3, 4, 50, 64
    N = S * P
    out_a = torch.randn(B * S, H, P, D, generator=g).to(dtype)
    out_b = torch.randn(B, H, N, D, generator=g).to(dtype)
    lse_a = torch.randn(B * S, H, P, generator=g) * 20
    lse_b = torch.randn(B, H, N, generator=g) * 20
    y = combine_by_lse(out_a.to(dev), lse_a.to(dev), out_b.to(dev), lse_b.to(dev), S).cpu()
    oa = out_a.float().view(B, S, H, P, D).permute(0, 2, 1, 3, 4).reshape(B, H, N, D)
    la = lse_a.view(B, S, H, P).permute(0, 2, 1, 3).reshape(B, H, N)
    ref = lse_combine(oa, la, out_b.float(), lse_b).transpose(1, 2).reshape(B, N, H * D)
    assert y.dtype == dtype
    err = (y.float() - ref).abs()
    # one rounding to the output format of values of magnitude <~ 4
    ulp = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    assert err.max().item() <= ulp * ref.abs().max().item() + 1e-6


def test_combine_accepts_strided_views(dev):
    g = torch.Generator().manual_seed(10)
    B, S, H, P, D = 1, 2, 2, 40, 64
    N = S * P
    out_a = torch.randn(B * S, P, H, D, generator=g).bfloat16().to(dev).transpose(1, 2)
    out_b = torch.randn(B, N, H, D, generator=g).bfloat16().to(dev).transpose(1, 2)
    lse_a = torch.randn(B * S, P, H, generator=g).to(dev).transpose(1, 2)
    lse_b = torch.randn(B, N, H, generator=g).to(dev).transpose(1, 2)
    y1 = combine_by_lse(out_a, lse_a, out_b, lse_b, S)
    y2 = combine_by_lse(out_a.contiguous(), lse_a.contiguous(), out_b.contiguous(),
                        lse_b.contiguous(), S)
    assert torch.equal(y1, y2)


def test_combine_argument_checks(dev):
    oa = torch.zeros(4, 2, 10, 64, device=dev, dtype=torch.bfloat16)
    la = torch.zeros(4, 2, 10, device=dev)
    ob = torch.zeros(2, 2, 20, 64, device=dev, dtype=torch.bfloat16)
    lb = torch.zeros(2, 2, 20, device=dev)
    combine_by_lse(oa, la, ob, lb, 2)
    with pytest.raises(ValueError):
        combine_by_lse(oa, la, ob, lb, 3)                  # frames do not divide
    with pytest.raises(ValueError):
        combine_by_lse(oa.float(), la, ob, lb, 2)          # dtype
    with pytest.raises(ValueError):
        combine_by_lse(oa.half(), la, ob, lb, 2)           # mixed bf16 / fp16


def test_200_frame_shapes_on_a_sample(dev):
    """Own-frame attention [3200 x 1374 x 1369] and shared attention
    [16 x 274,800 x 6,000] at the 200-frame shapes; checked on 3 frames."""
    B, S, H, P, pts, npool = 1, 200, 16, 1374, 5, 25
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    N = S * P
    q = (torch.randn(B, H, N, 64, generator=g, device=dev) / 8).bfloat16()
    k = (torch.randn(B, H, N, 64, generator=g, device=dev) / 8).bfloat16()
    v = (torch.randn(B, H, N, 64, generator=g, device=dev) / 8).bfloat16()
    pk = (torch.randn(B, H, S * npool, 64, generator=g, device=dev) / 8).bfloat16()
    pv = (torch.randn(B, H, S * npool, 64, generator=g, device=dev) / 8).bfloat16()
    psize = torch.randint(1, 12, (B, H, S * npool), generator=g, device=dev).float()
    y, (out_a, lse_a, out_b, lse_b) = _split_path(q, k, v, pk, pv, psize, S, P, pts)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all() and torch.isfinite(lse_a).all() and torch.isfinite(lse_b).all()
    frames = [0, 117, 199]
    rows = torch.cat([torch.arange(8), torch.arange(P - 8, P)])
    ref = _full_reference(q.cpu(), k.cpu(), v.cpu(), pk.cpu(), pv.cpu(), psize.cpu(), S, P, pts,
                          frames=frames, rows=rows)
    yc = y.float().cpu().view(B, S, P, H, 64)
    for f in frames:
        got = yc[:, f, rows].permute(0, 2, 1, 3)
        err = (got - ref[f]).abs()
        # Outputs here are ~1e-2 (v ~ N(0, 1/64)): each row is also held to
        # its own scale, |y - ref|_2 / |ref|_2.
        rel = ((got - ref[f]).norm(dim=-1) / ref[f].norm(dim=-1)).max().item()
        print(f"[frame special 200f] frame {f}: max-abs {err.max().item():.2e}, worst row "
              f"relative {rel:.2e}", flush=True)
        assert err.max().item() <= 2e-2 and err.mean().item() <= 5e-3, (f, err.max())
        assert rel <= 2e-2, (f, rel)
