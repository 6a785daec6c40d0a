"""token_merge_bipartite2d on the GPU against the oracle's restatement.

The window cells and the projection basis come from the device generators
(as in the reference, merging/merge.py:121-126, :181-184); the test draws
them the same way and hands them to the CPU restatement.  Given identical
node indices, the merge assignment and slot counts must be bit-exact; the
node indices themselves follow the similarity gap rule.
"""
import numpy as np
import pytest
import torch

import gpa_workloads as W
from merging.fused_attention import attention_keybias
from merging.merge import token_merge_bipartite2d
from oracle.attention import attention_reference
from oracle.merge import merge_heads_fp64, projection_basis, token_merge_reference, window_draw
from oracle.similarity import bf16_top2_gap

pytestmark = pytest.mark.gpu


def _device_draws(dev, frames, w, h, sx, sy, c, mdim, no_rand):
    gen = torch.Generator(device=dev)
    gen.manual_seed(33)
    cell = window_draw(frames, w, h, sx, sy, gen, device=dev) if frames > 1 and not no_rand else None
    proj = projection_basis(c, mdim, device=dev) if mdim and mdim < c else None
    return (None if cell is None else cell.cpu()), (None if proj is None else proj.cpu())


@pytest.mark.parametrize("frames,w,h,sx,sy,ns,c,mdim,ratio,no_rand", [
    (4, 37, 37, 2, 2, 5, 1024, 128, 0.98, False),
    (4, 37, 37, 2, 2, 5, 1024, 128, 0.2, False),
    (6, 9, 7, 2, 2, 5, 256, 64, 0.5, False),
    (3, 8, 8, 2, 2, 5, 128, 0, 0.98, True),
    (4, 10, 8, 3, 2, 3, 128, 32, 0.6, False),      # 3 x 2 windows, ragged grid edges
    (3, 9, 9, 3, 3, 1, 256, 128, 0.98, False),     # 3 x 3 windows, one special token
])
def test_merge_indices_bit_exact_given_node_indices(dev, frames, w, h, sx, sy, ns, c, mdim,
                                                    ratio, no_rand):
    n = frames * (w * h + ns)
    metric = W.shifted_basis_tokens(frames, dim=c, seed=frames)[:, :n] if w == 37 else \
        torch.randn(1, n, c, generator=torch.Generator().manual_seed(frames))
    r = int(n * ratio)
    gen = torch.Generator(device=dev)
    gen.manual_seed(33)
    m = token_merge_bipartite2d(metric.to(dev), w, h, sx, sy, r, no_rand, gen, metric_dim=mdim,
                                num_special=ns)
    ix = m.index
    cell, proj = _device_draws(dev, frames, w, h, sx, sy, c, mdim, no_rand)
    node = (ix.node_max.cpu(), ix.node_idx.cpu())
    o = token_merge_reference(metric, w, h, sx, sy, r, no_rand, None, mdim, ns, cell=cell,
                              proj=proj, sim=lambda a, b: node, stable=True)
    assert torch.equal(ix.mask.cpu(), o.mask)
    assert torch.equal(ix.a_idx.cpu(), o.a_idx) and torch.equal(ix.b_idx.cpu(), o.b_idx)
    assert torch.equal(ix.dst_idx.cpu(), o.dst_idx)
    assert torch.equal(ix.unm_abs_idx.cpu(), o.unm_abs_idx)
    assert torch.equal(ix.src_abs_idx.cpu(), o.src_abs_idx)
    assert torch.equal(m.size.cpu(), o.size)
    assert m.size.sum().item() == n and (m.size >= 1).all()

    # The node indices themselves: the reference torch path on the same
    # projected metric, under the bf16 top-2 gap rule.
    o_ref = token_merge_reference(metric, w, h, sx, sy, r, no_rand, None, mdim, ns, cell=cell,
                                  proj=proj, stable=True)
    x = metric @ proj if proj is not None else metric
    x = x / x.norm(dim=-1, keepdim=True)
    gap = bf16_top2_gap(x[:, o.a_idx], x[:, o.b_idx])
    keep = gap >= 1e-3
    assert torch.equal(ix.node_idx.cpu()[keep], o_ref.node_idx[keep])


def test_merge_heads_means(dev):
    frames, w, h, ns = 4, 37, 37, 5
    n = frames * (w * h + ns)
    metric = W.shifted_basis_tokens(frames, seed=0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(33)
    m = token_merge_bipartite2d(metric.to(dev), w, h, 2, 2, int(0.98 * n), False, gen,
                                metric_dim=128, num_special=ns)
    g = torch.Generator().manual_seed(1)
    k = torch.randn(1, 4, n, 64, generator=g)
    v = torch.randn(1, 4, n, 64, generator=g).bfloat16()
    ix = m.index
    args = (ix.unm_abs_idx[0].cpu().numpy(), ix.b_idx.cpu().numpy(),
            ix.src_abs_idx[0].cpu().numpy(), ix.dst_idx[0].cpu().numpy())
    km = m.heads(k.to(dev), "mean")[0].cpu().numpy()
    vm = m.heads(v.to(dev), "mean")[0].float().cpu().numpy()
    np.testing.assert_allclose(km, merge_heads_fp64(k[0].numpy(), *args), rtol=0, atol=2e-6)
    # bf16 storage: the fp32 mean is rounded once to bf16 (half an ulp, 2^-9 relative)
    v_ref = merge_heads_fp64(v[0].float().numpy(), *args)
    assert (np.abs(vm - v_ref) <= 2.0 ** -8 * np.abs(v_ref) + 1e-6).all()
    # Deterministic: a second merge of the same tensor is bit-identical.
    assert torch.equal(m.heads(v.to(dev), "mean"), m.heads(v.to(dev), "mean"))
    # merge(x) (token-major, H = 1) is the same reduction.
    x = torch.randn(1, n, 96, generator=g)
    np.testing.assert_allclose(m(x.to(dev), "mean")[0].cpu().numpy(),
                               merge_heads_fp64(x[0].numpy()[None], *args)[0], rtol=0, atol=2e-6)


def test_config1_end_to_end(dev):
    """4 frames x 1374 tokens, width 1024, 16 heads: merge K/V then biased attention."""
    frames, w, h, ns, H = 4, 37, 37, 5, 16
    n = frames * (w * h + ns)
    x = W.shifted_basis_tokens(frames, seed=0)
    g = torch.Generator().manual_seed(2)
    q = torch.randn(1, H, n, 64, generator=g) * 0.5
    k = torch.randn(1, H, n, 64, generator=g) * 0.5
    v = torch.randn(1, H, n, 64, generator=g)
    r = int(n * 0.98)
    gen = torch.Generator(device=dev)
    gen.manual_seed(33)
    m = token_merge_bipartite2d(x.to(dev), w, h, 2, 2, r, False, gen, metric_dim=128,
                                num_special=ns)
    km = m.heads(k.to(dev), "mean")
    vm = m.heads(v.to(dev), "mean")
    bias = m.size.reshape(1, 1, 1, -1).log().expand(1, H, 1, km.shape[2]).contiguous()
    o = attention_keybias(q.to(dev), km, vm, bias, 0.125)
    # Oracle: same draws, same node indices, fp32 attention on the same bf16-cast inputs.
    cell, proj = _device_draws(dev, frames, w, h, 2, 2, 1024, 128, False)
    ix = m.index
    node = (ix.node_max.cpu(), ix.node_idx.cpu())
    ref = token_merge_reference(x, w, h, 2, 2, r, False, None, 128, ns, cell=cell, proj=proj,
                                sim=lambda a, b: node, stable=True)
    assert torch.equal(m.size.cpu(), ref.size)
    k_ref, v_ref = ref.heads(k, "mean"), ref.heads(v, "mean")
    b_ref = ref.size.reshape(1, 1, 1, -1).log()
    o_ref, _ = attention_reference(q.bfloat16(), k_ref.bfloat16(), v_ref.bfloat16(),
                                   b_ref.bfloat16(), 0.125)
    err = (o.float().cpu() - o_ref).abs()
    print(f"\n[config1] N_m={km.shape[2]} max-abs {err.max().item():.3e} "
          f"mean-abs {err.mean().item():.3e}")
    assert err.max().item() <= 2e-2 and err.mean().item() <= 5e-3


@pytest.mark.parametrize("mdim", [128, 0])
def test_batched_merge_equals_per_element_merges(dev, mdim):
    """A batch of two scenes (the reference takes B > 1, merging/merge.py:
    39-256; `merge.size` is then None and the caller sums ones,
    vggt/layers/attention.py:250-253): every batch element's merge equals
    the merge of that element alone, bit for bit (node indices, assignment,
    merged K/V), and the summed sizes equal the single-scene sizes."""
    frames, w, h, ns, c = 3, 37, 37, 5, 1024
    n = frames * (w * h + ns)
    metric = torch.cat([W.shifted_basis_tokens(frames, dim=c, seed=s)[:, :n] for s in (3, 4)])
    r = int(0.98 * n)

    def merged(x):
        gen = torch.Generator(device=dev)
        gen.manual_seed(33)
        return token_merge_bipartite2d(x.to(dev), w, h, 2, 2, r, False, gen, metric_dim=mdim,
                                       num_special=ns)

    mb = merged(metric)
    assert mb.size is None
    g = torch.Generator().manual_seed(5)
    k = torch.randn(2, 4, n, 64, generator=g).to(dev)
    v = torch.randn(2, 4, n, 64, generator=g).bfloat16().to(dev)
    kb, vb = mb.heads(k, "mean"), mb.heads(v, "mean")
    sizes = mb(torch.ones(2, n, 1, device=dev), "sum")[..., 0]
    for e in range(2):
        m1 = merged(metric[e:e + 1])
        for name in ("node_idx", "dst_idx", "unm_abs_idx", "src_abs_idx"):
            assert torch.equal(getattr(mb.index, name)[e], getattr(m1.index, name)[0]), name
        assert torch.equal(sizes[e], m1.size[0])
        assert torch.equal(kb[e], m1.heads(k[e:e + 1], "mean")[0])
        assert torch.equal(vb[e], m1.heads(v[e:e + 1], "mean")[0])
