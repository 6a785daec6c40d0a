"""The fused merge front end (`gpa::merge_metric`) on the GPU.

Two independent checks of the same kernel output:
* against the torch op sequence it replaces (merging/merge.py:180-187 under
  bf16 autocast, then the bf16 cast of fused_similarity.py:90-95; or the
  same sequence on a bf16 metric without autocast): almost all elements
  bit-identical and the rest within 2^-6 relative (a y rounded to the
  neighbouring bf16 value, then the output's own rounding; plus an absolute
  floor for elements that cancel to near zero) -- the projection's
  accumulation order is the only freedom, so a rounding point moved or
  dropped (y not rounded before the norm, the norm rounded in the wrong
  mode) shows up as a mass of one-ulp differences;
* against fp64 arithmetic on the same bf16 operands (catches a transposed
  projection, a wrong gather or a missing normalisation): within 3 * 2^-8
  relative (the chain's two bf16 roundings), with the same floor.
"""
import numpy as np
import pytest
import torch

import gpa_workloads as W
from merging import _native
from merging.merge import _projection, dst_mask, num_dst_tokens, token_merge_bipartite2d
from oracle.similarity import bf16_top2_gap, fast_similarity_chunks

pytestmark = pytest.mark.gpu


def _torch_chain(metric, proj_f32, order, autocast, dtype=torch.bfloat16):
    if autocast:
        with torch.autocast("cuda", dtype=dtype):
            m = metric @ proj_f32.to(metric.dtype)
            m = m / m.norm(dim=-1, keepdim=True)
        return m.index_select(1, order).to(torch.bfloat16)
    m = metric @ proj_f32.to(metric.dtype)
    m = m / m.norm(dim=-1, keepdim=True)
    return m.index_select(1, order)


def _fp64_chain(metric, proj_bf16, order, norm_bf16):
    rnd = proj_bf16.dtype                  # bf16, or fp16 for the fp16-autocast chain
    x = metric.to(rnd).double().cpu()[:, order.cpu()]
    y = (x @ proj_bf16.double().cpu()).to(rnd).double()
    n = y.norm(dim=-1, keepdim=True)
    if norm_bf16:
        n = n.to(torch.bfloat16).double()
    return y / n


def _ordered(t):
    v = t.contiguous().view(torch.int16).int()
    return torch.where(v < 0, -(v & 0x7FFF), v)


# Elements of a unit row are ~0.09; a projection that cancels to near zero
# carries the fp32 accumulation error (~1e-7 of the row norm) into its bf16
# rounding, so small elements get an absolute floor of 2^-16.
ABS_FLOOR = 2.0 ** -16


def _compare(got, chain, ref64, what):
    ulps = (_ordered(got) - _ordered(chain)).abs()
    frac = (ulps > 0).float().mean().item()
    diff = (got.float() - chain.float()).abs()
    worst = ulps.flatten().argmax()
    print(f"\n[{what}] max ulps {ulps.max().item()} (at {chain.flatten()[worst].item():.3e}) "
          f"differing {frac:.2e} max diff {diff.max().item():.2e}")
    assert frac <= 2e-3
    # Where the two accumulation orders round y to neighbouring bf16 values
    # (at most 2^-7 apart), both outputs then round once more: 2^-7 + 2 * 2^-8.
    assert (diff <= 2.0 ** -6 * chain.float().abs() + ABS_FLOOR).all()
    g = got.double().cpu()
    assert ((g - ref64).abs() <= 3 * 2.0 ** -8 * ref64.abs() + ABS_FLOOR).all()


def _order(frames, dev, seed=33):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    mask = dst_mask(frames, 37, 37, 2, 2, 5, False, gen, dev)
    return torch.argsort(mask, stable=True)


@pytest.mark.parametrize("dtype,autocast", [(torch.float32, True), (torch.bfloat16, True),
                                            (torch.bfloat16, False)])
def test_vggt_width_against_the_chain(dev, dtype, autocast):
    frames = 4
    metric = W.shifted_basis_tokens(frames, seed=3).to(dev, dtype)     # [1, 5496, 1024]
    order = _order(frames, dev)
    proj_f32 = _projection(dev, 1024, 128, torch.float32)
    proj = _projection(dev, 1024, 128)
    if autocast:
        with torch.autocast("cuda", dtype=torch.bfloat16):
            got = _native.merge_metric(metric, proj, order, 0)
    else:
        got = _native.merge_metric(metric, proj, order, 1)
    chain = _torch_chain(metric, proj_f32, order, autocast)
    assert got.dtype == torch.bfloat16 and got.shape == (1, metric.shape[1], 128)
    _compare(got, chain, _fp64_chain(metric, proj, order, not autocast), f"{dtype} {autocast}")


@pytest.mark.parametrize("C", [256, 512, 768, 1024])
def test_widths_batches_strides_and_tails(dev, C):
    """B = 2, rows with a stride wider than C, N not a multiple of 16, a
    random order and the identity order."""
    g = torch.Generator().manual_seed(C)
    B, N = 2, 1001
    big = torch.randn(B, N, C + 64, generator=g)
    metric = big.to(dev)[:, :, :C]
    proj_f32 = torch.randn(C, 128, generator=g).to(dev)
    proj = proj_f32.to(torch.bfloat16)
    for order in (torch.randperm(N, generator=g).to(dev), None):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            got = _native.merge_metric(metric, proj, order, 0)
        o = torch.arange(N, device=dev) if order is None else order
        chain = _torch_chain(metric, proj_f32, o, True)
        _compare(got, chain, _fp64_chain(metric, proj, o, False), f"C={C}")


def test_many_blocks_per_workgroup(dev):
    """50,000 tokens: a dozen 16-row blocks per workgroup, both loads in flight."""
    g = torch.Generator().manual_seed(9)
    N, C = 50_000, 1024
    metric = torch.randn(1, N, C, generator=g).to(dev)
    order = torch.randperm(N, generator=g).to(dev)
    proj_f32 = _projection(dev, C, 128, torch.float32)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        got = _native.merge_metric(metric, _projection(dev, C, 128), order, 0)
    chain = _torch_chain(metric, proj_f32, order, True)
    ulps = (_ordered(got) - _ordered(chain)).abs()
    assert (ulps > 0).float().mean().item() <= 2e-3
    assert ((got.float() - chain.float()).abs() <= 2.0 ** -6 * chain.float().abs()
            + ABS_FLOOR).all()
    # Deterministic: the row sums meet in a fixed order.
    with torch.autocast("cuda", dtype=torch.bfloat16):
        again = _native.merge_metric(metric, _projection(dev, C, 128), order, 0)
    assert torch.equal(got, again)


def test_zero_row_gives_nan_like_the_reference(dev):
    metric = torch.randn(1, 40, 256, device=dev)
    metric[0, 7] = 0
    proj = torch.randn(256, 128, device=dev).to(torch.bfloat16)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        got = _native.merge_metric(metric, proj, None, 0)
    assert torch.isnan(got[0, 7]).all()
    assert torch.isfinite(got[0, torch.arange(40, device=dev) != 7]).all()


def test_token_merge_uses_the_front_end_under_autocast(dev):
    """The merge under autocast: node_max stays fp32 (the reference's division
    promotes to fp32), and the node indices agree with the oracle's chunked
    bf16 similarity (merging/merge.py:13-36, on the CPU) of the torch
    chain's operands under the top-2 gap rule."""
    frames, ns = 4, 5
    metric = W.shifted_basis_tokens(frames, seed=5).to(dev)
    n = metric.shape[1]
    gen = torch.Generator(device=dev)
    gen.manual_seed(33)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        m = token_merge_bipartite2d(metric, 37, 37, 2, 2, int(0.98 * n), False, gen,
                                    metric_dim=128, num_special=ns)
    ix = m.index
    assert ix.node_max.dtype == torch.float32
    num_dst = num_dst_tokens(frames, 37, 37, 2, 2, ns, False)
    order = torch.cat([ix.b_idx, ix.a_idx])
    ab = _torch_chain(metric, _projection(dev, 1024, 128, torch.float32), order, True)
    a, b = ab[:, num_dst:], ab[:, :num_dst]
    ref_max, ref_idx = fast_similarity_chunks(a.cpu(), b.cpu().transpose(1, 2), 5000)
    keep = (bf16_top2_gap(a, b) >= 1e-3).cpu()
    assert keep.float().mean() > 0.5
    assert torch.equal(ix.node_idx.cpu()[keep], ref_idx[keep])
    # the oracle's max is the bf16-rounded score, the kernel's the fp32 one
    assert (ix.node_max.cpu() - ref_max.float()).abs().max().item() <= 2.0 ** -8
    assert m.size.sum().item() == n


def test_fp16_autocast_chain(dev):
    """Mode 2: under fp16 autocast the projection runs in fp16 (metric and
    basis rounded to fp16, y rounded to fp16), then the fp32 norm and the
    bf16 cast of the similarity operands."""
    frames = 4
    metric = W.shifted_basis_tokens(frames, seed=8).to(dev)            # fp32
    order = _order(frames, dev)
    proj_f32 = _projection(dev, 1024, 128, torch.float32)
    proj16 = _projection(dev, 1024, 128, torch.float16)
    got = _native.merge_metric(metric, proj16, order, 2)
    chain = _torch_chain(metric, proj_f32, order, True, torch.float16)
    _compare(got, chain, _fp64_chain(metric, proj16, order, False), "fp16 autocast")
    with pytest.raises(ValueError):
        _native.merge_metric(metric, _projection(dev, 1024, 128), order, 2)   # bf16 basis


def test_token_merge_under_fp16_autocast(dev):
    frames, ns = 4, 5
    metric = W.shifted_basis_tokens(frames, seed=9).to(dev)
    n = metric.shape[1]
    gen = torch.Generator(device=dev)
    gen.manual_seed(33)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16):
        m = token_merge_bipartite2d(metric, 37, 37, 2, 2, int(0.98 * n), False, gen,
                                    metric_dim=128, num_special=ns)
    ix = m.index
    assert ix.node_max.dtype == torch.float32
    num_dst = num_dst_tokens(frames, 37, 37, 2, 2, ns, False)
    order = torch.cat([ix.b_idx, ix.a_idx])
    ab = _torch_chain(metric, _projection(dev, 1024, 128, torch.float32), order, True,
                      torch.float16)
    a, b = ab[:, num_dst:], ab[:, :num_dst]
    _, ref_idx = fast_similarity_chunks(a.cpu(), b.cpu().transpose(1, 2), 5000)
    keep = (bf16_top2_gap(a, b) >= 1e-3).cpu()
    assert keep.float().mean() > 0.5
    assert torch.equal(ix.node_idx.cpu()[keep], ref_idx[keep])
