"""The similarity-argmax above D = 256: the GEMM-tiled kernels that loop over
the features, 256 x 256 tiles for D = 512 ... 1024 in steps of 128 and
128 x 128 otherwise (the unprojected 1024-d metric of `metric_dim=0`,
eval/eval_co3d.py:121-122 and merging/merge.py:180, which the reference
kernel serves by tiling D with BLOCK_K, merging/fused_similarity.py:55-68).

Bars as for the projected metric: max within 1e-5 of the fp64 brute force
on the same 16-bit inputs; index equal to the fp64 argmax wherever the
top-2 gap exceeds 1e-5; ties to the lowest destination index; rows past the
end of a split never win; the merge at metric_dim=0 equal to the oracle's
chunked bf16 similarity under the reference's top-2 gap rule.
"""
import numpy as np
import pytest
import torch

import gpa_workloads as W
from merging.fused_similarity import fused_similarity_argmax
from merging.merge import token_merge_bipartite2d
from oracle.similarity import bf16_round, bf16_top2_gap, fast_similarity_chunks, sim_argmax_fp64

pytestmark = pytest.mark.gpu


def _unit_values(shape, seed, dtype=torch.bfloat16):
    """fp32 tensor of unit rows whose entries are exactly `dtype`-representable."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    return (x / x.norm(dim=-1, keepdim=True)).to(dtype).float()


def _check(a, b, vmax, vidx):
    vmax, vidx = vmax.float().cpu().numpy(), vidx.cpu().numpy()
    fmax, fidx, gap = sim_argmax_fp64(a, b)
    assert np.abs(vmax - fmax).max() < 1e-5
    sure = gap > 1e-5
    assert sure.mean() > 0.8
    assert np.array_equal(vidx[sure], fidx[sure])
    a64, b64 = a.double().numpy(), b.double().numpy()
    chosen = np.einsum("bmd,bmd->bm", a64, np.take_along_axis(b64, vidx[..., None], axis=1))
    assert np.abs(chosen - fmax).max() < 1e-5


@pytest.mark.parametrize("B,M,N,D", [
    (1, 1, 1, 1024), (1, 130, 200, 512), (2, 300, 1000, 1024), (1, 257, 9000, 544),
    (1, 1000, 333, 288), (1, 1024, 12_000, 1024), (3, 129, 129, 768),
    # 64 destination splits (8 per XCD); B > 1 at D = 512; every D the
    # 256 x 256-tile kernel is built for; above 1024 the GEMM-tiled kernel
    (1, 300, 50_000, 1024), (2, 300, 36_000, 512), (1, 300, 9_000, 640),
    (1, 257, 9_500, 896), (1, 200, 3_000, 1280),
])
def test_matches_fp64_brute_force(dev, B, M, N, D):
    print(f"[wide sim] B={B} M={M} N={N} D={D}", flush=True)
    a = _unit_values((B, M, D), seed=M + 7 * N + D)
    b = _unit_values((B, N, D), seed=M + 11 * N + D + 1)
    vmax, vidx = fused_similarity_argmax(a.to(dev), b.to(dev))
    assert vmax.dtype == torch.float32 and vidx.dtype == torch.int64
    _check(a, b, vmax, vidx)


@pytest.mark.parametrize("D", [512, 640, 768, 896, 1024])
def test_fp16_operands(dev, D):
    """Every D the 256 x 256-tile kernel is built for, on fp16 operands."""
    print(f"[wide sim] fp16 D={D}", flush=True)
    a = _unit_values((1, 700, D), seed=1 + D, dtype=torch.float16)
    b = _unit_values((1, 5000, D), seed=2 + D, dtype=torch.float16)
    vmax, vidx = fused_similarity_argmax(a.to(dev).half(), b.to(dev).half())
    assert vmax.dtype == torch.float16
    s = a.double().numpy()[0] @ b.double().numpy()[0].T       # fp64 on the fp16 values
    fidx = s.argmax(1)
    top = s[np.arange(len(fidx)), fidx]
    s[np.arange(len(fidx)), fidx] = -np.inf
    sure = top - s.max(1) > 1e-5
    assert sure.mean() > 0.8
    assert np.array_equal(vidx[0].cpu().numpy()[sure], fidx[sure])
    assert np.abs(vmax[0].float().cpu().numpy() - top).max() < 1e-3     # fp16 output


def test_padded_feature_dim(dev):
    """D = 1000 is padded to 1024 with zero features (exact)."""
    a = _unit_values((1, 400, 1000), seed=5)
    b = _unit_values((1, 3000, 1000), seed=6)
    vmax, vidx = fused_similarity_argmax(a.to(dev), b.to(dev))
    _check(a, b, vmax, vidx)


@pytest.mark.parametrize("N", [200, 20_000])
def test_ties_resolve_to_lowest_index(dev, N):
    """Three copies of each matched destination row: the first copy wins, in
    any tile or split."""
    nb = min(64, N // 3)
    base = _unit_values((1, nb, 1024), seed=N)
    g = torch.Generator().manual_seed(N + 1)
    b = _unit_values((1, N, 1024), seed=N + 2)
    slots = torch.randperm(N, generator=g)[:3 * nb].view(3, nb).sort(dim=0).values
    for c in range(3):
        b[0, slots[c]] = base[0]
    _, vidx = fused_similarity_argmax(base.to(dev), b.to(dev))
    assert torch.equal(vidx[0].cpu(), slots[0])


@pytest.mark.parametrize("M,N", [(300, 100), (500, 2000), (1300, 9001)])
def test_rows_past_n_never_win(dev, M, N):
    """b as a view of the first N rows of a larger buffer whose next rows are
    100x the source rows (each would beat every real score of its source
    row): the kernels fetch whole tiles and stages ahead of the one they
    score, and rows past N must neither win nor move the max."""
    a = _unit_values((1, M, 1024), seed=M + N)
    b = _unit_values((1, N, 1024), seed=M + N + 1)
    big = torch.cat([b, 100 * a, torch.zeros(1, 256, 1024)], dim=1)
    db = big.bfloat16().to(dev)[:, :N]
    vmax, vidx = fused_similarity_argmax(a.to(dev).bfloat16(), db)
    assert int(vidx.max()) < N
    fmax, fidx, gap = sim_argmax_fp64(a, b)
    assert np.abs(vmax.float().cpu().numpy() - fmax).max() < 4e-3          # bf16 output dtype
    sure = gap > 1e-5
    assert np.array_equal(vidx.cpu().numpy()[sure], fidx[sure])


@pytest.mark.parametrize("N", [1000, 40_000])
def test_last_tile_rows_scored_twice(dev, N):
    """A split that ends inside a 256-row tile has its last tile start 256
    rows before its end, so that tile's first rows (N - 256 on) were scored
    by the tile before too.  Maxima planted there, each with an exact copy
    later in the last tile, must report the first copy; maxima planted only
    in the last tile's own rows report theirs.  (N = 1000: one split, rows
    744..767 scored twice; N = 40,000: 32 splits, the last one 38,912 ..
    39,999, rows 39,744..39,935 scored twice.)"""
    print(f"[wide sim] overlap N={N}", flush=True)
    a = _unit_values((1, 48, 1024), seed=N + 3)
    b = _unit_values((1, N, 1024), seed=N + 4)
    want = []
    for i in range(24):                     # in the rows scored twice, a copy at N-1-i
        b[0, N - 256 + i] = a[0, i]
        b[0, N - 1 - i] = a[0, i]
        want.append(N - 256 + i)
    for i in range(24, 48):                 # once, in the last tile's own rows
        b[0, N - 1 - i] = a[0, i]
        want.append(N - 1 - i)
    vmax, vidx = fused_similarity_argmax(a.to(dev), b.to(dev))
    assert vidx[0].cpu().tolist() == want
    fmax, _, _ = sim_argmax_fp64(a, b)
    assert np.abs(vmax.float().cpu().numpy() - fmax).max() < 1e-5


def test_strided_views(dev):
    big_a = _unit_values((2, 600, 1088), seed=11)
    big_b = _unit_values((2, 900, 1152), seed=12)
    da, db = big_a.to(dev).bfloat16(), big_b.to(dev).bfloat16()
    a, b = da[:, 50:550, 64:1088], db[:, 10:810, 128:1152]      # row strides 1088, 1152
    vmax, vidx = fused_similarity_argmax(a, b)
    fmax, fidx, gap = sim_argmax_fp64(a.float().cpu(), b.float().cpu())
    assert np.abs(vmax.float().cpu().numpy() - fmax).max() < 4e-3
    sure = gap > 1e-5
    assert np.array_equal(vidx.cpu().numpy()[sure], fidx[sure])


def test_merge_without_projection(dev):
    """token_merge_bipartite2d with metric_dim=0 (full 1024-d cosine) under
    bf16 autocast: node indices equal to the oracle's chunked bf16
    similarity (merging/merge.py:13-36) under the top-2 gap rule, sizes
    summing to the token count."""
    frames, ns = 4, 5
    metric = W.shifted_basis_tokens(frames, seed=7).to(dev)
    n = metric.shape[1]
    gen = torch.Generator(device=dev)
    gen.manual_seed(33)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        m = token_merge_bipartite2d(metric, 37, 37, 2, 2, int(0.98 * n), False, gen,
                                    metric_dim=0, num_special=ns)
        unit = metric / metric.norm(dim=-1, keepdim=True)
    ix = m.index
    a = unit.index_select(1, ix.a_idx).to(torch.bfloat16)
    b = unit.index_select(1, ix.b_idx).to(torch.bfloat16)
    _, ref_idx = fast_similarity_chunks(a.cpu(), b.cpu().transpose(1, 2), 5000)
    keep = (bf16_top2_gap(a, b) >= 1e-3).cpu()
    assert keep.float().mean() > 0.5
    assert torch.equal(ix.node_idx.cpu()[keep], ref_idx[keep])
    fmax, fidx, gap = sim_argmax_fp64(a.float().cpu(), b.float().cpu())
    sure = gap > 1e-5
    assert np.array_equal(ix.node_idx.cpu().numpy()[sure], fidx[sure])
    assert m.size.sum().item() == n
