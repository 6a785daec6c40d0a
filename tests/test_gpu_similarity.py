"""Parity of the gfx950 similarity-argmax kernel with the oracle.

Bars:
  * max: within 1e-5 of the fp64 brute force on the same bf16 inputs
    (fp32 accumulation of exact bf16 products);
  * index: identical to the fp64 argmax wherever the fp64 top-2 gap exceeds
    1e-5, and identical to the reference torch path (bf16 bmm + torch.max,
    merging/merge.py:13-36) on every row whose bf16 top-2 gap is >= 1e-3;
  * ties: the lowest destination index, across tiles and across splits.
"""
import numpy as np
import pytest
import torch

import gpa_workloads as W
from merging.fused_similarity import fused_similarity_argmax
from oracle.similarity import bf16_round, bf16_top2_gap, fast_similarity_chunks, sim_argmax_fp64

pytestmark = pytest.mark.gpu


def _unit_bf16_values(shape, seed):
    """fp32 tensor of unit rows whose entries are exactly bf16-representable."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    return bf16_round(x / x.norm(dim=-1, keepdim=True))


@pytest.mark.parametrize("B,M,N,D", [
    (1, 1, 1, 32), (1, 5, 17, 64), (1, 100, 33, 128), (2, 257, 100, 128), (1, 300, 1000, 96),
    (1, 1000, 513, 256), (1, 4097, 65, 160), (1, 3000, 9000, 128), (1, 700, 20_000, 128),
])
def test_matches_fp64_brute_force(dev, B, M, N, D):
    a = _unit_bf16_values((B, M, D), seed=M + 7 * N + D)
    b = _unit_bf16_values((B, N, D), seed=M + 11 * N + D + 1)
    vmax, vidx = fused_similarity_argmax(a.to(dev), b.to(dev))
    assert vmax.dtype == torch.float32 and vidx.dtype == torch.int64
    vmax, vidx = vmax.cpu().numpy(), vidx.cpu().numpy()
    fmax, fidx, gap = sim_argmax_fp64(a, b)
    assert np.abs(vmax - fmax).max() < 1e-5
    sure = gap > 1e-5
    assert sure.mean() > 0.9
    assert np.array_equal(vidx[sure], fidx[sure])
    # every chosen index scores within 1e-5 of the row max
    a64, b64 = a.double().numpy(), b.double().numpy()
    chosen = np.einsum("bmd,bmd->bm", a64, np.take_along_axis(b64, vidx[..., None], axis=1))
    assert np.abs(chosen - fmax).max() < 1e-5


def test_planted_matches(dev):
    g = torch.Generator().manual_seed(5)
    b = _unit_bf16_values((1, 5000, 128), seed=6)
    perm = torch.randint(0, 5000, (20_000,), generator=g)
    a = b[:, perm] + 0.02 * torch.randn(1, 20_000, 128, generator=g)
    a = bf16_round(a / a.norm(dim=-1, keepdim=True))
    _, vidx = fused_similarity_argmax(a.to(dev), b.to(dev))
    assert torch.equal(vidx[0].cpu(), perm)


@pytest.mark.parametrize("N", [96, 1000, 20_000])
def test_ties_resolve_to_lowest_index(dev, N):
    """Duplicate destination rows: the first copy wins, in any tile or split."""
    nb = min(64, N // 3)
    base = _unit_bf16_values((1, nb, 128), seed=N)
    g = torch.Generator().manual_seed(N + 1)
    b = _unit_bf16_values((1, N, 128), seed=N + 2)
    slots = torch.randperm(N, generator=g)[:3 * nb].view(3, nb)
    slots = slots.sort(dim=0).values                    # three copies per base row
    for c in range(3):
        b[0, slots[c]] = base[0]
    a = base.clone()
    vmax, vidx = fused_similarity_argmax(a.to(dev), b.to(dev))
    assert torch.equal(vidx[0].cpu(), slots[0])
    _, fidx, _ = sim_argmax_fp64(a, b)
    assert np.array_equal(fidx[0], slots[0].numpy())


def test_strided_and_batched_inputs(dev):
    big_a = _unit_bf16_values((2, 600, 192), seed=1)
    big_b = _unit_bf16_values((2, 300, 192), seed=2)
    a = big_a[:, 50:550, :128]                            # row stride 192, offset rows
    b = big_b[:, :250, 64:192]
    a_n = a / a.norm(dim=-1, keepdim=True)
    b_n = b / b.norm(dim=-1, keepdim=True)
    a_n, b_n = bf16_round(a_n), bf16_round(b_n)
    big_a[:, 50:550, :128] = a_n
    big_b[:, :250, 64:192] = b_n
    da, db = big_a.to(dev).bfloat16(), big_b.to(dev).bfloat16()
    vmax, vidx = fused_similarity_argmax(da[:, 50:550, :128], db[:, :250, 64:192])
    fmax, fidx, gap = sim_argmax_fp64(a_n, b_n)
    assert np.abs(vmax.float().cpu().numpy() - fmax).max() < 4e-3     # bf16 output dtype
    sure = gap > 1e-5
    assert np.array_equal(vidx.cpu().numpy()[sure], fidx[sure])


@pytest.mark.parametrize("M,N", [(300, 17), (300, 64), (2000, 1000), (3000, 9001)])
def test_rows_past_n_never_win(dev, M, N):
    """b as a view of the first N rows of a larger buffer whose other rows
    would beat every real score (a constant vector of norm 90): the kernel
    fetches 16-row tiles and stages past the end of each destination split,
    and those rows must neither win nor move the maximum."""
    a = _unit_bf16_values((1, M, 128), seed=M + N)
    b = _unit_bf16_values((1, N, 128), seed=M + N + 1)
    big = torch.full((1, N + 300, 128), 8.0)
    big[:, :N] = b
    db = big.bfloat16().to(dev)[:, :N]
    vmax, vidx = fused_similarity_argmax(a.to(dev).bfloat16(), db)
    vmax, vidx = vmax.float().cpu().numpy(), vidx.cpu().numpy()
    assert vidx.max() < N
    fmax, fidx, gap = sim_argmax_fp64(a, b)
    assert np.abs(vmax - fmax).max() < 4e-3                          # bf16 output dtype
    sure = gap > 1e-5
    assert np.array_equal(vidx[sure], fidx[sure])


@pytest.mark.parametrize("D,half", [(96, False), (128, False), (512, False), (128, True)])
def test_nan_and_zero_rows(dev, D, half):
    """NaN scores never win (the strict > of fused_similarity.py:73 over
    tl.max's NaN-free maximum): a source row of NaN features scores NaN
    against everything and yields -inf with index 0; destination rows
    holding a NaN are never chosen; an all-zero source row scores 0 against
    every other row and takes index 0.  Covers the register-staged (D 96),
    pipelined (D 128, bf16 and fp16 operands) and 256 x 256-tile (D 512)
    kernels, with several destination splits."""
    M, N = 600, 3000
    a = _unit_bf16_values((1, M, D), seed=71 + D)
    b = _unit_bf16_values((1, N, D), seed=72 + D)
    nan_src = torch.arange(0, M, 37)
    zero_src = torch.arange(5, M, 41)
    zero_src = zero_src[~torch.isin(zero_src, nan_src)]     # disjoint (333 is in both)
    nan_dst = torch.arange(3, N, 7)                  # in every 16-row tile
    a[0, nan_src] = float("nan")
    a[0, zero_src] = 0.0
    b[0, nan_dst, D // 2] = float("nan")
    if half:        # fp16 holds these bf16 values to < 1e-7 (only tiny ones lose bits)
        vmax, vidx = fused_similarity_argmax(a.half().to(dev), b.half().to(dev))
        vmax = vmax.float()                  # returned in fp16, the input format
    else:
        vmax, vidx = fused_similarity_argmax(a.to(dev), b.to(dev))
    vmax, vidx = vmax[0].cpu(), vidx[0].cpu()
    assert torch.all(vmax[nan_src] == -float("inf")) and torch.all(vidx[nan_src] == 0)
    assert torch.all(vmax[zero_src] == 0) and torch.all(vidx[zero_src] == 0)
    assert not torch.isin(vidx, nan_dst).any()
    keep = torch.ones(N, dtype=torch.bool)
    keep[nan_dst] = False
    rows = torch.ones(M, dtype=torch.bool)
    rows[nan_src] = False
    rows[zero_src] = False
    fmax, fidx, gap = sim_argmax_fp64(a[:, rows], b[:, keep])
    assert np.abs(vmax[rows].numpy() - fmax[0]).max() < (1e-3 if half else 1e-5)
    sure = gap[0] > 1e-5
    kept = torch.nonzero(keep)[:, 0].numpy()
    assert np.array_equal(vidx[rows].numpy()[sure], kept[fidx[0]][sure])


def test_dtype_contract(dev):
    a = _unit_bf16_values((1, 64, 128), seed=3)
    b = _unit_bf16_values((1, 40, 128), seed=4)
    m32, i32 = fused_similarity_argmax(a.to(dev), b.to(dev))
    m16, i16 = fused_similarity_argmax(a.to(dev).bfloat16(), b.to(dev).bfloat16())
    assert m32.dtype == torch.float32 and m16.dtype == torch.bfloat16
    assert torch.equal(i32, i16)
    assert torch.equal(m32.bfloat16(), m16)


def test_feature_dim_padding_is_exact(dev):
    a = _unit_bf16_values((1, 300, 48), seed=8)
    b = _unit_bf16_values((1, 77, 48), seed=9)
    vmax, vidx = fused_similarity_argmax(a.to(dev), b.to(dev))
    fmax, fidx, gap = sim_argmax_fp64(a, b)
    assert np.abs(vmax.cpu().numpy() - fmax).max() < 1e-5
    sure = gap > 1e-5
    assert np.array_equal(vidx.cpu().numpy()[sure], fidx[sure])


def test_reference_torch_path_gap_rule(dev):
    """Shifted-basis data at a reduced size, against the CPU torch path."""
    src, dst = W.sim_inputs(m=12_000, n=4_000, seed=3)
    vmax, vidx = fused_similarity_argmax(src.to(dev), dst.to(dev))
    rmax, ridx = fast_similarity_chunks(src, dst.transpose(1, 2), 5000)
    gap = bf16_top2_gap(src, dst)
    keep = gap >= 1e-3
    assert keep.float().mean() > 0.5
    assert torch.equal(vidx.cpu()[keep], ridx[keep])
    # our fp32 max rounds to within one bf16 ulp of the torch path's bf16 max
    assert (vmax.float().cpu() - rmax.float()).abs().max() <= 2 ** -7


def test_full_size_similarity_workload(dev):
    """75,000 x 25,000 x 128 on the GPU, checked three ways."""
    src, dst = W.sim_inputs(m=75_000, n=25_000, seed=0, device=dev)
    vmax, vidx = torch.ops.gpa.sim_argmax(src, dst)          # fp32 max
    torch.cuda.synchronize()
    assert int(vidx.min()) >= 0 and int(vidx.max()) < 25_000
    # (1) the chosen destination scores the reported max (fp32 recompute)
    chosen = (src[0].float() * dst[0, vidx[0]].float()).sum(-1)
    assert (chosen - vmax[0].float()).abs().max().item() < 1e-5
    # (2) the reference torch path run on the same device: gap rule
    rmax, ridx = fast_similarity_chunks(src, dst.transpose(1, 2), 5000)
    gap = bf16_top2_gap(src, dst)
    keep = gap >= 1e-3
    mism = (vidx[keep] != ridx[keep]).sum().item()
    assert mism == 0, f"{mism} rows with bf16 gap >= 1e-3 disagree"
    print(f"\n[sim c2] rows compared under the gap rule: {keep.float().mean().item():.4f}")
    # (3) fp64 brute force on a sample of rows
    g = torch.Generator().manual_seed(0)
    rows = torch.randint(0, 75_000, (384,), generator=g)
    a = src[0, rows].float().cpu().unsqueeze(0)
    b = dst.float().cpu()
    fmax, fidx, fgap = sim_argmax_fp64(a, b)
    assert np.abs(vmax[0, rows.to(dev)].cpu().numpy() - fmax[0]).max() < 1e-5
    sure = fgap[0] > 1e-5
    assert np.array_equal(vidx[0, rows.to(dev)].cpu().numpy()[sure], fidx[0][sure])


def test_last_round_cut_into_sub_ranges(dev):
    """17,152 x 8,192 x 128: 67 source blocks x 16 destination splits = 1,072
    workgroups, two rounds of 512 plus 48, so the last 3 blocks give each
    split to 21 workgroups of 32 rows each, the last five of them empty
    (partials merged in destination order).  Against the fp64 brute force; tail rows whose best
    destination row is duplicated in other splits and sub-ranges resolve to
    the first copy."""
    M, N = 67 * 256, 8192
    a = _unit_bf16_values((1, M, 128), seed=91)
    b = _unit_bf16_values((1, N, 128), seed=92)
    g = torch.Generator().manual_seed(93)
    tail = torch.arange(64 * 256, M)
    rows = tail[torch.randperm(tail.numel(), generator=g)[:32]]
    copies = torch.randperm(N, generator=g)[:96].view(3, 32).sort(dim=0).values
    base = _unit_bf16_values((1, 32, 128), seed=94)
    for c in range(3):
        b[0, copies[c]] = base[0]
    a[0, rows] = base[0]
    vmax, vidx = fused_similarity_argmax(a.to(dev), b.to(dev))
    vmax, vidx = vmax.cpu().numpy(), vidx.cpu().numpy()
    fmax, fidx, gap = sim_argmax_fp64(a, b)
    assert np.abs(vmax - fmax).max() < 1e-5
    sure = gap > 1e-5
    assert sure.mean() > 0.9
    assert np.array_equal(vidx[sure], fidx[sure])
    assert np.array_equal(vidx[0, rows.numpy()], copies[0].numpy())
    assert np.array_equal(fidx[0, rows.numpy()], copies[0].numpy())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_max_written_in_the_input_dtype(dev, dtype):
    """fused_similarity_argmax returns node_max in a's dtype
    (merging/fused_similarity.py:112): the kernel writes it in that dtype,
    bit-identical to casting its fp32 max, with the same indices."""
    a = _unit_bf16_values((1, 9000, 128), seed=71).to(dtype)
    b = _unit_bf16_values((1, 30_000, 128), seed=72).to(dtype)
    vmax, vidx = fused_similarity_argmax(a.to(dev), b.to(dev))
    fmax, fidx = torch.ops.gpa.sim_argmax(a.to(dev), b.to(dev))
    assert vmax.dtype == dtype and fmax.dtype == torch.float32
    assert torch.equal(vmax, fmax.to(dtype)) and torch.equal(vidx, fidx)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_merge_module_fast_similarity_chunks(dev, dtype):
    """merging.merge.fast_similarity_chunks keeps the reference's name and
    arguments (merging/merge.py:13-36: a [B, M, C], b transposed [B, C, N],
    a chunk size) on the fused kernel: both operands cast to bf16 whatever
    their dtype, node_max a bf16 value returned in a's dtype, node_idx int64;
    against the oracle's restatement of the reference path under the gap
    rule, the max within one bf16 ulp, and no dependence on the chunk size."""
    from merging.merge import fast_similarity_chunks as product_chunks
    a = _unit_bf16_values((2, 3000, 128), seed=81).to(dtype)
    b = _unit_bf16_values((2, 5000, 128), seed=82).to(dtype)
    bt = b.transpose(1, 2)
    vmax, vidx = product_chunks(a.to(dev), bt.to(dev), 5000)
    assert vmax.dtype == dtype and vidx.dtype == torch.int64
    assert torch.equal(vmax.float(), vmax.float().bfloat16().float())    # a bf16 value
    rmax, ridx = fast_similarity_chunks(a, bt, 1000)
    gap = bf16_top2_gap(a.bfloat16().float(), b.bfloat16().float())
    keep = gap >= 1e-3
    assert keep.float().mean() > 0.5
    assert torch.equal(vidx.cpu()[keep], ridx[keep])
    assert (vmax.float().cpu() - rmax.float()).abs().max().item() <= 2 ** -7
    vmax2, vidx2 = product_chunks(a.to(dev), bt.to(dev), 7)
    assert torch.equal(vmax2, vmax) and torch.equal(vidx2, vidx)
