"""The merge's two orderings against the reference's own argsort calls.

merging/merge.py:165 orders tokens by `idx_buffer_seq.reshape(1, -1, 1)
.argsort(dim=1)` (a -1/0 destination mask) and :199 orders the source rows
by `node_max.argsort(dim=-1, descending=True)`; both are torch's default,
not-necessarily-stable sort.  `token_merge_bipartite2d` uses stable sorts
(tokens in increasing position within each class; ties of node_max by
increasing source row).  Here, on the device, the reference's literal calls
must give exactly the stable orders: for the masks of 1 to 200 frames (up to
274,800 tokens) and for node_max rows of 1,045 to 207,955 entries (the
source counts of 2 to 200 frames) with planted ties -- values rounded to
bf16 (a few hundred distinct levels), a run of exactly equal values, and a
constant row.
"""
import pytest
import torch

from merging.merge import dst_mask, num_dst_tokens

pytestmark = pytest.mark.gpu

GRID, PTS = 37, 5


@pytest.mark.parametrize("frames", [1, 2, 3, 100, 200])
def test_dst_order_is_the_reference_argsort(dev, frames):
    gen = torch.Generator(device=dev)
    gen.manual_seed(33)
    mask = dst_mask(frames, GRID, GRID, 2, 2, PTS, False, gen, dev)
    ref = mask.reshape(1, -1, 1).argsort(dim=1).view(-1)                  # merge.py:165
    ours = torch.argsort(mask, stable=True)
    nd = num_dst_tokens(frames, GRID, GRID, 2, 2, PTS, False)
    assert int((mask == -1).sum()) == nd
    assert torch.equal(ref, ours)


@pytest.mark.parametrize("m", [1_045, 3_135, 4_096, 103_455, 207_955])
@pytest.mark.parametrize("kind", ["bf16_levels", "equal_run", "constant"])
def test_edge_order_is_the_reference_argsort(dev, m, kind):
    g = torch.Generator(device=dev)
    g.manual_seed(m)
    x = torch.rand(1, m, generator=g, device=dev) * 0.4 + 0.6
    if kind == "bf16_levels":
        x = x.bfloat16().float()                        # ~100 distinct values
    elif kind == "equal_run":
        x[:, m // 3: m // 3 + 997] = 0.75               # a run of exact ties
        x[:, ::5] = 0.875                               # and a strided set
    else:
        x = torch.full((1, m), 0.5, device=dev)
    assert (x.unique().numel() < m)
    ref = x.argsort(dim=-1, descending=True)                               # merge.py:199
    ours = torch.argsort(x, dim=-1, descending=True, stable=True)
    assert torch.equal(ref, ours)
