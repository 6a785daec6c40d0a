"""Pins the similarity oracle (oracle/similarity.py) without a GPU.

fast_similarity_chunks restates merging/merge.py:13-36.  It is pinned by
the fp64 brute force on the same bf16-rounded inputs, by planted matches
with a known answer, by the first-index tie rule and by chunk invariance.
"""
import numpy as np
import pytest
import torch

from oracle.similarity import bf16_round, bf16_top2_gap, fast_similarity_chunks, sim_argmax_fp64


def _unit(x):
    return x / x.norm(dim=-1, keepdim=True)


def test_chunked_matches_fp64_brute_force():
    g = torch.Generator().manual_seed(0)
    a = _unit(torch.randn(1, 600, 64, generator=g))
    b = _unit(torch.randn(1, 250, 64, generator=g))
    vmax, vidx = fast_similarity_chunks(a, b.transpose(1, 2), 97)
    fmax, fidx, gap = sim_argmax_fp64(a, b)
    # bf16-rounded scores: the max is the fp64 max rounded to bf16 (one
    # rounding of an fp32 accumulation of exact products).
    ref = bf16_round(torch.from_numpy(fmax).float())
    assert torch.allclose(vmax, ref, atol=0, rtol=2 ** -7)
    # Wherever two bf16 ulps separate the top two scores, the index agrees.
    sure = torch.from_numpy(gap > 2 * 2 ** -8)
    assert sure.float().mean() > 0.5
    assert torch.equal(vidx[sure], torch.from_numpy(fidx)[sure])


def test_planted_matches_known_answer():
    g = torch.Generator().manual_seed(1)
    b = _unit(torch.randn(1, 300, 128, generator=g))
    perm = torch.randint(0, 300, (1000,), generator=g)
    a = _unit(b[:, perm] + 0.01 * torch.randn(1, 1000, 128, generator=g))
    _, vidx = fast_similarity_chunks(a, b.transpose(1, 2), 5000)
    _, fidx, _ = sim_argmax_fp64(a, b)
    assert torch.equal(vidx[0], perm)
    assert np.array_equal(fidx[0], perm.numpy())


def test_tie_goes_to_lowest_index():
    g = torch.Generator().manual_seed(2)
    base = _unit(torch.randn(1, 10, 32, generator=g))
    b = torch.cat([base, base, base], dim=1)          # every row appears 3 times
    a = base[:, torch.tensor([3, 0, 9, 9])]
    _, vidx = fast_similarity_chunks(a, b.transpose(1, 2), 2)
    _, fidx, gap = sim_argmax_fp64(a, b)
    assert vidx[0].tolist() == [3, 0, 9, 9]
    assert fidx[0].tolist() == [3, 0, 9, 9]
    assert np.all(gap == 0.0)


def test_chunking_does_not_change_the_result():
    g = torch.Generator().manual_seed(3)
    a = _unit(torch.randn(2, 333, 64, generator=g))
    b = _unit(torch.randn(2, 77, 64, generator=g))
    ref = fast_similarity_chunks(a, b.transpose(1, 2), 333)
    for chunk in (1, 7, 100, 5000):
        out = fast_similarity_chunks(a, b.transpose(1, 2), chunk)
        assert torch.equal(out[0], ref[0]) and torch.equal(out[1], ref[1])


def test_max_keeps_input_dtype():
    a = _unit(torch.randn(1, 8, 32))
    b = _unit(torch.randn(1, 5, 32))
    vmax, vidx = fast_similarity_chunks(a, b.transpose(1, 2), 4)
    assert vmax.dtype == torch.float32 and vidx.dtype == torch.int64
    vmax16, _ = fast_similarity_chunks(a.bfloat16(), b.bfloat16().transpose(1, 2), 4)
    assert vmax16.dtype == torch.bfloat16


def test_bf16_top2_gap_matches_definition():
    g = torch.Generator().manual_seed(4)
    a = _unit(torch.randn(1, 50, 32, generator=g))
    b = _unit(torch.randn(1, 40, 32, generator=g))
    gap = bf16_top2_gap(a, b, chunk_size=13)
    s = torch.bmm(a.bfloat16(), b.bfloat16().transpose(1, 2)).float()
    srt = s.sort(dim=-1, descending=True).values
    assert torch.equal(gap, srt[..., 0] - srt[..., 1])


def test_fp64_gap_is_inf_for_single_destination():
    a = _unit(torch.randn(1, 4, 32))
    b = _unit(torch.randn(1, 1, 32))
    _, idx, gap = sim_argmax_fp64(a, b)
    assert np.all(idx == 0) and np.all(np.isinf(gap))
