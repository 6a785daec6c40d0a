"""Pins the merge oracle (oracle/merge.py) without a GPU.

The restatement of merging/merge.py:39-256 is checked bit-for-bit against
vectors written by running the reference itself on the CPU
(tests/golden/make_merge_golden.py), then against closed-form invariants
and a brute-force fp64 mean merge.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.merge import (build_dst_mask, merge_heads_fp64, projection_basis,
                          token_merge_reference, window_draw)

GOLDEN = Path(__file__).resolve().parent / "golden" / "merge_golden.npz"


def _cases():
    z = np.load(GOLDEN)
    return z, [str(c) for c in z["cases"]]


@pytest.mark.parametrize("case", _cases()[1])
def test_matches_reference_run(case):
    z, _ = _cases()
    frames, w, h, sx, sy, ns, c, mdim, r, no_rand, seed = (int(x) for x in z[f"{case}/params"])
    metric = torch.from_numpy(z[f"{case}/metric"])
    t = torch.from_numpy(z[f"{case}/t"])
    gen = torch.Generator().manual_seed(33)
    o = token_merge_reference(metric, w, h, sx, sy, r, bool(no_rand), gen, mdim, ns, stable=False)
    n = metric.shape[1]
    pos = torch.arange(n, dtype=torch.float64).view(1, n, 1)
    ones = torch.ones(1, n, 1, dtype=torch.float64)
    assert np.array_equal(o.size.numpy(), z[f"{case}/size"])
    assert np.array_equal(o.merge(ones, "sum")[0, :, 0].numpy(), z[f"{case}/count"])
    assert np.array_equal(o.merge(pos, "amin")[0, :, 0].numpy(), z[f"{case}/pos_min"])
    assert np.array_equal(o.merge(pos, "amax")[0, :, 0].numpy(), z[f"{case}/pos_max"])
    np.testing.assert_allclose(o.heads(t, "mean").numpy(), z[f"{case}/heads_mean"], rtol=0,
                               atol=1e-13)


def _assignment(o):
    """{source token: (its max score, the dst token it merged into)}."""
    rows = {int(t): i for i, t in enumerate(o.a_idx.tolist())}
    out = {}
    for s, d in zip(o.src_abs_idx[0].tolist(), o.dst_idx[0].tolist()):
        out[s] = (float(o.node_max[0, rows[s]]), int(o.b_idx[d]))
    return out


@pytest.mark.parametrize("case", ["all_merged", "no_rand"])
def test_stable_order_changes_only_tied_choices(case):
    """The dst/src order only matters where bf16 scores tie at the maximum."""
    z, _ = _cases()
    frames, w, h, sx, sy, ns, c, mdim, r, no_rand, seed = (int(x) for x in z[f"{case}/params"])
    metric = torch.from_numpy(z[f"{case}/metric"])
    o_ref = token_merge_reference(metric, w, h, sx, sy, r, bool(no_rand),
                                  torch.Generator().manual_seed(33), mdim, ns, stable=False)
    o_st = token_merge_reference(metric, w, h, sx, sy, r, bool(no_rand),
                                 torch.Generator().manual_seed(33), mdim, ns, stable=True)
    assert torch.equal(o_st.b_idx, torch.sort(o_st.b_idx).values)
    assert torch.equal(o_st.a_idx, torch.sort(o_st.a_idx).values)
    assert torch.equal(torch.sort(o_ref.b_idx).values, o_st.b_idx)
    x = metric @ projection_basis(c, mdim) if mdim and mdim < c else metric
    x = (x / x.norm(dim=-1, keepdim=True))[0].bfloat16()
    ref, st = _assignment(o_ref), _assignment(o_st)
    assert ref.keys() == st.keys()
    differ = 0
    for s in ref:
        assert ref[s][0] == st[s][0]                      # same max score
        if ref[s][1] != st[s][1]:
            differ += 1
            s_ref = (x[s].float() @ x[ref[s][1]].float()).bfloat16()
            s_st = (x[s].float() @ x[st[s][1]].float()).bfloat16()
            assert s_ref == s_st                          # a tie in bf16
    assert differ < len(ref)


@pytest.mark.parametrize("frames,w,h,sx,sy,ns,no_rand", [
    (200, 37, 37, 2, 2, 5, False), (100, 37, 37, 2, 2, 5, False), (4, 37, 37, 2, 2, 5, False),
    (5, 7, 5, 2, 2, 5, False), (3, 9, 9, 3, 3, 1, False), (6, 6, 6, 2, 2, 5, True),
])
def test_dst_count_closed_form(frames, w, h, sx, sy, ns, no_rand):
    cell = window_draw(frames, w, h, sx, sy, torch.Generator().manual_seed(33))
    mask = build_dst_mask(frames, w, h, sx, sy, ns, no_rand, cell)
    per = ns + (0 if no_rand else (h // sy) * (w // sx))
    expect = (w * h + ns) + (frames - 1) * per
    assert int((mask == -1).sum()) == expect
    if (frames, w) == (200, 37):
        assert expect == 66_845          # 200-frame destination count
    if (frames, w) == (100, 37):
        assert expect == 33_945


def test_window_cells_are_one_per_window():
    frames, w, h, s = 3, 9, 7, 2
    cell = window_draw(frames, w, h, s, s, torch.Generator().manual_seed(5))
    mask = build_dst_mask(frames, w, h, s, s, 2, False, cell)
    tpi = w * h + 2
    row = (w // s) * s
    for f in range(1, frames):
        pat = mask[f * tpi + 2: f * tpi + 2 + (h // s) * s * row].view((h // s) * s, row)
        win = pat.view(h // s, s, w // s, s).permute(0, 2, 1, 3).reshape(h // s, w // s, s * s)
        assert torch.equal((win == -1).sum(-1), torch.ones(h // s, w // s, dtype=torch.int64))
        picked = (win == -1).float().argmax(-1)
        assert torch.equal(picked, cell[f - 1])
        assert (mask[f * tpi + 2 + (h // s) * s * row:(f + 1) * tpi] == 0).all()


@pytest.mark.parametrize("r", [10_000, 40, 1])
def test_invariants_and_brute_force_heads(r):
    g = torch.Generator().manual_seed(11)
    frames, w, h, ns = 4, 8, 6, 5
    n = frames * (w * h + ns)
    metric = torch.randn(1, n, 64, generator=g)
    o = token_merge_reference(metric, w, h, 2, 2, r, False, torch.Generator().manual_seed(33),
                              metric_dim=16, num_special=ns)
    assert o.size.sum().item() == n
    assert (o.size >= 1).all()
    assert o.size.shape[1] == n - o.r
    if r >= o.num_src:
        assert o.unm_len == 0
    t = torch.randn(1, 3, n, 8, generator=g, dtype=torch.float64)
    got = o.heads(t, "mean")[0].numpy()
    want = merge_heads_fp64(t[0].numpy(), o.unm_abs_idx[0].numpy(), o.b_idx.numpy(),
                            o.src_abs_idx[0].numpy(), o.dst_idx[0].numpy())
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12)
    # counts from the merge itself equal merge.size
    ones = torch.ones(1, n, 1, dtype=torch.float64)
    assert torch.equal(o.merge(ones, "sum")[0, :, 0].float(), o.size[0])


def test_invalid_arguments():
    metric = torch.randn(1, 2 * (4 * 4 + 5), 16)
    with pytest.raises(ValueError):
        token_merge_reference(metric, 4, 4, 2, 2, 0)
    with pytest.raises(AssertionError):
        token_merge_reference(metric[:, :-1], 4, 4, 2, 2, 3)
