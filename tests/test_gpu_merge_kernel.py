"""The deterministic segmented merge kernel (gpa::merge_heads) on its own.

Against an fp64 brute force over random slot lists: every input token in
exactly one list, lists in arbitrary order, B > 1, strided inputs, fp32 /
bf16 / fp16 rows, sum and mean.  Bars: fp32 within fp32 summation error;
16-bit outputs within one rounding of the exact value (2^-8 relative for
bf16, 2^-11 for fp16).  Out-of-range list entries are caught by the kernel
(the slot becomes NaN; nothing is read out of bounds).
"""
import math

import numpy as np
import pytest
import torch

from merging import _native

pytestmark = pytest.mark.gpu


def _random_lists(B, N, S, g):
    """Random partition of each batch element's N tokens into S non-empty
    lists: (offsets [B*S+1], tokens [B*N], lists as python lists)."""
    offsets, tokens, lists = [0], [], []
    for _ in range(B):
        perm = torch.randperm(N, generator=g)
        cuts = torch.sort(torch.randperm(N - 1, generator=g)[: S - 1] + 1).values.tolist()
        bounds = [0] + cuts + [N]
        for s in range(S):
            lst = perm[bounds[s]:bounds[s + 1]].tolist()
            lists.append(lst)
            tokens.extend(lst)
            offsets.append(offsets[-1] + len(lst))
    return (torch.tensor(offsets, dtype=torch.int64), torch.tensor(tokens, dtype=torch.int64),
            lists)


def _fp64(t, lists, B, S, mean):
    t64 = t.double().numpy()
    H, D = t64.shape[1], t64.shape[3]
    out = np.zeros((B, H, S, D))
    for b in range(B):
        for s in range(S):
            lst = lists[b * S + s]
            acc = t64[b][:, lst, :].sum(axis=1)
            out[b, :, s] = acc / len(lst) if mean else acc
    return out


@pytest.mark.parametrize("dtype,rel", [(torch.float32, 1e-6), (torch.bfloat16, 2.0 ** -8),
                                       (torch.float16, 2.0 ** -11)])
@pytest.mark.parametrize("mean", [True, False])
@pytest.mark.parametrize("B,H,N,S,D", [(1, 4, 300, 77, 64), (2, 3, 257, 40, 64), (1, 1, 130, 9, 1024),
                                       (3, 2, 1, 1, 8), (1, 16, 5000, 1300, 64)])
def test_matches_fp64(dev, dtype, rel, mean, B, H, N, S, D):
    g = torch.Generator().manual_seed(B * 1000 + N + S)
    t = torch.randn(B, H, N, D, generator=g).to(dtype)
    off, tok, lists = _random_lists(B, N, S, g)
    out, size, log_size = _native.merge_heads(t.to(dev), off.to(dev), tok.to(dev), S, mean)
    assert out.shape == (B, H, S, D) and out.dtype == dtype
    ref = _fp64(t, lists, B, S, mean)
    got = out.double().cpu().numpy()
    assert (np.abs(got - ref) <= rel * np.abs(ref) + 1e-5).all(), np.abs(got - ref).max()
    counts = np.array([len(x) for x in lists], dtype=np.float32).reshape(B, S)
    assert np.array_equal(size.cpu().numpy(), counts)
    np.testing.assert_allclose(log_size.cpu().numpy(), np.log(counts), rtol=1e-6, atol=1e-7)


def test_strided_heads_view(dev):
    """K as a permuted view of a [B, N, H, D] projection (no copy)."""
    g = torch.Generator().manual_seed(3)
    B, N, H, D, S = 2, 400, 4, 64, 100
    base = torch.randn(B, N, H, D, generator=g).to(dev)
    t = base.permute(0, 2, 1, 3)
    assert not t.is_contiguous()
    off, tok, lists = _random_lists(B, N, S, g)
    out, _, _ = _native.merge_heads(t, off.to(dev), tok.to(dev), S, True)
    ref = _fp64(t.cpu(), lists, B, S, True)
    assert np.abs(out.double().cpu().numpy() - ref).max() < 1e-5


def test_bit_identical_repeats(dev):
    g = torch.Generator().manual_seed(4)
    t = torch.randn(1, 8, 3000, 64, generator=g).bfloat16().to(dev)
    off, tok, _ = _random_lists(1, 3000, 500, g)
    off, tok = off.to(dev), tok.to(dev)
    a = _native.merge_heads(t, off, tok, 500, True)[0]
    for _ in range(3):
        assert torch.equal(a, _native.merge_heads(t, off, tok, 500, True)[0])


def test_out_of_range_entries_poison_only_their_slot(dev):
    g = torch.Generator().manual_seed(5)
    B, H, N, D, S = 1, 2, 100, 64, 10
    t = torch.randn(B, H, N, D, generator=g)
    off, tok, lists = _random_lists(B, N, S, g)
    bad = tok.clone()
    bad[int(off[3])] = N            # first entry of slot 3: one past the end
    bad[int(off[7])] = -5           # first entry of slot 7: negative
    out, size, _ = _native.merge_heads(t.to(dev), off.to(dev), bad.to(dev), S, True)
    out = out.cpu()
    ref = _fp64(t, lists, B, S, True)
    for s in range(S):
        if s in (3, 7):
            assert torch.isnan(out[0, :, s]).all()
        else:
            assert np.abs(out[0, :, s].double().numpy() - ref[0, :, s]).max() < 1e-5
    # a list running past the token array is refused the same way
    off2 = off.clone()
    off2[-1] = B * N + 7
    out2, size2, _ = _native.merge_heads(t.to(dev), off2.to(dev), tok.to(dev), S, True)
    assert torch.isnan(out2[0, :, S - 1].cpu()).all() and math.isnan(size2[0, S - 1].item())


def test_argument_checks(dev):
    t = torch.randn(1, 2, 10, 64, device=dev)
    off = torch.tensor([0, 10], device=dev)
    tok = torch.arange(10, device=dev)
    with pytest.raises(ValueError):
        _native.merge_heads(t, off, tok, 2, True)            # offsets size mismatch
    with pytest.raises(ValueError):
        _native.merge_heads(t, off.int(), tok, 1, True)      # wrong index dtype
    with pytest.raises(NotImplementedError):
        _native.merge_heads(t.double(), off, tok, 1, True)
