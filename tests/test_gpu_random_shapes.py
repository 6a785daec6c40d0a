"""Seeded random-shape sweep of the two hot-path operators against the oracle.

Each case draws its sizes, head or feature dim, operand format, bias kind and
memory layout from a fixed seed, so the sweep covers combinations the
hand-picked tests do not (ragged key and query counts next to every head dim,
head-transposed views, head-broadcast and wide-range biases, batched
similarity with fp32 inputs) and stays the same from run to run.

Bars, as in the hand-picked tests:
  * attention_keybias (merging/fused_attention.py:130-180): output within
    2e-2 max-abs and 5e-3 mean-abs of the fp32 oracle on the same 16-bit
    inputs, log2 LSE within 2^-8 / ln 2;
  * fused_similarity_argmax (merging/fused_similarity.py:81-112): max within
    1e-5 of the fp64 brute force on the same 16-bit inputs, the index equal
    to the fp64 argmax wherever the top-2 gap exceeds 1e-5, and every chosen
    index scoring within 1e-5 of the row max.
"""
import math

import numpy as np
import pytest
import torch

from merging.fused_attention import attention_keybias
from merging.fused_similarity import fused_similarity_argmax
from oracle.attention import attention_reference

pytestmark = pytest.mark.gpu

ATTN_MAX, ATTN_MEAN = 2e-2, 5e-3
LSE_TOL = 2.0 ** -8 / math.log(2.0) + 1e-5


def _log_uniform(rng, lo, hi):
    return int(round(math.exp(rng.uniform(math.log(lo), math.log(hi)))))


def _attention_cases(n=80, seed=2024):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        D = int(rng.choice([16, 32, 64, 64, 64, 128, 256]))
        B, H = int(rng.integers(1, 4)), int(rng.integers(1, 5))
        M, N = _log_uniform(rng, 1, 3000), _log_uniform(rng, 1, 6000)
        if B * H * M * N * D > 3e9:                  # keeps the CPU oracle to seconds
            continue
        cases.append(dict(
            B=B, H=H, M=M, N=N, D=D,
            dtype=str(rng.choice(["bf16", "f16"])),
            bias=str(rng.choice(["none", "f32", "same", "f32_heads", "wide"])),
            layout=str(rng.choice(["contiguous", "heads_inner"])),
            qk=float(rng.choice([0.5, 1.0, 2.0])),
            lse=bool(rng.integers(0, 2)),
            seed=int(rng.integers(0, 1 << 30))))
    return cases


def _attention_inputs(c):
    B, H, M, N, D = c["B"], c["H"], c["M"], c["N"], c["D"]
    dtype = torch.bfloat16 if c["dtype"] == "bf16" else torch.float16
    g = torch.Generator().manual_seed(c["seed"])
    s = c["qk"] * (64.0 / D) ** 0.25                   # logit spread independent of D
    if c["layout"] == "heads_inner":                   # [B, T, H, D] storage, heads-major view
        q = (torch.randn(B, M, H, D, generator=g) * s).to(dtype).permute(0, 2, 1, 3)
        k = (torch.randn(B, N, H, D, generator=g) * s).to(dtype).permute(0, 2, 1, 3)
        v = torch.randn(B, N, H, D, generator=g).to(dtype).permute(0, 2, 1, 3)
    else:
        q = (torch.randn(B, H, M, D, generator=g) * s).to(dtype)
        k = (torch.randn(B, H, N, D, generator=g) * s).to(dtype)
        v = torch.randn(B, H, N, D, generator=g).to(dtype)
    counts = torch.randint(1, 9, (B, 1, 1, N), generator=g).float()
    if c["bias"] == "none":
        b = None
    elif c["bias"] == "f32":
        b = counts.log().expand(B, H, 1, N).contiguous()
    elif c["bias"] == "same":
        b = counts.log().expand(B, H, 1, N).to(dtype).contiguous()
    elif c["bias"] == "f32_heads":
        b = counts.log()                               # [B, 1, 1, N], broadcast over heads
    else:                                              # wide range, per head
        b = torch.randn(B, H, 1, N, generator=g) * 4.0
    return q, k, v, b, D ** -0.5


CASES = _attention_cases()


@pytest.mark.parametrize("case", range(len(CASES)))
def test_attention_random_shape(dev, case):
    c = CASES[case]
    print(f"\n[attn sweep {case}] {c}", flush=True)
    q, k, v, b, scale = _attention_inputs(c)
    args = (q.to(dev), k.to(dev), v.to(dev), None if b is None else b.to(dev), scale)
    if c["lse"]:
        o, lse = attention_keybias(*args, return_lse=True)
    else:
        o, lse = attention_keybias(*args), None
    assert o.shape == q.shape and o.dtype == q.dtype
    ref, ref_lse = attention_reference(q, k, v, b, scale)
    err = (o.float().cpu() - ref).abs()
    assert err.max().item() <= ATTN_MAX, err.max().item()
    assert err.mean().item() <= ATTN_MEAN, err.mean().item()
    # each row at its own scale too: |o - ref|_2 / |ref|_2 (16-bit P and output)
    rel = ((o.float().cpu() - ref).norm(dim=-1) / ref.norm(dim=-1)).max().item()
    assert rel <= 2e-2, rel
    if lse is not None:
        assert (lse.cpu() - ref_lse).abs().max().item() < LSE_TOL


def _similarity_cases(n=60, seed=4048):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        D = int(rng.choice([32, 64, 96, 128, 128, 160, 256, 288, 512, 640, 1024]))
        B = int(rng.integers(1, 3))
        M, N = _log_uniform(rng, 1, 6000), _log_uniform(rng, 1, 40_000)
        if B * M * N * D > 6e9:                        # keeps the fp64 brute force to seconds
            continue
        cases.append(dict(B=B, M=M, N=N, D=D,
                          fmt=str(rng.choice(["bf16", "f16", "f32"])),
                          strided=bool(rng.integers(0, 2)),
                          seed=int(rng.integers(0, 1 << 30))))
    return cases


def _fp64_argmax(a, b, chunk=2048):
    """Row max, first argmax and top-2 gap of a @ b^T in fp64."""
    a64, b64 = a.double().numpy(), b.double().numpy()
    bsz, m, _ = a64.shape
    vmax, vidx = np.empty((bsz, m)), np.empty((bsz, m), dtype=np.int64)
    gap = np.full((bsz, m), np.inf)
    for bi in range(bsz):
        bt = np.ascontiguousarray(b64[bi].T)
        for lo in range(0, m, chunk):
            s = a64[bi, lo:lo + chunk] @ bt
            idx = np.argmax(s, axis=1)
            top = s[np.arange(s.shape[0]), idx]
            vmax[bi, lo:lo + chunk], vidx[bi, lo:lo + chunk] = top, idx
            if s.shape[1] > 1:
                s[np.arange(s.shape[0]), idx] = -np.inf
                gap[bi, lo:lo + chunk] = top - s.max(axis=1)
    return vmax, vidx, gap


SIM_CASES = _similarity_cases() + [                    # the 1024-d metric in every run
    dict(B=1, M=300, N=9000, D=1024, fmt="bf16", strided=True, seed=11),
    dict(B=2, M=1000, N=1300, D=1024, fmt="f32", strided=False, seed=12),
    dict(B=1, M=257, N=5000, D=1024, fmt="f16", strided=False, seed=13),
]


@pytest.mark.parametrize("case", range(len(SIM_CASES)))
def test_similarity_random_shape(dev, case):
    c = SIM_CASES[case]
    print(f"\n[sim sweep {case}] {c}", flush=True)
    B, M, N, D = c["B"], c["M"], c["N"], c["D"]
    g = torch.Generator().manual_seed(c["seed"])
    # 16-bit-representable unit rows (fp32 inputs are cast to bf16 by the
    # wrapper, so their values are bf16-representable too)
    kernel_dtype = torch.float16 if c["fmt"] == "f16" else torch.bfloat16
    a = torch.randn(B, M, D, generator=g)
    b = torch.randn(B, N, D, generator=g)
    a = (a / a.norm(dim=-1, keepdim=True)).to(kernel_dtype).float()
    b = (b / b.norm(dim=-1, keepdim=True)).to(kernel_dtype).float()
    in_dtype = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[c["fmt"]]
    if c["strided"]:                                   # row views into wider rows
        a_d = torch.zeros(B, M, D + 32, dtype=in_dtype, device=dev)[..., 16:16 + D]
        b_d = torch.zeros(B, N, D + 64, dtype=in_dtype, device=dev)[..., :D]
        a_d.copy_(a.to(dev, in_dtype))
        b_d.copy_(b.to(dev, in_dtype))
    else:
        a_d, b_d = a.to(dev, in_dtype), b.to(dev, in_dtype)
    vmax, vidx = fused_similarity_argmax(a_d, b_d)
    assert vmax.dtype == in_dtype and vidx.dtype == torch.int64
    assert vmax.shape == (B, M) and vidx.shape == (B, M)
    fmax, fidx, gap = _fp64_argmax(a, b)
    vidx = vidx.cpu().numpy()
    assert vidx.min() >= 0 and vidx.max() < N
    # the max comes back in a's dtype: compare within that rounding
    tol = 1e-5 if in_dtype == torch.float32 else 1e-5 + 2.0 ** -8
    assert np.abs(vmax.float().cpu().numpy() - fmax).max() < tol
    sure = gap > 1e-5
    assert np.array_equal(vidx[sure], fidx[sure])
    a64, b64 = a.double().numpy(), b.double().numpy()
    chosen = np.einsum("bmd,bmd->bm", a64, np.take_along_axis(b64, vidx[..., None], axis=1))
    assert np.abs(chosen - fmax).max() < 1e-5
