"""The allocation-free attention entry point against the allocating one.

`gpa_attn_keybias_bf16_noalloc` runs the same kernels as
`gpa_attn_keybias_bf16` with the library's static device scratch as the
workspace, so on the same inputs its outputs must be bit-identical.  Two
calls in a row (the second on a smaller problem, so stale scratch contents
from the first call are present) with a bias, the LSE and sharp logits that
send some waves onto the lazily moved offset (whose flags live in the
scratch); both calls go through the C ABI directly.  At head dim 128 the
tiled kernel keeps its fp32 bias rows in the same scratch.
"""
import ctypes

import pytest
import torch

from merging import _native

pytestmark = pytest.mark.gpu

SM_SCALE = 0.125


def _inputs(dev, B, H, M, N, q_scale, seed, D=64):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = (torch.randn(B, H, M, D, generator=g) * q_scale).bfloat16().to(dev)
    k = torch.randn(B, H, N, D, generator=g).bfloat16().to(dev)
    v = torch.randn(B, H, N, D, generator=g).bfloat16().to(dev)
    bias = torch.randint(1, 9, (B, 1, 1, N), generator=g).float().log().to(dev)
    return q, k, v, bias.expand(B, H, 1, N)


def _strides(t):
    return t.stride(0), t.stride(1), t.stride(2)


def _call(noalloc, q, k, v, bias, o, lse, ws=None):
    L = _native.lib()
    B, H, M, D = q.shape
    N = k.shape[2]
    stream = torch.cuda.current_stream(q.device).cuda_stream
    if bias is None:
        bias_args = [None, _native.GPA_BIAS_NONE, 0, 0, 0]
    else:
        bias_args = [bias.data_ptr(), _native.GPA_BIAS_F32, bias.stride(0), bias.stride(1),
                     bias.stride(3)]
    args = [q.data_ptr(), k.data_ptr(), v.data_ptr(), *bias_args, o.data_ptr(), lse.data_ptr(),
            B, H, M, N, D, *_strides(q), *_strides(k), *_strides(v), *_strides(o),
            lse.stride(0), lse.stride(1)]
    if noalloc:
        rc = L.gpa_attn_keybias_bf16_noalloc(*args, ctypes.c_float(SM_SCALE), stream)
    else:
        rc = L.gpa_attn_keybias_bf16(*args, ws.data_ptr(), ws.numel(), ctypes.c_float(SM_SCALE),
                                     stream)
    assert rc == _native.GPA_OK, L.gpa_last_error()


def _run_pair(dev, B, H, M, N, q_scale, seed, with_bias=True, D=64):
    q, k, v, bias = _inputs(dev, B, H, M, N, q_scale, seed, D)
    if not with_bias:
        bias = None
    ws_bytes = _native.lib().gpa_attn_keybias_workspace_bytes(B, H, M, N)
    assert 0 < ws_bytes <= _native.NOALLOC_SCRATCH_BYTES
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    o_ref = torch.empty(B, H, M, D, device=dev, dtype=torch.bfloat16)
    lse_ref = torch.empty(B, H, M, device=dev, dtype=torch.float32)
    o = torch.full_like(o_ref, float("nan"))
    lse = torch.full_like(lse_ref, float("nan"))
    _call(False, q, k, v, bias, o_ref, lse_ref, ws)
    _call(True, q, k, v, bias, o, lse)
    torch.cuda.synchronize()
    assert torch.isfinite(o_ref.float()).all() and torch.isfinite(lse_ref).all()
    assert torch.equal(o.view(torch.int16), o_ref.view(torch.int16))
    assert torch.equal(lse.view(torch.int32), lse_ref.view(torch.int32))
    return ws


def test_noalloc_matches_allocating_entry_point_twice(dev):
    print("[no-alloc] call 1: B=2 H=4 M=3000 N=2100, sharp logits", flush=True)
    _run_pair(dev, 2, 4, 3000, 2100, 4.0, 0)
    print("[no-alloc] call 2: B=1 H=2 M=700 N=333, smaller", flush=True)
    _run_pair(dev, 1, 2, 700, 333, 0.5, 1)


def test_noalloc_without_bias_after_biased_calls(dev):
    print("[no-alloc] biased call: B=2 H=4 M=3000 N=2100, sharp logits", flush=True)
    _run_pair(dev, 2, 4, 3000, 2100, 4.0, 2)
    print("[no-alloc] call without bias: B=8 H=16 M=1374 N=1369 (own-frame shape)", flush=True)
    _run_pair(dev, 8, 16, 1374, 1369, 0.5, 3, with_bias=False)
    print("[no-alloc] call without bias: B=3 H=16 M=1374 N=1369, smaller", flush=True)
    _run_pair(dev, 3, 16, 1374, 1369, 2.0, 4, with_bias=False)


def test_noalloc_head_dim_128_after_other_calls(dev):
    """Head dim 128 (the tiled kernel, bias rows in the scratch) after a head
    dim 64 call has left records and flags there, then a smaller call
    without bias over the first call's bias rows."""
    print("[no-alloc] head dim 64 call: B=2 H=4 M=3000 N=2100", flush=True)
    _run_pair(dev, 2, 4, 3000, 2100, 1.0, 5)
    print("[no-alloc] head dim 128 call: B=1 H=8 M=2000 N=3001, q x 3", flush=True)
    _run_pair(dev, 1, 8, 2000, 3001, 3.0, 6, D=128)
    print("[no-alloc] head dim 128 call without bias: B=1 H=4 M=600 N=999, smaller", flush=True)
    _run_pair(dev, 1, 4, 600, 999, 0.5, 7, with_bias=False, D=128)
