"""The torch.library registration of every custom op: `torch.library.opcheck`
(schema, fake implementation against the real op's outputs, AOT dispatch
with dynamic shapes) on small inputs, and a compiled graph (fullgraph,
`aot_eager`, which traces through the fake implementations and generates
no kernels of its own) equal to the eager calls bit for bit.  What the
ops compute is pinned elsewhere; here only that a traced or compiled
caller sees the same ops, shapes and dtypes."""
import pytest
import torch

import gpa_aggregator as A
from merging import _native  # noqa: F401  (registers the ops)
from merging.fused_attention import attention_keybias
from merging.fused_similarity import fused_similarity_argmax

pytestmark = pytest.mark.gpu


def _g(seed):
    return torch.Generator(device="cuda").manual_seed(seed)


def _op_cases(dev):
    g = _g(0)
    bf = torch.bfloat16
    a = torch.randn(1, 300, 128, device=dev, generator=g).to(bf)
    b = torch.randn(1, 70, 128, device=dev, generator=g).to(bf)
    q = torch.randn(2, 3, 100, 64, device=dev, generator=g).to(bf)
    k = torch.randn(2, 3, 50, 64, device=dev, generator=g).to(bf)
    v = torch.randn(2, 3, 50, 64, device=dev, generator=g).to(bf)
    bias = torch.randn(2, 3, 1, 50, device=dev, generator=g)
    t = torch.randn(1, 2, 40, 64, device=dev, generator=g)
    tokens = torch.randperm(40, device=dev, generator=g)
    offsets = torch.tensor([0, 3, 10, 11, 25, 40], device=dev)
    frames, P = 3, 41                         # 5 specials + 6 x 6 patches
    oa = torch.randn(frames, 2, P, 64, device=dev, generator=g).to(bf)
    la = torch.randn(frames, 2, P, device=dev, generator=g)
    ob = torch.randn(1, 2, frames * P, 64, device=dev, generator=g).to(bf)
    lb = torch.randn(1, 2, frames * P, device=dev, generator=g)
    qkv = torch.randn(1, frames * P, 3 * 2 * 64, device=dev, generator=g).to(bf)
    ln = torch.randn(2, 64, device=dev, generator=g)
    rope = A.Rope2D(100.0).table(A.frame_positions(6, 5, dev), 64)
    kk = torch.randn(1, 2, frames * P, 64, device=dev, generator=g).to(bf)
    metric = torch.randn(1, 200, 256, device=dev, generator=g)
    proj = torch.randn(256, 128, device=dev, generator=g).to(bf)
    order = torch.randperm(200, device=dev, generator=g)
    x = torch.randn(64, 512, device=dev, generator=g).to(bf)
    y = torch.randn(64, 512, device=dev, generator=g).to(bf)
    w = torch.randn(512, device=dev, generator=g).to(bf)
    return [
        ("sim_argmax", torch.ops.gpa.sim_argmax, (a, b, False)),
        ("attn_keybias", torch.ops.gpa.attn_keybias, (q, k, v, bias, 0.125, True)),
        ("attn_keybias_nobias", torch.ops.gpa.attn_keybias, (q, k, v, None, 0.125, False)),
        ("merge_heads", torch.ops.gpa.merge_heads, (t, offsets, tokens, 5, True)),
        ("lse_combine", torch.ops.gpa.lse_combine, (oa, la, ob, lb, frames)),
        ("qk_norm_rope", torch.ops.gpa.qk_norm_rope,
         (qkv, ln, ln, 1e-6, rope.pos, rope.cs, 2, False, True)),
        ("pool_shared", torch.ops.gpa.pool_shared, (kk, kk, frames, 5, 6, 6, 2, True)),
        ("merge_metric", torch.ops.gpa.merge_metric, (metric, proj, order, 0)),
        ("residual_layernorm", torch.ops.gpa.residual_layernorm, (x, y, w, w, w, 1e-6, True)),
    ]


@pytest.mark.parametrize("case", range(9))
def test_opcheck(dev, case):
    name, op, args = _op_cases(dev)[case]
    torch.library.opcheck(op, args)


def test_compiled_graph_matches_eager(dev):
    """The drop-in entry points in one fullgraph-compiled function (the
    similarity, its indices gathering the keys, the biased attention with
    the LSE) give the eager results bit for bit."""
    g = _g(1)
    a = torch.randn(1, 2000, 128, device=dev, generator=g)
    b = torch.randn(1, 500, 128, device=dev, generator=g)
    q = torch.randn(1, 4, 700, 64, device=dev, generator=g).bfloat16()
    kv = torch.randn(1, 4, 500, 64, device=dev, generator=g).bfloat16()

    def fn(a, b, q, kv):
        node_max, node_idx = fused_similarity_argmax(a / a.norm(dim=-1, keepdim=True),
                                                     b / b.norm(dim=-1, keepdim=True))
        counts = torch.ones(b.shape[1], device=a.device).scatter_add(
            0, node_idx[0], torch.ones_like(node_max[0]))
        bias = counts.log().view(1, 1, 1, -1).expand(1, 4, 1, -1)
        o, lse = attention_keybias(q, kv, kv, bias, 0.125, return_lse=True)
        return node_max, node_idx, o, lse

    eager = fn(a, b, q, kv)
    compiled = torch.compile(fn, backend="aot_eager", fullgraph=True)(a, b, q, kv)
    for e, c in zip(eager, compiled):
        assert e.dtype == c.dtype and e.shape == c.shape
        assert torch.equal(e, c)
