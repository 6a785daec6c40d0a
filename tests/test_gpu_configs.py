"""The two end-to-end workloads at their full size, on the GPU.

* One merged GPA global block of a random-init VGGT-1B aggregator on 100
  frames x 1374 tokens (137,400 tokens -> 33,945 merged keys; block 9 of
  vggt/models/aggregator.py:133-150 at merge ratio 0.98), its tokens made by
  the harness's own patch embedder from shifted-texture images:
  - the block is exactly LayerNorm -> QKV + qk-norm/RoPE -> merge -> K/V
    means -> biased attention -> proj -> residual + LayerNorm -> MLP ->
    residual (recomposed step by step, bit-identical), and bit-identical on
    a second call;
  - merge invariants: the closed-form destination count, every source
    merged (r >= number of sources), sizes >= 1 summing to the token count,
    slot lists that partition the tokens;
  - the merge's orders are those of the reference's own argsort calls on
    the device (merging/merge.py:165 and :199);
  - similarity row max / argmax on 512 sampled source rows against the
    fp64 brute force over all 33,945 destinations (index exact where the
    top-2 gap exceeds 1e-5);
  - K and V slot means on 256 sampled slots against fp64 means;
  - the attention output on 64 sampled query rows x 16 heads against the
    oracle over all 33,945 merged keys (max-abs <= 2e-2, mean-abs <= 2e-3).
* The whole 200-frame aggregator (DINOv2 patch embed, 24 frame + 24 global
  blocks), on the reference's default GPA schedule and on the schedule the
  200-frame workload states (64 pooled summaries per frame, 25 % keep in
  every merged block): finite outputs of the DPT shapes, bit-identical on a
  second forward, and for every merged block the slot count (66,845, or
  219,840 in the core blocks 13-16), sizes summing to 274,800, and every
  frame-special pooling's group sizes summing to the 1,369 patches of each
  frame.
"""
import numpy as np
import pytest
import torch

import gpa_aggregator as A
from merging import _native
from merging.fused_attention import attention_keybias
from merging.merge import _projection, num_dst_tokens, token_merge_bipartite2d
from oracle.attention import attention_reference
from oracle.similarity import bf16_round, sim_argmax_fp64

pytestmark = pytest.mark.gpu

GRID, PTS, P = 37, 5, 1374
BF16 = torch.bfloat16


@pytest.fixture(scope="module")
def aggregator(dev):
    cfg = A.GpaConfig()
    return cfg, A.build_aggregator(cfg, device=dev, seed=0)


def test_config4_merged_block_100_frames(dev, aggregator):
    cfg, agg = aggregator
    frames = 100
    imgs = A.shifted_texture_images(frames, device=dev).to(BF16)
    with torch.no_grad(), torch.autocast("cuda", dtype=BF16):
        x = agg.embed(imgs).reshape(1, frames * P, cfg.embed_dim)
    del imgs
    N = x.shape[1]
    rope = agg.rope_table(dev)
    blk = agg.global_blocks[9]
    assert cfg.block_kind(9) == "merged" and blk.attn.merge_ratio == 0.98
    print(f"[config 4] block 9 on {N} tokens", flush=True)

    log = []
    blk.attn.merge_log = log
    with torch.no_grad(), torch.autocast("cuda", dtype=BF16):
        y1 = blk(x, rope, 9)
        y2 = blk(x, rope, 9)
    blk.attn.merge_log = None
    torch.cuda.synchronize()
    assert y1.shape == x.shape and y1.dtype == BF16 and torch.isfinite(y1).all()
    assert torch.equal(y1, y2), "the block is not bit-reproducible"

    nd = num_dst_tokens(frames, GRID, GRID, 2, 2, PTS, False)
    assert nd == 1374 + 99 * (5 + 18 * 18) == 33_945
    assert len(log) == 2
    for rec in log:
        assert rec["num_dst"] == nd and rec["keys"] == nd and rec["r"] == N - nd
        size = rec["size"]
        assert size.shape == (1, nd)
        assert size.sum().item() == N and size.min().item() >= 1
        assert torch.equal(size, size.round())
        assert rec["slot_offsets"][-1].item() == N
    assert torch.equal(log[0]["size"], log[1]["size"])

    # The block recomposed step by step from its parts.
    at = blk.attn
    rl = torch.ops.gpa.residual_layernorm
    with torch.no_grad(), torch.autocast("cuda", dtype=BF16):
        _, ln1 = rl(x, None, None, blk.norm1.weight, blk.norm1.bias, blk.norm1.eps, False)
        gen = torch.Generator(device=dev)
        gen.manual_seed(A.MERGE_GENERATOR_SEED)
        m = token_merge_bipartite2d(ln1, GRID, GRID, 2, 2, int(N * 0.98), False, gen,
                                    metric_dim=128, num_special=PTS)
        q, k, v = at.qk(ln1, rope, k_f32=True)
        km, vm = m.heads(k, "mean"), m.heads(v, "mean")
        bias = m.size.reshape(1, 1, 1, -1).log().to(q.dtype).expand(1, 16, 1, km.shape[2])
        o = attention_keybias(q, km, vm, bias, at.scale)
        a = at.proj(o.transpose(1, 2).reshape(1, N, cfg.embed_dim))
        h, ln2 = rl(x, a, blk.ls1.gamma, blk.norm2.weight, blk.norm2.bias, blk.norm2.eps, True)
        y3, _ = rl(h, blk.mlp(ln2), blk.ls2.gamma, None, None, 0.0, True)
    torch.cuda.synchronize()
    assert torch.equal(y3, y1), "the block differs from its step-by-step composition"
    assert torch.equal(m.size, log[0]["size"])

    ix = m.index
    # The orders are the reference's own argsort calls on this device.
    ref_order = ix.mask.reshape(1, -1, 1).argsort(dim=1).view(-1)          # merge.py:165
    assert torch.equal(torch.cat([ix.b_idx, ix.a_idx]), ref_order)
    ref_edge = ix.node_max.argsort(dim=-1, descending=True)               # merge.py:199
    assert torch.equal(ix.edge_idx, ref_edge)
    # The slot lists partition the tokens.
    tok_sorted = torch.sort(ix.slot_tokens).values
    assert torch.equal(tok_sorted, torch.arange(N, device=dev))
    assert int(ix.node_idx.min()) >= 0 and int(ix.node_idx.max()) < nd

    cpu = torch.Generator().manual_seed(4)
    # Similarity on sampled source rows, from the front end's own operands.
    order = torch.cat([ix.b_idx, ix.a_idx])
    with torch.no_grad(), torch.autocast("cuda", dtype=BF16):
        ab = _native.merge_metric(ln1, _projection(dev, cfg.embed_dim, 128), order, 0)
    a_op, b_op = ab[:, nd:], ab[:, :nd]
    rows = torch.randperm(N - nd, generator=cpu)[:512]
    # the front end on those rows: fp64 chain on the same bf16 operands
    t = ln1[0, ix.a_idx[rows.to(dev)]].double().cpu()
    y = bf16_round(t @ _projection(dev, cfg.embed_dim, 128).double().cpu()).double()
    want_ab = y / y.norm(dim=-1, keepdim=True)
    got_ab = a_op[0, rows.to(dev)].double().cpu()
    assert ((got_ab - want_ab).abs() <= 3 * 2.0 ** -8 * want_ab.abs() + 2.0 ** -16).all()
    fmax, fidx, gap = sim_argmax_fp64(a_op[:, rows.to(dev)].float().cpu(), b_op.float().cpu())
    got_idx = ix.node_idx[0, rows.to(dev)].cpu().numpy()
    got_max = ix.node_max[0, rows.to(dev)].double().cpu().numpy()
    sure = gap[0] > 1e-5
    print(f"[config 4] similarity: {int(sure.sum())}/512 sampled rows with a top-2 gap > 1e-5",
          flush=True)
    assert sure.mean() > 0.8
    assert np.array_equal(got_idx[sure], fidx[0][sure])
    assert np.abs(got_max - fmax[0]).max() < 1e-5

    # K / V slot means on sampled slots, against fp64 means over the lists.
    off = ix.slot_offsets.cpu()
    slots = torch.randperm(nd, generator=cpu)[:256]
    seg = torch.cat([torch.full((int(off[s + 1] - off[s]),), i) for i, s in enumerate(slots)])
    toks = torch.cat([ix.slot_tokens[int(off[s]):int(off[s + 1])].cpu() for s in slots])
    cnt = torch.bincount(seg, minlength=len(slots)).double()
    for src, merged, tol in ((k, km, 2.0 ** -20), (v, vm, 2.0 ** -8)):
        rows_t = src[0][:, toks.to(dev)].double().cpu()                     # [16, T, 64]
        sums = torch.zeros(16, len(slots), 64, dtype=torch.float64).index_add_(1, seg, rows_t)
        want = sums / cnt.view(1, -1, 1)
        got = merged[0][:, slots.to(dev)].double().cpu()
        assert ((got - want).abs() <= tol * want.abs() + 1e-6).all(), \
            f"{merged.dtype} slot means off by {(got - want).abs().max().item():.3e}"

    # Attention on sampled query rows against the oracle over every key.
    qrows = torch.randperm(N, generator=cpu)[:64].to(dev)
    ref_o, _ = attention_reference(q[:, :, qrows], km.to(BF16), vm, bias, at.scale)
    got = o[:, :, qrows].float().cpu()
    err = (got - ref_o).abs()
    rel = ((got - ref_o).norm(dim=-1) / ref_o.norm(dim=-1)).max().item()
    print(f"[config 4] attention on 64 x 16 rows: max-abs {err.max().item():.2e}, mean-abs "
          f"{err.mean().item():.2e} (|ref| mean {ref_o.abs().mean().item():.2e}), worst row "
          f"relative {rel:.2e}", flush=True)
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3
    assert rel <= 2e-2           # each row at its own scale (bf16 P and output: ~2^-9)


@pytest.mark.parametrize("schedule", ["reference_defaults", "pool64_keep25"])
def test_config5_aggregator_200_frames(dev, aggregator, schedule):
    """`reference_defaults`: 25 pooled seeds per frame (broadcast_pool 8) and
    80 % keep in the core blocks 13-16 (aggregator.py:76-78).
    `pool64_keep25`: the workload as the 200-frame config states it, 64
    pooled patch summaries per frame (pool stride 5) and 25 % keep in every
    merged block (no core blocks)."""
    if schedule == "reference_defaults":
        cfg, agg = aggregator
    else:
        cfg = A.GpaConfig(broadcast_pool=5, core_blocks=())
        agg = A.build_aggregator(cfg, device=dev, seed=0)
    frames = 200
    N = frames * P
    imgs = A.shifted_texture_images(frames, device=dev).to(BF16)
    logs = ([], [])
    outs = []
    for i, log in enumerate(logs):
        print(f"[config 5, {schedule}] forward {i + 1} of 2 on {frames} frames", flush=True)
        agg.set_merge_log(log)
        with torch.no_grad(), torch.autocast("cuda", dtype=BF16):
            outs.append(agg(imgs))
        agg.set_merge_log(None)
        torch.cuda.synchronize()
    out1, out2 = outs
    assert len(out1) == len(cfg.dpt_blocks) == 4
    for a, b in zip(out1, out2):
        assert a.shape == (1, frames, P, 2 * cfg.embed_dim) and a.dtype == BF16
        assert torch.isfinite(a).all()
        assert torch.equal(a, b), "the aggregator is not bit-reproducible"

    log1, log2 = logs
    merged = [r for r in log1 if r["kind"] == "merged"]
    pools = [r for r in log1 if r["kind"] == "pool"]
    assert [r["block"] for r in merged] == list(range(9, 24))
    assert len(pools) == 9
    for r in merged:
        want = N - int(N * 0.2) if r["block"] in cfg.core_blocks else 66_845
        assert r["keys"] == want == r["size"].shape[1], r["block"]
        assert r["size"].sum().item() == N and r["size"].min().item() >= 1
        assert r["slot_offsets"][-1].item() == N
    assert {r["keys"] for r in merged} == ({66_845, 219_840} if cfg.core_blocks else {66_845})
    npool = (-(-GRID // cfg.broadcast_pool)) ** 2
    assert npool == (25 if cfg.broadcast_pool == 8 else 64)
    for r in pools:
        ps = r["pool_size"]
        assert ps.shape == (1, 16, frames, npool)
        assert torch.equal(ps.sum(-1), torch.full((1, 16, frames), float(GRID * GRID), device=dev))
    for r1, r2 in zip(log1, log2):
        key = "size" if r1["kind"] == "merged" else "pool_size"
        assert torch.equal(r1[key], r2[key])
    if schedule != "reference_defaults":
        del agg, outs, out1, out2, logs, log1, log2
        torch.cuda.empty_cache()


def test_config5_fp16_evaluation_stack(dev):
    """The same 200-frame aggregator as the reference's accuracy evaluation
    runs it (eval/eval_co3d.py:152, 226): the fp16 model under fp16
    autocast, reference defaults.  Every stage runs its fp16 kernel twin;
    finite fp16 outputs of the DPT shapes, bit-identical on a second forward,
    and the merge and pooling invariants of the bf16 run."""
    cfg = A.GpaConfig()
    f16 = torch.float16
    agg = A.build_aggregator(cfg, device=dev, dtype=f16, seed=0)
    frames = 200
    N = frames * P
    imgs = A.shifted_texture_images(frames, device=dev).to(f16)
    logs = ([], [])
    outs = []
    for i, log in enumerate(logs):
        print(f"[config 5, fp16] forward {i + 1} of 2 on {frames} frames", flush=True)
        agg.set_merge_log(log)
        with torch.no_grad(), torch.autocast("cuda", dtype=f16):
            outs.append(agg(imgs))
        agg.set_merge_log(None)
        torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert a.shape == (1, frames, P, 2 * cfg.embed_dim) and a.dtype == f16
        assert torch.isfinite(a).all()
        assert torch.equal(a, b), "the fp16 aggregator is not bit-reproducible"
    merged = [r for r in logs[0] if r["kind"] == "merged"]
    assert [r["block"] for r in merged] == list(range(9, 24))
    for r in merged:
        assert r["size"].sum().item() == N and r["size"].min().item() >= 1
    assert {r["keys"] for r in merged} == {66_845, 219_840}
    pools = [r for r in logs[0] if r["kind"] == "pool"]
    assert len(pools) == 9
    for r in pools:
        assert torch.equal(r["pool_size"].sum(-1),
                           torch.full((1, 16, frames), float(GRID * GRID), device=dev))
    del agg
    torch.cuda.empty_cache()
