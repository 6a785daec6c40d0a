"""GPU checks of the GPA aggregator harness: the merged and frame-special
global attention of a VGGT-1B-width block against an fp32 CPU restatement.

The CPU side recomputes the attention module from the block's own weights:
qkv projection (bf16 operands, fp32 accumulation, bf16 result, as autocast
does), qk LayerNorm, textbook RoPE, then
  * merged block (vggt/layers/attention.py:233-268): K/V means over the
    device merge's slot lists in fp64, bias log(size), the oracle attention;
  * frame-special block (attention.py:148-176): per frame, one attention
    over [own patch keys | every frame's special keys | pooled summaries]
    with bias log(size) on the summaries -- the unsplit form the split path
    must equal -- with the summaries averaged in fp64 over the device's
    pool assignment;
then the output projection.  Given identical merge / pool assignments the
two must agree to bf16 rounding of the module's intermediates.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import gpa_aggregator as A
import gpa_workloads as W
from merging.merge import token_merge_bipartite2d
from oracle.attention import attention_reference, kernel_inputs

pytestmark = pytest.mark.gpu

FRAMES = 3
GRID = 37
PTS = 5
P = GRID * GRID + PTS


def _rope_ref(x: torch.Tensor, pos: torch.Tensor, freq: float = 100.0) -> torch.Tensor:
    """Rotate-half RoPE per axis (rope.py:139-209) in fp64 on the CPU."""
    x = x.double()
    out = x.clone()
    j = torch.arange(16, dtype=torch.float64)
    for a in range(2):
        th = pos[:, a].double()[:, None] * freq ** (-2.0 * j / 32)
        c, s = th.cos(), th.sin()
        x1, x2 = x[..., a * 32:a * 32 + 16], x[..., a * 32 + 16:a * 32 + 32]
        out[..., a * 32:a * 32 + 16] = x1 * c - x2 * s
        out[..., a * 32 + 16:a * 32 + 32] = x2 * c + x1 * s
    return out.float()


def _block(dev, seed=0, gh=GRID, gw=GRID):
    cfg = A.GpaConfig(img_size=14 * gh, img_width=14 * gw)
    blk = A.Block(1024, 16, 4.0, 1.0, True, 1e-5, cfg).to(dev)
    A.init_random_(blk, seed)
    with torch.no_grad():   # non-trivial qk-norm affine parameters
        g = torch.Generator(device=dev).manual_seed(seed + 5)
        for ln in (blk.attn.q_norm, blk.attn.k_norm):
            ln.weight.copy_(1 + 0.2 * torch.randn(64, generator=g, device=dev))
            ln.bias.copy_(0.1 * torch.randn(64, generator=g, device=dev))
    return cfg, blk.bfloat16().eval()


def _inputs(dev, gh=GRID, gw=GRID):
    """Tokens of FRAMES frames on a gh x gw patch grid (the first
    gh*gw + PTS tokens of each 1,374-token frame of the shifted basis)."""
    x = W.shifted_basis_tokens(FRAMES, seed=4, device=dev).to(torch.bfloat16)
    p_ = gh * gw + PTS
    x = x.view(1, FRAMES, P, -1)[:, :, :p_].reshape(1, FRAMES * p_, -1)
    pos1 = A.frame_positions(gh, PTS, dev, grid_w=gw)
    return x, pos1.repeat(FRAMES, 1), A.Rope2D(100.0).table(pos1, 64)


def _qkv_ref(blk, xn: torch.Tensor, pos: torch.Tensor):
    """CPU restatement of qkv -> qk-norm -> RoPE (attention.py:210-220)."""
    at = blk.attn
    w, b = at.qkv.weight.float().cpu(), at.qkv.bias.float().cpu()
    x16 = xn.cpu().bfloat16().float()
    qkv = (x16 @ w.T + b).bfloat16().float()
    N = qkv.shape[1]
    q, k, v = qkv.view(1, N, 3, 16, 64).permute(2, 0, 3, 1, 4).unbind(0)

    def ln(t, mod):
        return F.layer_norm(t, (64,), mod.weight.float().cpu(), mod.bias.float().cpu(), 1e-5)

    q, k = ln(q, at.q_norm), ln(k, at.k_norm)
    pc = pos.cpu()
    return _rope_ref(q, pc), _rope_ref(k, pc), v


def _proj_ref(blk, o: torch.Tensor) -> torch.Tensor:
    w, b = blk.attn.proj.weight.float().cpu(), blk.attn.proj.bias.float().cpu()
    N = o.shape[2]
    y = o.transpose(1, 2).reshape(1, N, 1024).bfloat16().float()
    return y @ w.T + b


def _slot_means(t: torch.Tensor, offsets: torch.Tensor, tokens: torch.Tensor) -> torch.Tensor:
    """fp64 mean of t [1,H,N,D] rows over CSR slot lists -> [1,H,S,D]."""
    t64 = t.double()
    off = offsets.cpu().numpy()
    tok = tokens.cpu().numpy()
    seg = np.repeat(np.arange(len(off) - 1), np.diff(off))
    out = torch.zeros(1, t.shape[1], len(off) - 1, t.shape[3], dtype=torch.float64)
    out.index_add_(2, torch.from_numpy(seg), t64[:, :, torch.from_numpy(tok)])
    cnt = torch.from_numpy(np.diff(off)).double()
    return out / cnt.view(1, 1, -1, 1)


def _compare(got: torch.Tensor, ref: torch.Tensor, what: str):
    err = (got.float().cpu() - ref).abs()
    scale = ref.abs().mean().item()
    rel_max, rel_mean = err.max().item() / scale, err.mean().item() / scale
    print(f"[{what}] |ref| mean {scale:.3e}, max err {err.max().item():.3e} "
          f"({rel_max:.2e} rel), mean err {err.mean().item():.3e} ({rel_mean:.2e} rel)", flush=True)
    # bf16 intermediates (qkv, attention output, merged V) give ~1e-2 relative
    # scatter per element; a layout, scale or bias mistake gives O(1).
    assert rel_max < 0.06, f"{what}: max error {rel_max:.3e} of mean |ref|"
    assert rel_mean < 0.006, f"{what}: mean error {rel_mean:.3e} of mean |ref|"


@pytest.mark.parametrize("gh,gw", [(37, 37), (28, 37)])
def test_merged_block_attention_matches_reference(dev, gh, gw):
    """Square (518 x 518) and rectangular (392 x 518 images: 28 patch rows
    x 37 columns, the reference module's default) patch grids."""
    cfg, blk = _block(dev, gh=gh, gw=gw)
    x, pos, rope = _inputs(dev, gh, gw)
    N = x.shape[1]
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        xn = blk.norm1(x)
        got = blk.attn(xn, rope, 9)
        gen = torch.Generator(device=dev)
        gen.manual_seed(A.MERGE_GENERATOR_SEED)
        m = token_merge_bipartite2d(xn, gw, gh, 2, 2, int(N * 0.98), False, gen,
                                    metric_dim=128, num_special=PTS)
    assert xn.dtype == torch.float32
    q, k, v = _qkv_ref(blk, xn, pos)
    off, tok = m.index.slot_offsets, m.index.slot_tokens
    km = _slot_means(k, off, tok).float()
    vm = _slot_means(v, off, tok)
    size = m.size.cpu()
    assert km.shape[2] == size.shape[1] == m.index.num_dst   # all sources merged at 0.98
    bias = size.log().view(1, 1, 1, -1)
    o, _ = attention_reference(*kernel_inputs(q, km, vm.float(), bias.expand(1, 16, 1, -1)),
                               blk.attn.scale)
    _compare(got, _proj_ref(blk, o), f"merged block ({gh} x {gw})")


@pytest.mark.parametrize("kp,gh,gw", [(8, 37, 37), (5, 37, 37), (4, 37, 37), (0, 37, 37),
                                      (-1, 37, 37), (8, 28, 37), (4, 28, 37), (5, 37, 28)])
def test_frame_special_block_attention_matches_reference(dev, kp, gh, gw):
    """The frame-special block for the pool strides the reference accepts
    (attention.py:106-108, 178-190): kp > 0 pooled summaries (the pooling
    kernel: 25, 64 and, in super-chunks of 64, 100 seeds at kp 8, 5 and 4 on
    37 x 37), kp = 0 the special tokens only, kp < 0 plain frame attention;
    on square and rectangular patch grids (ph x pw = gh x gw)."""
    cfg, blk = _block(dev, seed=1, gh=gh, gw=gw)
    cfg.broadcast_pool = kp
    blk.attn.frame_special = True
    x, pos, rope = _inputs(dev, gh, gw)
    P = gh * gw + PTS
    N = x.shape[1]
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        xn = blk.norm1(x)
        got = blk.attn(xn, rope, None)
        # the device's pool assignment, from the module's own K/V
        _, kd, vd = blk.attn.qk(xn, rope)
        if kp > 0:
            _, _, size_d, assign_d = A.pool_shared_set(kd, vd, FRAMES, PTS, gh, gw, kp, True)
    q, k, v = _qkv_ref(blk, xn, pos)
    q16, k16, v16 = q.bfloat16().float(), k.bfloat16().float(), v
    k5, v5 = k16.view(1, 16, FRAMES, P, 64), v16.view(1, 16, FRAMES, P, 64)
    out = torch.empty(1, 16, N, 64)
    if kp < 0:
        for s in range(FRAMES):
            o, _ = attention_reference(*kernel_inputs(q16[:, :, s * P:(s + 1) * P], k5[:, :, s],
                                                      v5[:, :, s], None), blk.attn.scale)
            out[:, :, s * P:(s + 1) * P] = o
        _compare(got, _proj_ref(blk, out), f"frame attention (kp {kp}, {gh} x {gw})")
        return
    sp_k = k5[:, :, :, :PTS].reshape(1, 16, FRAMES * PTS, 64)
    sp_v = v5[:, :, :, :PTS].reshape(1, 16, FRAMES * PTS, 64)
    extra_k, extra_v, extra_b = [sp_k], [sp_v], [torch.zeros(1, 16, 1, FRAMES * PTS)]
    if kp > 0:
        assign = assign_d.cpu().long()
        npool = (-(-gh // kp)) * (-(-gw // kp))
        onehot = F.one_hot(assign, npool).double()                     # [1,16,S,gh*gw,np]
        cnt = onehot.sum(3)                                            # [1,16,S,np]
        assert torch.equal(cnt.float(), size_d.cpu())
        pk = torch.einsum("bhspg,bhspd->bhsgd", onehot, k5[:, :, :, PTS:].double()) / cnt[..., None]
        pv = torch.einsum("bhspg,bhspd->bhsgd", onehot, v5[:, :, :, PTS:].double()) / cnt[..., None]
        extra_k.append(pk.reshape(1, 16, -1, 64).float())
        extra_v.append(pv.reshape(1, 16, -1, 64).float())
        extra_b.append(cnt.reshape(1, 16, 1, -1).log().float())
    for s in range(FRAMES):
        kk = torch.cat([k5[:, :, s, PTS:]] + extra_k, dim=2)
        vv = torch.cat([v5[:, :, s, PTS:]] + extra_v, dim=2)
        bias = torch.cat([torch.zeros(1, 16, 1, gh * gw)] + extra_b, dim=3)
        o, _ = attention_reference(*kernel_inputs(q16[:, :, s * P:(s + 1) * P], kk, vv, bias),
                                   blk.attn.scale)
        out[:, :, s * P:(s + 1) * P] = o
    _compare(got, _proj_ref(blk, out), f"frame-special block (kp {kp}, {gh} x {gw})")


@pytest.mark.parametrize("hw,dt", [((518, 518), torch.bfloat16), ((392, 518), torch.bfloat16),
                                   ((518, 518), torch.float16)])
def test_small_aggregator_runs_every_global_path(dev, hw, dt):
    """Every global path (frame-special pooling, merged, core merged) on
    square and rectangular images, as the bf16 benchmark stack and as the
    fp16 accuracy-evaluation stack (fp16 model under fp16 autocast,
    eval/eval_co3d.py:226 and :152): finite outputs of the DPT shapes in the
    model's dtype, bit-identical on a second forward."""
    cfg = A.GpaConfig(depth=3, vit_depth=1, early_frame_split=1, merging=1,
                      core_blocks=(2,), core_merge_ratio=0.5, dpt_blocks=(0, 1, 2),
                      img_size=hw[0], img_width=hw[1])
    assert [cfg.block_kind(i) for i in range(3)] == ["frame_special", "merged", "merged"]
    P = cfg.tokens_per_frame
    model = A.build_aggregator(cfg, device=dev, dtype=dt, seed=2)
    imgs = A.shifted_texture_images(FRAMES, size=hw, device=dev).to(dt)
    tracer = A.StageTimer()
    model.set_tracer(tracer)
    tracer.start()
    with torch.no_grad(), torch.autocast("cuda", dtype=dt):
        outs = model(imgs)
        again = model(imgs)
    assert all(torch.equal(a, b) for a, b in zip(outs, again))
    stages = tracer.totals()
    assert {"frame_special_attn", "pool", "merge", "merged_attn", "frame_attn"} <= set(stages)
    assert len(outs) == 3
    for o in outs:
        assert o.shape == (1, FRAMES, P, 2048) and o.dtype == dt
        assert torch.isfinite(o).all()
    flops = A.aggregator_flops(cfg, FRAMES)
    assert flops["similarity"] > 0 and flops["global_attn"] > 0


def test_small_aggregator_two_scenes(dev):
    """A batch of two scenes ([2, S, 3, H, W] images, as the reference's
    aggregator takes them): the merged blocks take their key sizes from
    summed ones (vggt/layers/attention.py:250-253) since `merge.size` is
    None; the same scene twice gives bit-identical outputs for both batch
    elements, close to the one-scene forward (the dense GEMMs may run other
    kernels for twice the rows)."""
    cfg = A.GpaConfig(depth=3, vit_depth=1, early_frame_split=1, merging=1,
                      core_blocks=(2,), core_merge_ratio=0.5, dpt_blocks=(0, 1, 2))
    P = cfg.tokens_per_frame
    model = A.build_aggregator(cfg, device=dev, seed=2)
    img = A.shifted_texture_images(FRAMES, device=dev).to(torch.bfloat16)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        two = model(torch.cat([img, img]))
        one = model(img)
    for o2, o1 in zip(two, one):
        assert o2.shape == (2, FRAMES, P, 2048) and torch.isfinite(o2).all()
        assert torch.equal(o2[0], o2[1])
        d = (o2[0].float() - o1[0].float()).abs()
        assert d.mean().item() <= 1e-2 * o1.float().abs().mean().item()


def test_small_aggregator_unprojected_metric(dev):
    """merge_metric_dim=0 (eval/eval_co3d.py:121-122): the merged blocks
    match tokens on the full 1024-d cosine (the 256 x 256-tile similarity
    kernel above 256 destinations, no projection or fused front end);
    finite outputs, bit-identical on a second forward, every merge keeping
    all tokens (sizes sum to the token count) and merging r of them."""
    cfg = A.GpaConfig(depth=3, vit_depth=1, early_frame_split=1, merging=1,
                      core_blocks=(2,), core_merge_ratio=0.5, dpt_blocks=(0, 1, 2),
                      merge_metric_dim=0)
    P = cfg.tokens_per_frame
    model = A.build_aggregator(cfg, device=dev, seed=3)
    imgs = A.shifted_texture_images(FRAMES, device=dev).to(torch.bfloat16)
    log = []
    model.set_merge_log(log)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        outs = model(imgs)
    model.set_merge_log(None)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        again = model(imgs)
    assert all(torch.equal(a, b) for a, b in zip(outs, again))
    for o in outs:
        assert o.shape == (1, FRAMES, P, 2048) and torch.isfinite(o).all()
    merged = [r for r in log if r["kind"] == "merged"]
    assert len(merged) == 2
    for rec in merged:
        T = rec["tokens"]
        assert int(rec["size"].sum().item()) == T
        assert rec["keys"] == T - int(rec["r"])


@pytest.mark.parametrize("frames,k_f32,half", [(3, True, torch.bfloat16), (2, False, torch.bfloat16),
                                               (3, True, torch.float16), (2, False, torch.float16)])
def test_qk_norm_rope_kernel_matches_textbook(dev, frames, k_f32, half):
    """gpa::qk_norm_rope against LayerNorm + rotate-half RoPE in fp64, on a
    bf16 and an fp16 projection (16-bit outputs in the projection's format)."""
    g = torch.Generator(device=dev).manual_seed(frames)
    N = frames * P
    qkv = (torch.randn(1, N, 3 * 1024, generator=g, device=dev) * 1.5 + 0.3).to(half)
    ln_w = 1 + 0.3 * torch.randn(2, 64, generator=g, device=dev)
    ln_b = 0.2 * torch.randn(2, 64, generator=g, device=dev)
    pos1 = A.frame_positions(GRID, PTS, dev)
    rope = A.Rope2D(100.0).table(pos1, 64)
    q, k = torch.ops.gpa.qk_norm_rope(qkv, ln_w, ln_b, 1e-5, rope.pos, rope.cs, 16, False, k_f32)
    assert q.dtype == half and q.shape == (1, 16, N, 64)
    assert k.dtype == (torch.float32 if k_f32 else half)
    x = qkv.cpu().double().view(1, N, 3, 16, 64).permute(2, 0, 3, 1, 4)
    pos = pos1.cpu().repeat(frames, 1)
    for got, t, i in ((q, x[0], 0), (k, x[1], 1)):
        mu = t.mean(-1, keepdim=True)
        var = ((t - mu) ** 2).mean(-1, keepdim=True)
        y = (t - mu) / torch.sqrt(var + 1e-5) * ln_w[i].cpu().double() + ln_b[i].cpu().double()
        want = _rope_ref(y, pos).double()
        err = (got.cpu().double() - want).abs()
        rel = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}.get(got.dtype, 1e-5)
        bound = rel * want.abs() + 1e-5
        assert (err <= bound).all(), f"max err {err.max().item():.3e}"
    # no rotation: plain LayerNorm
    q0, _ = torch.ops.gpa.qk_norm_rope(qkv, ln_w, ln_b, 1e-5, None, None, 16, True, True)
    t = x[0]
    y = (t - t.mean(-1, keepdim=True)) / torch.sqrt(t.var(-1, unbiased=False, keepdim=True) + 1e-5)
    y = y * ln_w[0].cpu().double() + ln_b[0].cpu().double()
    assert (q0.cpu().double() - y).abs().max().item() < 1e-4


@pytest.mark.parametrize("B,H,pad", [(2, 5, 64), (1, 24, 0), (3, 1, 8)])
def test_qk_norm_rope_other_head_counts_and_strides(dev, B, H, pad):
    """Any head count (the kernel walks (token, q|k head) items in projection
    order, so a workgroup's items cross token rows whenever 2H is not 32),
    B > 1, and projection rows wider than 3*H*64 (a view of a padded
    tensor); against the fp64 textbook, fp32 outputs."""
    g = torch.Generator(device=dev).manual_seed(B * 100 + H)
    N = P + 37                      # not a multiple of the frame period
    C = 3 * H * 64
    wide = (torch.randn(B, N, C + pad, generator=g, device=dev) * 1.5 + 0.3).bfloat16()
    qkv = wide[:, :, :C]
    ln_w = 1 + 0.3 * torch.randn(2, 64, generator=g, device=dev)
    ln_b = 0.2 * torch.randn(2, 64, generator=g, device=dev)
    pos1 = A.frame_positions(GRID, PTS, dev)
    rope = A.Rope2D(100.0).table(pos1, 64)
    q, k = torch.ops.gpa.qk_norm_rope(qkv, ln_w, ln_b, 1e-5, rope.pos, rope.cs, H, True, True)
    assert q.shape == (B, H, N, 64) and k.shape == (B, H, N, 64)
    x = qkv.cpu().double().view(B, N, 3, H, 64).permute(2, 0, 3, 1, 4)
    pos = pos1.cpu().repeat(2, 1)[:N]
    for got, t, i in ((q, x[0], 0), (k, x[1], 1)):
        mu = t.mean(-1, keepdim=True)
        var = ((t - mu) ** 2).mean(-1, keepdim=True)
        y = (t - mu) / torch.sqrt(var + 1e-5) * ln_w[i].cpu().double() + ln_b[i].cpu().double()
        want = _rope_ref(y, pos).double()
        err = (got.cpu().double() - want).abs()
        assert (err <= 1e-5 * want.abs() + 1e-5).all(), f"max err {err.max().item():.3e}"


def _pool_bf16_fp64(x: torch.Tensor, gh: int, gw: int, kp: int):
    """fp64 scores of bf16-rounded normalised rows against bf16-rounded
    normalised seeds (the einsum of attention.py:130 under bf16 autocast,
    before its own bf16 rounding): x [G, gh*gw, 64] -> [G, gh*gw, npool]."""
    def nb(t):
        t = t.float()
        return (t / t.norm(dim=-1, keepdim=True).clamp_min(1e-6)).bfloat16().double()
    G = x.shape[0]
    seeds = x.view(G, gh, gw, 64)[:, ::kp, ::kp].reshape(G, -1, 64)
    return torch.einsum("gpd,gsd->gps", nb(x), nb(seeds))


@pytest.mark.parametrize("gh,gw,kp", [
    (37, 37, 8), (37, 37, 5),     # the 518 x 518 grid: 25 and 64 seeds
    (28, 37, 8), (37, 28, 5),     # 392 x 518 and 518 x 392 images: 20 and 48 seeds
    (13, 50, 7),                  # ragged last tile and lattice row
    (64, 64, 8),                  # 4096 patches (the kernel's limit), 64 seeds
    (1, 1, 8),                    # one patch, one seed
    (37, 37, 4), (28, 37, 3),     # more than 64 seeds: 100 and 130 (super-chunks of 64)
    (37, 37, 2), (37, 37, 1),     # 361 seeds; every patch a seed (1,369)
    (64, 64, 2),                  # 4096 patches, 1,024 seeds
])
def test_pool_shared_kernel_matches_reference(dev, gh, gw, kp):
    """gpa::pool_shared against the scores in fp64 (assignment, except rows
    whose best two scores are within two bf16 steps, where the bf16 rounding
    of the reference's scores decides) and, given its own assignment, exact
    sizes and fp64 means of the K and V rows; bit-identical on a second call
    and on strided V rows.  Square and rectangular patch grids, every pool
    stride the reference accepts down to 1 (attention.py:106-140)."""
    g = torch.Generator(device=dev).manual_seed(gh * 100 + gw + kp)
    B, H, S = 1, 4, 3
    P_ = PTS + gh * gw
    npatch = gh * gw
    k = (torch.randn(B, H, S * P_, 64, generator=g, device=dev) * 0.7).bfloat16()
    v = torch.randn(B, H, S * P_, 64, generator=g, device=dev).bfloat16()
    pk, pv, size, assign = torch.ops.gpa.pool_shared(k, v, S, PTS, gh, gw, kp, True)
    npool = -(-gh // kp) * -(-gw // kp)
    assert pk.shape == (B, H, S * npool, 64) and size.shape == (B, H, S, npool)
    assert assign.shape == (B, H, S, npatch)
    kp5 = k.view(B, H, S, P_, 64)[:, :, :, PTS:].reshape(-1, npatch, 64).cpu()
    vp5 = v.view(B, H, S, P_, 64)[:, :, :, PTS:].reshape(-1, npatch, 64).cpu()
    sc = _pool_bf16_fp64(kp5, gh, gw, kp)
    a = assign.cpu().long().reshape(-1, npatch)
    if npool > 1:
        top2 = sc.topk(2, dim=-1).values
        sure = (top2[..., 0] - top2[..., 1]) > 2 * 2.0 ** -8
        assert sure.float().mean() > 0.5
    else:
        sure = torch.ones_like(a, dtype=torch.bool)
    assert torch.equal(a[sure], sc.argmax(-1)[sure])
    # seeds belong to their own group
    seeds_pos = [(y * gw + x) for y in range(0, gh, kp) for x in range(0, gw, kp)]
    assert torch.equal(a[:, seeds_pos], torch.arange(npool).expand(a.shape[0], npool))
    onehot = torch.nn.functional.one_hot(a, npool).double()          # [G, p, npool]
    cnt = onehot.sum(1)
    assert torch.equal(size.cpu().reshape(-1, npool).double(), cnt)
    mk = torch.einsum("gps,gpd->gsd", onehot, kp5.double()) / cnt.clamp_min(1)[..., None]
    mv = torch.einsum("gps,gpd->gsd", onehot, vp5.double()) / cnt.clamp_min(1)[..., None]
    for got, want in ((pk, mk), (pv, mv)):
        got = got.cpu().double().reshape(-1, npool, 64)
        err = (got - want).abs()
        assert (err <= 2.0 ** -8 * want.abs() + 1e-6).all(), f"max err {err.max().item():.3e}"
    # the torch restatement on the same device agrees on the sure rows
    _, _, _, a_t = A.pool_shared_torch(k.view(B, H, S, P_, 64), v.view(B, H, S, P_, 64),
                                       PTS, gh, gw, kp)
    assert torch.equal(a_t.cpu().reshape(-1, npatch)[sure], a[sure])
    # deterministic sums (fixed order), and strided rows give the same result
    pk2, pv2, size2, _ = torch.ops.gpa.pool_shared(k, v, S, PTS, gh, gw, kp, False)
    assert torch.equal(pk2, pk) and torch.equal(pv2, pv) and torch.equal(size2, size)
    wide = torch.zeros(B, H, S * P_, 128, device=dev, dtype=torch.bfloat16)
    wide[..., 32:96] = v
    pk3, pv3, _, _ = torch.ops.gpa.pool_shared(k, wide[..., 32:96], S, PTS, gh, gw, kp, False)
    assert torch.equal(pk3, pk) and torch.equal(pv3, pv)


@pytest.mark.parametrize("gh,gw,kp", [(37, 37, 8), (37, 37, 4), (37, 37, 1)])
def test_pool_shared_kernel_empty_seeds(dev, gh, gw, kp):
    """Seeds whose key equals an earlier seed's tie with it on every patch,
    and the lowest seed wins (`argmax`'s first maximum), so they end with no
    members: size 0 and a zero summary (the count clamp).  Seeds 1-3 of
    every frame are copies of seed 0's key; the other groups keep their fp64
    means over the kernel's own assignment, and a second call is
    bit-identical (both the 64-seed kernel and the sorted member lists of
    the many-seed kernel)."""
    g = torch.Generator(device=dev).manual_seed(gh + gw + 10 * kp)
    B, H, S = 1, 2, 3
    P_ = PTS + gh * gw
    npatch = gh * gw
    k = (torch.randn(B, H, S * P_, 64, generator=g, device=dev) * 0.7).bfloat16()
    v = torch.randn(B, H, S * P_, 64, generator=g, device=dev).bfloat16()
    seeds_pos = [(y * gw + x) for y in range(0, gh, kp) for x in range(0, gw, kp)]
    kv = k.view(B, H, S, P_, 64)
    for j in (1, 2, 3):
        kv[:, :, :, PTS + seeds_pos[j]] = kv[:, :, :, PTS + seeds_pos[0]]
    pk, pv, size, assign = torch.ops.gpa.pool_shared(k, v, S, PTS, gh, gw, kp, True)
    npool = len(seeds_pos)
    a = assign.cpu().long().reshape(-1, npatch)
    cnt = torch.nn.functional.one_hot(a, npool).double().sum(1)
    assert torch.equal(size.cpu().reshape(-1, npool).double(), cnt)
    assert (cnt[:, 1:4] == 0).all() and (cnt[:, 0] >= 4).all()
    kp5 = k.view(B, H, S, P_, 64)[:, :, :, PTS:].reshape(-1, npatch, 64).cpu()
    vp5 = v.view(B, H, S, P_, 64)[:, :, :, PTS:].reshape(-1, npatch, 64).cpu()
    onehot = torch.nn.functional.one_hot(a, npool).double()
    for got, rows in ((pk, kp5), (pv, vp5)):
        want = torch.einsum("gps,gpd->gsd", onehot, rows.double()) / cnt.clamp_min(1)[..., None]
        got = got.cpu().double().reshape(-1, npool, 64)
        assert (got[:, 1:4] == 0).all()
        err = (got - want).abs()
        assert (err <= 2.0 ** -8 * want.abs() + 1e-6).all(), f"max err {err.max().item():.3e}"
    pk2, pv2, size2, _ = torch.ops.gpa.pool_shared(k, v, S, PTS, gh, gw, kp, False)
    assert torch.equal(pk2, pk) and torch.equal(pv2, pv) and torch.equal(size2, size)


@pytest.mark.parametrize("gh,gw,kp", [(37, 37, 8), (28, 37, 5), (37, 37, 3)])
def test_pool_shared_kernel_fp16(dev, gh, gw, kp):
    """The fp16 instantiation (the pooling under fp16 autocast): assignment
    equal to the fp64 argmax over fp16-rounded normalised rows wherever the
    top two scores are more than two fp16 steps apart, exact sizes, fp16
    means within 2^-11 relative of fp64 means over the kernel's own
    assignment, and the torch restatement under fp16 autocast agreeing on
    the sure rows."""
    g = torch.Generator(device=dev).manual_seed(gh + gw + kp)
    B, H, S = 1, 4, 3
    P_ = PTS + gh * gw
    npatch = gh * gw
    k = (torch.randn(B, H, S * P_, 64, generator=g, device=dev) * 0.7).half()
    v = torch.randn(B, H, S * P_, 64, generator=g, device=dev).half()
    pk, pv, size, assign = torch.ops.gpa.pool_shared(k, v, S, PTS, gh, gw, kp, True)
    assert pk.dtype == pv.dtype == torch.float16
    npool = -(-gh // kp) * -(-gw // kp)
    kp5 = k.view(B, H, S, P_, 64)[:, :, :, PTS:].reshape(-1, npatch, 64).cpu()
    vp5 = v.view(B, H, S, P_, 64)[:, :, :, PTS:].reshape(-1, npatch, 64).cpu()

    def nh(t):
        t = t.float()
        return (t / t.norm(dim=-1, keepdim=True).clamp_min(1e-6)).half().double()
    G = kp5.shape[0]
    seeds = kp5.view(G, gh, gw, 64)[:, ::kp, ::kp].reshape(G, -1, 64)
    sc = torch.einsum("gpd,gsd->gps", nh(kp5), nh(seeds))
    top2 = sc.topk(2, dim=-1).values
    sure = (top2[..., 0] - top2[..., 1]) > 2 * 2.0 ** -11
    a = assign.cpu().long().reshape(-1, npatch)
    assert sure.float().mean() > 0.5
    assert torch.equal(a[sure], sc.argmax(-1)[sure])
    onehot = torch.nn.functional.one_hot(a, npool).double()
    cnt = onehot.sum(1)
    assert torch.equal(size.cpu().reshape(-1, npool).double(), cnt)
    for got, rows in ((pk, kp5), (pv, vp5)):
        want = torch.einsum("gps,gpd->gsd", onehot, rows.double()) / cnt.clamp_min(1)[..., None]
        err = (got.cpu().double().reshape(-1, npool, 64) - want).abs()
        assert (err <= 2.0 ** -11 * want.abs() + 1e-6).all(), f"max err {err.max().item():.3e}"
    with torch.autocast("cuda", dtype=torch.float16):
        _, _, _, a_t = A.pool_shared_torch(k.view(B, H, S, P_, 64), v.view(B, H, S, P_, 64),
                                           PTS, gh, gw, kp)
    assert torch.equal(a_t.cpu().reshape(-1, npatch)[sure], a[sure])


def test_pool_shared_batches_and_strided_k(dev):
    """B = 2 with batch strides of a head-major view (k and v sliced out of a
    [B, 2H, N, 64] buffer, heads 1, 3, 5, 7): each (batch, head, frame) equals
    the same group pooled on its own as a contiguous B = 1 tensor."""
    g = torch.Generator(device=dev).manual_seed(77)
    B, H, S, gh, gw, kp = 2, 4, 3, 28, 37, 8
    P_ = PTS + gh * gw
    big_k = (torch.randn(B, 2 * H, S * P_, 64, generator=g, device=dev) * 0.7).bfloat16()
    big_v = torch.randn(B, 2 * H, S * P_, 64, generator=g, device=dev).bfloat16()
    k, v = big_k[:, 1::2], big_v[:, 1::2]
    assert not k.is_contiguous()
    pk, pv, size, assign = torch.ops.gpa.pool_shared(k, v, S, PTS, gh, gw, kp, True)
    for b in range(B):
        for h in range(H):
            kk = k[b:b + 1, h:h + 1].contiguous()
            vv = v[b:b + 1, h:h + 1].contiguous()
            pk1, pv1, size1, a1 = torch.ops.gpa.pool_shared(kk, vv, S, PTS, gh, gw, kp, True)
            assert torch.equal(pk[b:b + 1, h:h + 1], pk1)
            assert torch.equal(pv[b:b + 1, h:h + 1], pv1)
            assert torch.equal(size[b:b + 1, h:h + 1], size1)
            assert torch.equal(assign[b:b + 1, h:h + 1], a1)
