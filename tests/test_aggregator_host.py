"""CPU checks of the GPA aggregator harness (no GPU, no kernel calls).

The schedule against aggregator.py:133-150 / :317-325, the RoPE angle table
against the frequencies of rope.py:92-123 (the rotation itself runs in the
fused qk kernel and is pinned on the GPU), the shared-set pooling against a brute-force loop over
attention.py:113-140, the token layout of aggregator.py:249-291, and the
FLOP accounting against the closed-form 200-frame totals.
"""
import math

import numpy as np
import pytest
import torch

import gpa_aggregator as A


def test_default_schedule():
    cfg = A.GpaConfig()
    kinds = [cfg.block_kind(i) for i in range(cfg.depth)]
    assert kinds[:9] == ["frame_special"] * 9
    assert kinds[9:] == ["merged"] * 15
    ratios = [cfg.block_merge_ratio(i) for i in range(9, 24)]
    assert ratios == [0.98] * 4 + [0.2] * 4 + [0.98] * 7


def test_schedule_variants():
    van = A.vanilla_config()
    assert all(van.block_kind(i) == "global" for i in range(24))
    # core blocks at ratio 0 are not merged (aggregator.py:322-323)
    cfg = A.GpaConfig(core_merge_ratio=0.0)
    assert [cfg.block_kind(i) for i in (12, 13, 16, 17)] == ["merged", "global", "global", "merged"]
    # merge window end
    cfg = A.GpaConfig(merge_end=20)
    assert cfg.block_kind(20) == "merged" and cfg.block_kind(21) == "global"
    cfg = A.GpaConfig(merge_end=-1, early_frame_split=3, merging=5)
    assert [cfg.block_kind(i) for i in (2, 3, 4, 5, 23)] == \
        ["frame_special", "global", "global", "merged", "merged"]


def test_rope_table_matches_textbook_angles():
    rope = A.Rope2D(100.0)
    cs = rope.cs_table(40, 64)
    assert cs.shape == (40, 16, 2) and cs.dtype == torch.float32
    for p in (0, 1, 7, 39):
        for j in range(16):
            th = p * 100.0 ** (-2.0 * j / 32)      # rope.py:109-114: base^(-2j/dim), dim 32
            assert abs(float(cs[p, j, 0]) - math.cos(th)) < 1e-7
            assert abs(float(cs[p, j, 1]) - math.sin(th)) < 1e-7
    t = rope.table(A.frame_positions(37, 5), 64)
    assert t.pos.dtype == torch.int32 and t.cs.shape == (38, 16, 2)


def test_frame_positions_layout():
    pos = A.frame_positions(37, 5)
    assert pos.shape == (1374, 2)
    assert (pos[:5] == 0).all()
    assert pos[5].tolist() == [1, 1] and pos[6].tolist() == [1, 2]
    assert pos[5 + 37].tolist() == [2, 1] and pos[-1].tolist() == [37, 37]


def _pool_bruteforce(k5, v5, pts, grid_h, grid_w, kp):
    B, H, S, P, D = k5.shape
    seeds_yx = [(y, x) for y in range(0, grid_h, kp) for x in range(0, grid_w, kp)]
    npool = len(seeds_yx)
    pk = np.zeros((B, H, S, npool, D))
    pv = np.zeros((B, H, S, npool, D))
    size = np.zeros((B, H, S, npool))
    assign = np.zeros((B, H, S, grid_h * grid_w), dtype=np.int64)
    k = k5.double().numpy()
    v = v5.double().numpy()
    for b in range(B):
        for h in range(H):
            for s in range(S):
                patches = k[b, h, s, pts:]
                seeds = np.stack([patches[y * grid_w + x] for y, x in seeds_yx])
                pn = patches / np.maximum(np.linalg.norm(patches, axis=1, keepdims=True), 1e-6)
                sn = seeds / np.maximum(np.linalg.norm(seeds, axis=1, keepdims=True), 1e-6)
                sc = pn @ sn.T
                top2 = np.sort(sc, axis=1)[:, -2:]
                assert (top2[:, 1] - top2[:, 0]).min() > 1e-4, "near tie in the test data"
                idx = sc.argmax(axis=1)
                assign[b, h, s] = idx
                for g in range(npool):
                    sel = idx == g
                    size[b, h, s, g] = sel.sum()
                    pk[b, h, s, g] = k[b, h, s, pts:][sel].mean(axis=0)
                    pv[b, h, s, g] = v[b, h, s, pts:][sel].mean(axis=0)
    return pk, pv, size, assign


@pytest.mark.parametrize("gh,gw,kp,npool", [(7, 7, 3, 9), (5, 8, 3, 6), (8, 5, 3, 6),
                                            (4, 10, 4, 3)])
def test_pool_shared_matches_bruteforce(gh, gw, kp, npool):
    """Square and rectangular patch grids (ph != pw): the seeds walk the rows
    of a row-major grid_h x grid_w layout."""
    g = torch.Generator().manual_seed(1)
    B, H, S, pts, D = 1, 2, 3, 5, 16
    k5 = torch.randn(B, H, S, pts + gh * gw, D, generator=g)
    v5 = torch.randn(B, H, S, pts + gh * gw, D, generator=g)
    pk, pv, size, assign = A.pool_shared_torch(k5, v5, pts, gh, gw, kp)
    bpk, bpv, bsize, bassign = _pool_bruteforce(k5, v5, pts, gh, gw, kp)
    assert np.array_equal(assign.numpy(), bassign)
    assert np.array_equal(size.numpy(), bsize)
    assert np.abs(pk.double().numpy().reshape(B, H, S, npool, D) - bpk).max() < 1e-5
    assert np.abs(pv.double().numpy().reshape(B, H, S, npool, D) - bpv).max() < 1e-5
    # every seed belongs to its own group: no empty summary
    assert (size > 0).all() and (size.sum(-1) == gh * gw).all()


def test_frame_positions_rectangular():
    pos = A.frame_positions(3, 5, grid_w=4)
    assert pos.shape == (17, 2)
    assert (pos[:5] == 0).all()
    want = [[y + 1, x + 1] for y in range(3) for x in range(4)]
    assert pos[5:].tolist() == want


def test_rectangular_config_and_embed():
    """A 42 x 56 image: 3 patch rows x 4 columns (ph x pw), row-major."""
    cfg = A.GpaConfig(vit_depth=0, depth=1, img_size=42, img_width=56)
    assert (cfg.grid_h, cfg.grid_w, cfg.tokens_per_frame) == (3, 4, 17)
    with pytest.raises(ValueError):
        cfg.grid
    model = A.GpaAggregator(cfg)
    A.init_random_(model)
    imgs = A.shifted_texture_images(3, size=(42, 56), shift=4)
    assert imgs.shape == (1, 3, 3, 42, 56)
    with torch.no_grad():
        tok = model.embed(imgs)
    assert tok.shape == (3, 17, 1024)
    assert model.positions("cpu").shape == (17, 2)


def test_shifted_texture_images_are_translations():
    imgs = A.shifted_texture_images(4, size=40, shift=6, seed=3)
    assert imgs.shape == (1, 4, 3, 40, 40)
    assert float(imgs.min()) >= 0.0 and float(imgs.max()) <= 1.0
    g = torch.Generator().manual_seed(3)
    tex = torch.rand(3, 46, 46, generator=g)
    off = torch.randint(0, 6, (4, 2), generator=g).tolist()
    for f, (y, x) in enumerate(off):
        assert torch.equal(imgs[0, f], tex[:, y:y + 40, x:x + 40])


def test_embed_token_layout_without_vit_blocks():
    cfg = A.GpaConfig(vit_depth=0, depth=1, img_size=56)
    model = A.GpaAggregator(cfg)
    A.init_random_(model)
    imgs = A.shifted_texture_images(3, size=56, shift=4)
    with torch.no_grad():
        tok = model.embed(imgs)
    assert tok.shape == (3, 4 * 4 + 5, 1024)
    assert torch.equal(tok[0, 0], model.camera_token[0, 0, 0])
    assert torch.equal(tok[1, 0], model.camera_token[0, 1, 0])
    assert torch.equal(tok[2, 1:5], model.register_token[0, 1])
    assert torch.equal(tok[0, 1:5], model.register_token[0, 0])


def test_patchify_equals_the_strided_convolution():
    cfg = A.GpaConfig(vit_depth=0, depth=1, img_size=56)
    emb = A.DinoV2Reg(cfg)
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        emb.patch.weight.copy_(torch.randn(emb.patch.weight.shape, generator=g) * 0.05)
        emb.patch.bias.copy_(torch.randn(emb.patch.bias.shape, generator=g))
        img = torch.rand(2, 3, 56, 56, generator=g)
        want = emb.patch(img).flatten(2).transpose(1, 2)
        got = emb.patchify(img)
    assert got.shape == want.shape == (2, 16, 1024)
    assert torch.allclose(got, want, atol=1e-4, rtol=1e-4)


def test_aggregator_flops_closed_form():
    cfg = A.GpaConfig()
    f = A.aggregator_flops(cfg, 200)
    T, H, D = 274_800, 16, 64
    own = 4.0 * 200 * H * 1374 * 1369 * D
    shared = 4.0 * H * T * 200 * 30 * D
    merged = 11 * 4.0 * H * T * 66_845 * D + 4 * 4.0 * H * T * 219_840 * D
    assert f["global_attn"] == pytest.approx(9 * (own + shared) + merged, rel=1e-12)
    assert f["similarity"] == pytest.approx(15 * 2.0 * 207_955 * 66_845 * 128, rel=1e-12)
    assert f["frame_attn"] == pytest.approx(48 * 4.0 * 200 * H * 1374 * 1374 * D, rel=1e-12)


def test_aggregator_flops_unprojected_metric():
    """merge_metric_dim=0 (eval/eval_co3d.py:121-122): no projection GEMM,
    the similarity over all 1024 features."""
    base = A.aggregator_flops(A.GpaConfig(), 200)
    f = A.aggregator_flops(A.GpaConfig(merge_metric_dim=0), 200)
    assert f["similarity"] == pytest.approx(15 * 2.0 * 207_955 * 66_845 * 1024, rel=1e-12)
    assert base["dense"] - f["dense"] == pytest.approx(15 * 2.0 * 274_800 * 1024 * 128, rel=1e-12)
    assert f["global_attn"] == base["global_attn"]


def test_aggregator_flops_rectangular_and_frame_only():
    """392 x 518 images (28 x 37 patches): 20 pooled summaries per frame at
    kp 8; kp < 0 is plain attention over each frame's own tokens."""
    cfg = A.GpaConfig(img_size=392, img_width=518)
    P = 28 * 37 + 5
    T, H, D = 200 * P, 16, 64
    f = A.aggregator_flops(cfg, 200)
    own = 4.0 * 200 * H * P * (P - 5) * D
    shared = 4.0 * H * T * 200 * (5 + 20) * D
    f_nomerge = A.aggregator_flops(A.GpaConfig(img_size=392, img_width=518, merging=None), 200)
    plain = 4.0 * H * T * T * D
    assert f_nomerge["global_attn"] == pytest.approx(9 * (own + shared) + 15 * plain, rel=1e-12)
    assert f["frame_attn"] == pytest.approx(48 * 4.0 * 200 * H * P * P * D, rel=1e-12)
    f_neg = A.aggregator_flops(A.GpaConfig(img_size=392, img_width=518, merging=None,
                                           broadcast_pool=-1), 200)
    assert f_neg["global_attn"] == pytest.approx(9 * 4.0 * 200 * H * P * P * D + 15 * plain,
                                                 rel=1e-12)
