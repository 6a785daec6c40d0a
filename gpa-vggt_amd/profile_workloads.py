#!/usr/bin/env python3
"""Run each hot kernel a few times at its benchmark shape, for profilers.

    python3 gpa-vggt_amd/profile_workloads.py {sim|sim200|sim1024|attn|core|probe|sharp|own|shared|merge|front|pool|qk|combine|sim16|attn16|attn0|copy|all} [reps]

  sim    fused similarity-argmax, 75,000 x 25,000 x 128 (bf16)
  sim200 the similarity at the 200-frame merge shape, 207,955 x 66,845 x 128
         (not in `all`)
  sim1024 the unprojected 1024-d similarity at the 200-frame shape (not in `all`)
  attn   biased attention, 16 heads x 274,800 queries x 68,700 keys x 64
  sharp  the attention workload with q and k scaled by 40: the score bound
         no longer certifies the fixed softmax offset; most waves take it
         from tile 0 (verified after the loop), the rest the lazily moved
         one (not in `all`)
  own    own-frame attention of the frame-special split, 3,200 (frame, head)
         pairs x 1,374 queries x 1,369 keys, no bias, with LSE (not in `all`)
  shared shared-set attention of the frame-special split, 16 heads x 274,800
         queries x 6,000 keys (1,000 specials + 5,000 pooled), log-size bias,
         with LSE (not in `all`)
  merge  deterministic K/V merge, [1,16,274800,64] fp32 rows into 66,845 slots
  front  merge front end: 274,800 fp32 metric rows of 1024 -> bf16 [dst | src] x 128
  pool   pooled shared set: 16 heads x 200 frames x 1369 patches, 25 seeds
  pool4  the same at pool stride 4: 100 seeds per frame, the super-chunked
         kernel (not in `all`)
  probe  the register-only MFMA probes of csrc/probe/ (32x32x16, 16x16x32,
         the attention's key tile), each on random and on all-zero
         operands, in that order (not in `all`)
  core   biased attention at the 200-frame core-block shape: 16 heads x
         274,800 queries x 219,840 merged keys (not in `all`)
  attn128 attention at head dim 128: 16 heads x 65,536 queries x 68,700 keys,
         log-count bias (the tiled kernel; not in `all`)
  qk     qk LayerNorm + 2D RoPE of a 200-frame block: the bf16 QKV projection
         [1, 274800, 3072] to bf16 q and k, then to bf16 q and fp32 k
  combine LSE combine of the frame-special split at 200 frames (bf16)
  sim16  the similarity workload in fp16
  attn16 the attention workload in fp16
  attn0  the attention workload with all-zero q, k, v (same shapes, bias and
         code path): the instruction stream of `attn` with almost no
         switching in the multipliers, to read the clock the power limit
         allows against `attn` (GRBM_GUI_ACTIVE per dispatch; not in `all`)
  copy   a plain device copy of 1 GiB (bf16), the calibration for HBM byte
         counters: FETCH_SIZE / WRITE_SIZE of this dispatch should read
         1 GiB each, and the ratio to that is the counters' scale factor

Meant to run under `rocprofv3 --kernel-trace --stats` or one
`rocprofv3 --pmc ...` pass at a time; it prints one line per phase.
"""
from __future__ import annotations

import sys
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent
for _p in (str(REPO), str(REPO / "gpa-vggt_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

COPY_BYTES = 1 << 30


def main(argv=None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    which = argv[0] if argv else "all"
    reps = int(argv[1]) if len(argv) > 1 else 3
    if which not in ("sim", "sim200", "sim1024", "attn", "core", "probe", "sharp", "own", "shared", "merge", "front",
                     "pool", "pool4", "attn128", "qk", "combine", "sim16", "attn16", "attn0",
                     "copy", "all"):
        print(__doc__, file=sys.stderr)
        return 2

    import torch
    import gpa_workloads as W
    from merging import _native
    from merging.fused_attention import attention_keybias
    from merging.fused_similarity import fused_similarity_argmax

    dev = torch.device("cuda", 0)
    if which in ("copy", "all"):
        a = torch.empty(COPY_BYTES // 2, dtype=torch.bfloat16, device=dev).fill_(1.0)
        b = torch.empty_like(a)
        for _ in range(reps):
            b.copy_(a)
        torch.cuda.synchronize()
        print(f"copy {COPY_BYTES} bytes x {reps} done", flush=True)
        del a, b
    if which in ("sim", "all"):
        s, d = W.sim_inputs(device=dev)
        for _ in range(reps):
            fused_similarity_argmax(s, d)
        torch.cuda.synchronize()
        print(f"sim 75000x25000x128 x {reps} done", flush=True)
        del s, d
    if which == "sim200":
        s, d = W.sim_inputs(m=207_955, n=66_845, seed=1, device=dev)
        for _ in range(reps):
            fused_similarity_argmax(s, d)
        torch.cuda.synchronize()
        print(f"sim200 207955x66845x128 x {reps} done", flush=True)
        del s, d
    if which == "sim1024":
        s, d = W.sim_inputs(m=207_955, n=66_845, out_dim=1024, seed=4, device=dev)
        for _ in range(reps):
            fused_similarity_argmax(s, d)
        torch.cuda.synchronize()
        print(f"sim1024 207955x66845x1024 x {reps} done", flush=True)
        del s, d
    if which == "sharp":
        q, k, v, b = W.attn_inputs(device=dev)
        q, k = (q.float() * 40).bfloat16(), (k.float() * 40).bfloat16()
        for _ in range(reps):
            attention_keybias(q, k, v, b, 0.125)
        torch.cuda.synchronize()
        print(f"sharp 16x274800x68700x64 (q, k x 40) x {reps} done", flush=True)
        del q, k, v, b
    if which in ("merge", "all"):
        t, off, tok = W.merge_inputs(device=dev)
        for _ in range(reps):
            _native.merge_heads(t, off, tok, off.numel() - 1, True)
        torch.cuda.synchronize()
        print(f"merge [1,16,274800,64] f32 -> 66845 slots x {reps} done", flush=True)
        del t, off, tok
    if which in ("front", "all"):
        from merging.merge import _projection, dst_mask
        g = torch.Generator(device=dev)
        g.manual_seed(33)
        order = torch.argsort(dst_mask(200, 37, 37, 2, 2, 5, False, g, dev), stable=True)
        metric = torch.randn(1, 200 * 1374, 1024, device=dev)
        proj = _projection(dev, 1024, 128)
        for _ in range(reps):
            _native.merge_metric(metric, proj, order, 0)
        torch.cuda.synchronize()
        print(f"front 274800x1024 f32 -> 128 x {reps} done", flush=True)
        del metric, order
    if which in ("pool", "all"):
        kk = (torch.randn(1, 16, 200 * 1374, 64, device=dev) / 8).bfloat16()
        vv = (torch.randn(1, 16, 200 * 1374, 64, device=dev) / 8).bfloat16()
        for _ in range(reps):
            torch.ops.gpa.pool_shared(kk, vv, 200, 5, 37, 37, 8, False)
        torch.cuda.synchronize()
        print(f"pool 16x200 frames kp 8 x {reps} done", flush=True)
        del kk, vv
    if which == "pool4":
        kk = (torch.randn(1, 16, 200 * 1374, 64, device=dev) / 8).bfloat16()
        vv = (torch.randn(1, 16, 200 * 1374, 64, device=dev) / 8).bfloat16()
        for _ in range(reps):
            torch.ops.gpa.pool_shared(kk, vv, 200, 5, 37, 37, 4, False)
        torch.cuda.synchronize()
        print(f"pool4 16x200 frames kp 4 (100 seeds) x {reps} done", flush=True)
        del kk, vv
    if which == "probe":
        import bench
        for _ in range(reps):
            for name, entry in bench.mix_ceiling(dev).items():
                print(f"{name}: {entry['ms']:.3f} ms, {entry['tflops']:.0f} TFLOP/s", flush=True)
        print(f"probe x {reps} done", flush=True)
    if which == "core":
        q, k, v, b = W.attn_inputs(m=274_800, n=219_840, device=dev)
        for _ in range(reps):
            attention_keybias(q, k, v, b, 0.125)
        torch.cuda.synchronize()
        print(f"core 16x274800x219840x64 x {reps} done", flush=True)
        del q, k, v, b
    if which == "attn128":
        q, k, v, b = W.attn_inputs(m=274_800, n=68_700, d=128, device=dev)
        q = q[:, :, :65_536].contiguous()
        for _ in range(reps):
            attention_keybias(q, k, v, b, 128 ** -0.5)
        torch.cuda.synchronize()
        print(f"attn128 16x65536x68700x128 x {reps} done", flush=True)
        del q, k, v, b
    if which in ("qk", "all"):
        import gpa_aggregator as A
        qkv = torch.randn(1, 200 * 1374, 3 * 1024, device=dev).bfloat16()
        ln_w, ln_b = torch.ones(2, 64, device=dev), torch.zeros(2, 64, device=dev)
        rope = A.Rope2D(100.0).table(A.frame_positions(37, 5, dev), 64)
        for k_f32 in (False, True):
            for _ in range(reps):
                torch.ops.gpa.qk_norm_rope(qkv, ln_w, ln_b, 1e-5, rope.pos, rope.cs, 16, False,
                                           k_f32)
        torch.cuda.synchronize()
        print(f"qk 274800 tokens x 16 heads (bf16 k, fp32 k) x {reps} done", flush=True)
        del qkv
    if which in ("combine", "all"):
        oa = (torch.randn(200, 16, 1374, 64, device=dev) / 8).bfloat16()
        la = torch.randn(200, 16, 1374, device=dev)
        ob = (torch.randn(1, 16, 200 * 1374, 64, device=dev) / 8).bfloat16()
        lb = torch.randn(1, 16, 200 * 1374, device=dev)
        for _ in range(reps):
            torch.ops.gpa.lse_combine(oa, la, ob, lb, 200)
        torch.cuda.synchronize()
        print(f"combine 200 frames x 16 heads x 1374 x {reps} done", flush=True)
        del oa, la, ob, lb
    if which == "shared":
        q = (torch.randn(1, 16, 200 * 1374, 64, device=dev) / 8).bfloat16()
        k = (torch.randn(1, 16, 6000, 64, device=dev) / 8).bfloat16()
        v = (torch.randn(1, 16, 6000, 64, device=dev) / 8).bfloat16()
        bias = torch.zeros(1, 16, 1, 6000, device=dev)
        bias[..., 1000:] = torch.randint(1, 100, (1, 16, 1, 5000), device=dev).float().log()
        bias = bias.bfloat16()
        for _ in range(reps):
            attention_keybias(q, k, v, bias, 0.125, return_lse=True)
        torch.cuda.synchronize()
        print(f"shared 16x274800x6000x64 x {reps} done", flush=True)
        del q, k, v, bias
    if which in ("sim16", "all"):
        s, d = W.sim_inputs(device=dev)
        s, d = s.half(), d.half()
        for _ in range(reps):
            fused_similarity_argmax(s, d)
        torch.cuda.synchronize()
        print(f"sim16 75000x25000x128 x {reps} done", flush=True)
        del s, d
    if which in ("attn", "attn16", "all"):
        q, k, v, b = W.attn_inputs(device=dev)
        if which in ("attn", "all"):
            for _ in range(reps):
                attention_keybias(q, k, v, b, 0.125)
            torch.cuda.synchronize()
            print(f"attn 16x274800x68700x64 x {reps} done", flush=True)
        if which in ("attn16", "all"):
            q, k, v, b = q.half(), k.half(), v.half(), b.half()
            for _ in range(reps):
                attention_keybias(q, k, v, b, 0.125)
            torch.cuda.synchronize()
            print(f"attn16 16x274800x68700x64 x {reps} done", flush=True)
    if which == "own":
        qf = (torch.randn(200, 16, 1374, 64, device=dev) / 8).bfloat16()
        kf = (torch.randn(200, 16, 1369, 64, device=dev) / 8).bfloat16()
        vf = (torch.randn(200, 16, 1369, 64, device=dev) / 8).bfloat16()
        for _ in range(reps):
            attention_keybias(qf, kf, vf, None, 0.125, return_lse=True)
        torch.cuda.synchronize()
        print(f"own 3200x1374x1369x64 x {reps} done", flush=True)
        del qf, kf, vf
    if which == "attn0":
        q, k, v, b = W.attn_inputs(device=dev)
        q, k, v = torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
        for _ in range(reps):
            attention_keybias(q, k, v, b, 0.125)
        torch.cuda.synchronize()
        print(f"attn0 16x274800x68700x64 (zero q, k, v) x {reps} done", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
