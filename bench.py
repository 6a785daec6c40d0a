#!/usr/bin/env python3
"""Benchmark of the GPA-VGGT merging hot path on one MI355X.

One step = one fused similarity-argmax call on the 75,000 x 25,000 x 128
workload plus one biased-attention call on the 200-frame merged-block
workload (16 heads, 274,800 queries, 68,700 merged keys, head_dim 64), both
on synthetic inputs already resident in HBM.  `value` is the step's
algorithmic TFLOP/s (2*M*N*D for the similarity, 4*BH*M*N*D for attention).
The JSON line also carries per-kernel ms / TFLOP/s / % of the bf16 dense
MFMA peak (the reference 200-frame shapes, the unprojected 1024-d
similarity, the frame-special calls, the HBM-bound kernels around the path,
the fp16 twins, and attention on larger logits -- LayerNorm-scale and sharp
q/k -- with the shares of waves on the tile-0 and the lazily moved softmax
offsets), the practical MFMA ceiling (a hipBLASLt bf16 GEMM on random and on
all-zero data, and register-only probes of the MFMA shapes and of the
attention's own instruction mix), the end-to-end latency of one GPA block (100
frames) and of the whole aggregator (200 frames) on the random-init VGGT-1B
harness for the GPA schedule and for vanilla VGGT, the roofline of the
dominant kernel and a CPU baseline (the torch restatement of the reference
path, timed on a bounded sample on this host).

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (str(REPO), str(REPO / "gpa-vggt_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_BF16_TFLOPS = 2516.6     # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 FLOP/clk)
HBM_BYTES_PER_S = 8.0e12      # MI355X HBM3E
SM_SCALE = 64 ** -0.5
TRAFFIC_FILE = REPO / "profiles" / "attn_keybias_traffic.json"
PROBE_LIB = REPO / "gpa-vggt_amd" / "merging" / "_lib" / "libgpa_probe.so"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description="GPA-VGGT merging hot path benchmark (1 GPU)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-200f", action="store_true", help="skip the 200-frame shape sweep")
    ap.add_argument("--cpu-budget", type=float, default=8.0,
                    help="seconds of CPU work per baseline leg (similarity, attention)")
    ap.add_argument("--no-e2e", action="store_true",
                    help="skip the GPA block (100 frames) and aggregator (200 frames) latencies")
    return ap.parse_args(argv)


def e2e_latency(dev) -> dict:
    """End-to-end latencies on the random-init VGGT-1B aggregator harness.

    * GPA block: one merged global block (LayerNorm -> QKV -> projected
      similarity-argmax -> K/V merge -> biased attention -> proj -> MLP) on
      100 frames x 1374 tokens from shifted-texture images;
    * aggregator: the full stack (DINOv2 ViT-L/14 patch embed, 24 frame + 24
      global blocks on the GPA schedule) on 200 frames of 518 x 518 images,
      with the reference defaults, and with the variant of 64 pooled patch
      summaries per frame in the shared set (pool stride 5) and every merged
      block at 25 % keep (no core blocks), and with the unprojected 1024-d
      merge metric (`--merge_metric_dim 0`, eval/eval_co3d.py:121-122);
    * the same aggregator without GPA (vanilla VGGT) and, with the reference
      defaults, as the fp16 accuracy-evaluation stack.
    Timing follows eval/bench_e2e.py: 2 warm-up calls, mean of 3 (1 and 2 for
    the vanilla and fp16 forwards).
    """
    import torch
    import gpa_aggregator as A

    res = {}
    bf16 = torch.bfloat16

    def run(fn):
        def call():
            with torch.no_grad(), torch.autocast("cuda", dtype=bf16):
                return fn()
        return call

    cfg = A.GpaConfig()
    model = A.build_aggregator(cfg, device=dev)
    frames = 100
    imgs = A.shifted_texture_images(frames, device=dev).to(bf16)
    with torch.no_grad(), torch.autocast("cuda", dtype=bf16):
        tokens = model.embed(imgs).reshape(1, frames * cfg.tokens_per_frame, cfg.embed_dim)
    rope = model.rope_table(dev)
    blk = model.global_blocks[9]
    ms, peak = A.timed(run(lambda: blk(tokens, rope, 9)))
    res["gpa_block_100f"] = {
        "ms": round(ms, 2), "peak_gib": round(peak, 2),
        "workload": "merged global block 9 (ratio 0.98): 137,400 tokens -> 33,945 merged keys"}
    del tokens, imgs
    log(f"[bench] GPA block 100 frames: {ms:.1f} ms")

    frames = 200
    imgs = A.shifted_texture_images(frames, device=dev).to(bf16)
    variants = (("reference_defaults", cfg, model),
                ("pool64_keep25", A.GpaConfig(broadcast_pool=5, core_blocks=()), None),
                ("metric_dim0", A.GpaConfig(merge_metric_dim=0), None))
    for tag, c, m in variants:
        if m is None:
            m = A.build_aggregator(c, device=dev)
        ms, peak = A.timed(run(lambda: m(imgs)))
        tracer = A.StageTimer()
        m.set_tracer(tracer)
        tracer.start()
        run(lambda: m(imgs))()
        stages = tracer.totals()
        m.set_tracer(None)
        flops = A.aggregator_flops(c, frames)
        res[f"aggregator_200f_{tag}"] = {
            "ms": round(ms, 1), "peak_gib": round(peak, 2),
            "stages_ms": {k: round(v, 2) for k, v in sorted(stages.items(), key=lambda kv: -kv[1])},
            "tflop": {k: round(v / 1e12, 2) for k, v in flops.items()},
            "schedule": {"early_frame_split": c.early_frame_split, "broadcast_pool": c.broadcast_pool,
                         "merge": [c.merging, c.merge_end, c.merge_ratio],
                         "core_blocks": list(c.core_blocks), "core_merge_ratio": c.core_merge_ratio,
                         "merge_metric_dim": c.merge_metric_dim}}
        log(f"[bench] aggregator 200 frames ({tag}): {ms:.1f} ms")
        del m
        torch.cuda.empty_cache()
    # Vanilla VGGT on the same harness and images (eval_co3d.py:127-128: no
    # merging, no frame-special blocks): every global block attends over all
    # 274,800 tokens.  ~7 s per forward, so 1 warm-up call and the mean of 2.
    vcfg = A.vanilla_config()
    vm = A.build_aggregator(vcfg, device=dev)
    ms, peak = A.timed(run(lambda: vm(imgs)), warmup=1, iters=2)
    flops = A.aggregator_flops(vcfg, frames)
    gpa_ms = res["aggregator_200f_reference_defaults"]["ms"]
    res["aggregator_200f_vanilla"] = {
        "ms": round(ms, 1), "peak_gib": round(peak, 2),
        "tflop": {k: round(v / 1e12, 2) for k, v in flops.items()},
        "protocol": "1 warm-up call, mean of 2",
        "gpa_speedup": round(ms / gpa_ms, 3),
        "reference_speedup": "2.58x at 200 frames (README.md:21, reference hardware not stated)"}
    log(f"[bench] aggregator 200 frames (vanilla): {ms:.1f} ms, GPA speed-up {ms / gpa_ms:.2f}x")
    del vm
    torch.cuda.empty_cache()
    # The accuracy-evaluation stack of the reference (eval_co3d.py:152, 226):
    # the fp16 model under fp16 autocast, reference defaults; every kernel
    # runs as its fp16 twin.
    f16 = torch.float16
    fm = A.build_aggregator(cfg, device=dev, dtype=f16)
    imgs16 = imgs.to(f16)

    def run16():
        with torch.no_grad(), torch.autocast("cuda", dtype=f16):
            return fm(imgs16)
    ms, peak = A.timed(run16, warmup=1, iters=2)
    tracer = A.StageTimer()
    fm.set_tracer(tracer)
    tracer.start()
    run16()
    stages = tracer.totals()
    fm.set_tracer(None)
    res["aggregator_200f_fp16_eval_stack"] = {
        "ms": round(ms, 1), "peak_gib": round(peak, 2), "protocol": "1 warm-up call, mean of 2",
        "stages_ms": {k: round(v, 2) for k, v in sorted(stages.items(), key=lambda kv: -kv[1])},
        "workload": "reference defaults, fp16 model under fp16 autocast (eval_co3d.py:152, 226)"}
    log(f"[bench] aggregator 200 frames (fp16 evaluation stack): {ms:.1f} ms")
    del fm, imgs16, imgs
    torch.cuda.empty_cache()
    return res


def event_ms(fn, reps: int):
    """Per-call device time (ms) from events on torch's current stream."""
    import torch
    out = []
    for _ in range(reps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        out.append((s, e))
    torch.cuda.synchronize()
    return [s.elapsed_time(e) for s, e in out]


def attention_floor(q, k, v, bias, biased_ms: float) -> dict:
    """The unbiased floor of the headline attention on this box, measured
    the way the reference judges its own kernel (merging/fused_attention.py:
    23-25: the biased kernel against a flash kernel without bias).

    * this kernel with bias=None on the same q, k, v;
    * torch's unmasked F.scaled_dot_product_attention, restricted to one
      fused backend at a time (flash, then memory-efficient; the math
      backend is never allowed: it would materialise a 274,800 x 68,700
      score matrix per head);
    * torch's masked SDPA with the same log-count bias, the reference's
      own GPU fallback (vggt/layers/attention.py:270-276).
    Each entry: ms, TFLOP/s, % of peak, and biased_ms / its ms.
    """
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    import gpa_workloads as W
    from merging.fused_attention import attention_keybias

    f = W.attn_flops(q.shape[1], q.shape[2], k.shape[2], q.shape[3])
    out = {}

    def entry(name, fn, reps=3, **extra):
        try:
            fn()
            t = statistics.median(event_ms(fn, reps))
        except RuntimeError as e:       # backend not built for this device / shape
            out[name] = {"error": str(e).splitlines()[0][:200]}
            log(f"[bench] {name}: unavailable ({out[name]['error']})")
            return
        ent = kernel_entry(f, t)
        ent["biased_over_this"] = round(biased_ms / t, 4)
        ent.update(extra)
        out[name] = ent
        log(f"[bench] {name}: {t:.2f} ms")

    entry("gpa_attn_no_bias", lambda: attention_keybias(q, k, v, None, SM_SCALE))
    for be, tag in ((SDPBackend.FLASH_ATTENTION, "flash"),
                    (SDPBackend.EFFICIENT_ATTENTION, "efficient")):
        def sdpa(be=be):
            with sdpa_kernel([be]):
                return F.scaled_dot_product_attention(q, k, v, scale=SM_SCALE)
        entry(f"torch_sdpa_unmasked_{tag}", sdpa, backend=str(be))
    def sdpa_masked():
        # [B, H, 1, N], broadcast over the queries, as the reference passes it
        with sdpa_kernel([SDPBackend.EFFICIENT_ATTENTION]):
            return F.scaled_dot_product_attention(q, k, v, attn_mask=bias, scale=SM_SCALE)
    entry("torch_sdpa_masked_efficient", sdpa_masked, backend=str(SDPBackend.EFFICIENT_ATTENTION))
    torch.cuda.empty_cache()
    nb = out.get("gpa_attn_no_bias", {})
    if "ms" in nb:
        out["bias_overhead_pct"] = round(100.0 * (biased_ms / nb["ms"] - 1.0), 2)
    return out


def mix_ceiling(dev) -> dict:
    """What the power limit leaves for an instruction mix, from the
    register-only probes of csrc/probe/mfma_mix_probe.hip (no memory traffic
    in the loop; two waves per SIMD as the attention runs): 32x32x16 and
    16x16x32 bf16 MFMAs alone, and one key tile of the attention main loop
    (its 16 MFMAs of 32x32x16, row-sum MFMAs and softmax VALU work, FLOPs
    counted as the attention counts them), each on random operands and on
    all-zero ones.  {} when the probe library is not built."""
    import ctypes

    import torch
    if not PROBE_LIB.exists():
        log(f"[bench] {PROBE_LIB.name} not built: no instruction-mix ceiling")
        return {}
    lib = ctypes.CDLL(str(PROBE_LIB))
    lib.gpa_probe_mfma_mix.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                       ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    lib.gpa_probe_flops.restype = ctypes.c_double
    lib.gpa_probe_flops.argtypes = [ctypes.c_int, ctypes.c_int]
    nsrc = 1 << 20                                   # 16-byte fragments
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    srcs = {"random": (torch.rand(nsrc * 8, generator=g, device=dev) * 2 - 1).bfloat16(),
            "zeros": torch.zeros(nsrc * 8, device=dev, dtype=torch.bfloat16)}
    out = torch.empty(lib.gpa_probe_threads(), device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    res = {}
    for mode, iters, name in ((0, 600_000, "mfma_32x32x16"), (1, 600_000, "mfma_16x16x32"),
                              (2, 250_000, "attention_tile_mix")):
        for tag, src in srcs.items():
            def fn(mode=mode, src=src, iters=iters):
                rc = lib.gpa_probe_mfma_mix(mode, src.data_ptr(), nsrc, out.data_ptr(), iters,
                                            stream)
                if rc != 0:
                    raise RuntimeError(f"gpa_probe_mfma_mix mode {mode} returned {rc}")
            fn()
            t = statistics.median(event_ms(fn, 3))
            res[f"probe_{name}_{tag}"] = kernel_entry(lib.gpa_probe_flops(mode, iters), t)
    del srcs, out
    return res


def kernel_entry(flops: float, ms: float) -> dict:
    tf = flops / (ms * 1e-3) / 1e12
    return {"ms": round(ms, 4), "tflops": round(tf, 2), "pct_peak": round(100 * tf / PEAK_BF16_TFLOPS, 2),
            "flops": flops}


def cpu_baseline(src, dst, q, k, v, bias, budget: float) -> dict:
    """Reference torch path on the host, on a bounded sample of the same workload."""
    import torch
    import gpa_workloads as W
    from oracle.attention import sdpa_reference
    from oracle.similarity import fast_similarity_chunks

    threads = torch.get_num_threads()
    a_h, b_h = src.cpu(), dst.cpu()
    m_full, n_sim, d_sim = a_h.shape[1], b_h.shape[1], a_h.shape[2]
    bt = b_h.transpose(1, 2)

    def sim_rows(rows):
        t = time.perf_counter()
        fast_similarity_chunks(a_h[:, :rows], bt, 5000)
        return time.perf_counter() - t

    rows = 1000
    dt = sim_rows(rows)
    rows = int(min(m_full, max(rows, rows * budget / max(dt, 1e-3))))
    dt = sim_rows(rows)
    sim_rate = W.sim_flops(1, rows, n_sim, d_sim) / dt

    qh = q[:, :, :4096].float().cpu()
    kh, vh, bh = k.float().cpu(), v.float().cpu(), bias.float().cpu()
    H, n_attn, d = kh.shape[1], kh.shape[2], kh.shape[3]

    def attn_rows(rows):
        t = time.perf_counter()
        sdpa_reference(qh[:, :, :rows], kh, vh, bh, SM_SCALE)
        return time.perf_counter() - t

    qrows = 16
    dt = attn_rows(qrows)
    qrows = int(min(4096, max(qrows, qrows * budget / max(dt, 1e-3))))
    dt = attn_rows(qrows)
    attn_rate = W.attn_flops(H, qrows, n_attn, d) / dt

    f_sim = W.sim_flops(1, m_full, n_sim, d_sim)
    f_attn = W.attn_flops(H, q.shape[2], n_attn, d)
    value = (f_sim + f_attn) / (f_sim / sim_rate + f_attn / attn_rate) / 1e12
    return {
        "value": round(value, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
        "sample": (f"torch CPU restatement of the reference path: fast_similarity_chunks "
                   f"(bf16 bmm+max, chunk 5000) on {rows} of {m_full} source rows "
                   f"({sim_rate / 1e12:.4f} TFLOP/s), fp32 SDPA with the log-count bias on "
                   f"{qrows} of {q.shape[2]} queries x {H} heads x {n_attn} keys "
                   f"({attn_rate / 1e12:.4f} TFLOP/s); per-step time extrapolated linearly "
                   f"(rows are independent)"),
        "host_cpus": os.cpu_count(),
        "cpu_model": _cpu_model(),
    }


def _cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or "" where it is not readable."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def main(argv=None) -> int:
    args = parse_args(argv)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the merging hot path has no multi-GPU path here "
              f"(asked for --gpus {args.gpus}, WORLD_SIZE {world}).", file=sys.stderr)
        return 2

    import torch
    import gpa_workloads as W
    from merging import _native
    from merging.fused_attention import attention_keybias
    from merging.fused_similarity import fused_similarity_argmax

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log(f"[bench] device {torch.cuda.get_device_name(dev)}; library {_native.LIB_PATH}")

    src, dst = W.sim_inputs(m=75_000, n=25_000, seed=0, device=dev)
    q, k, v, bias = W.attn_inputs(m=274_800, n=68_700, seed=0, device=dev)
    torch.cuda.synchronize()
    f_sim = W.sim_flops(1, src.shape[1], dst.shape[1], src.shape[2])
    f_attn = W.attn_flops(q.shape[1], q.shape[2], k.shape[2], q.shape[3])

    def sim():
        return fused_similarity_argmax(src, dst)

    def attn():
        return attention_keybias(q, k, v, bias, SM_SCALE)

    for _ in range(args.warmup):
        sim()
        attn()
    torch.cuda.synchronize()
    log(f"[bench] warmup {args.warmup} done; timing {args.steps} steps")

    ev = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record()
        sim()
        e[1].record()
        attn()
        e[2].record()
        ev.append(e)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_step = elapsed / args.steps * 1e3
    sim_ms = statistics.median(e[0].elapsed_time(e[1]) for e in ev)
    attn_ms = statistics.median(e[1].elapsed_time(e[2]) for e in ev)
    value = (f_sim + f_attn) / (ms_step * 1e-3) / 1e12
    log(f"[bench] step {ms_step:.3f} ms: sim {sim_ms:.3f} ms, attn {attn_ms:.3f} ms")

    kernels = {"sim_argmax_75000x25000x128": kernel_entry(f_sim, sim_ms),
               "attn_keybias_16h_274800x68700": kernel_entry(f_attn, attn_ms)}
    # The similarity call alone, back to back (in the step it follows a
    # 65 ms attention call: cold caches for its operands and the clock the
    # power limit left).
    fn = lambda: fused_similarity_argmax(src, dst)  # noqa: E731
    fn()
    kernels["sim_argmax_75000x25000x128_back_to_back"] = kernel_entry(
        f_sim, statistics.median(event_ms(fn, 20)))

    floor = attention_floor(q, k, v, bias, attn_ms)

    if not args.no_200f:
        # Reference defaults at 200 frames x 1374 tokens: 207,955 source and
        # 66,845 destination tokens; merged keys 66,845 (aggressive blocks) and
        # 219,840 (core blocks, 80% kept).
        del src, dst
        s2, d2 = W.sim_inputs(m=207_955, n=66_845, seed=1, device=dev)
        fn = lambda: fused_similarity_argmax(s2, d2)  # noqa: E731
        fn()
        t = statistics.median(event_ms(fn, 5))
        kernels["sim_argmax_200f_207955x66845x128"] = kernel_entry(W.sim_flops(1, 207_955, 66_845, 128), t)
        del s2, d2
        for nk, tag in ((66_845, "aggressive"), (219_840, "core")):
            q2, k2, v2, b2 = W.attn_inputs(m=274_800, n=nk, seed=2, device=dev)
            fn = lambda: attention_keybias(q2, k2, v2, b2, SM_SCALE)  # noqa: E731
            fn()
            t = statistics.median(event_ms(fn, 3))
            kernels[f"attn_keybias_200f_{tag}_16h_274800x{nk}"] = kernel_entry(
                W.attn_flops(16, 274_800, nk, 64), t)
            del q2, k2, v2, b2
        # Row f1: the deterministic K/V merge at the 200-frame shape (all
        # 207,955 source tokens merged into 66,845 slots), K fp32 and V bf16.
        from merging import _native
        for dt, tag, elem in ((torch.float32, "k_f32", 4), (torch.bfloat16, "v_bf16", 2)):
            t3, off3, tok3 = W.merge_inputs(m=274_800, n=66_845, dtype=dt, seed=3, device=dev)
            fn = lambda: _native.merge_heads(t3, off3, tok3, 66_845, True)  # noqa: E731
            fn()
            t = statistics.median(event_ms(fn, 5))
            nbytes = W.merge_bytes(274_800, 66_845, 16, 64, elem)
            kernels[f"merge_heads_200f_{tag}_16h_274800to66845"] = {
                "ms": round(t, 4), "gbps": round(nbytes / (t * 1e-3) / 1e9, 1),
                "pct_hbm": round(100 * nbytes / (t * 1e-3) / HBM_BYTES_PER_S, 2), "bytes": nbytes}
            del t3, off3, tok3
        # Row f2: the frame-special split path at 200 frames: own-frame
        # attention (200 frames x 16 heads, 1374 queries x 1369 keys, LSE),
        # shared-set attention (274,800 queries x 6,000 keys with the pooled
        # log-size bias, LSE), and the LSE combine into [1, 274800, 1024].
        from merging.fused_attention import combine_by_lse
        S, P, pts, npool = 200, 1374, 5, 25
        qf = (torch.randn(S, 16, P, 64, device=dev) / 8).bfloat16()
        kf = (torch.randn(S, 16, P - pts, 64, device=dev) / 8).bfloat16()
        vf = (torch.randn(S, 16, P - pts, 64, device=dev) / 8).bfloat16()
        fn = lambda: attention_keybias(qf, kf, vf, None, SM_SCALE, return_lse=True)  # noqa: E731
        out_a, lse_a = fn()
        t = statistics.median(event_ms(fn, 5))
        kernels["attn_frame_own_3200bh_1374x1369"] = kernel_entry(W.attn_flops(S * 16, P, P - pts, 64), t)
        # The same call on torch's own fused kernels (no bias, so flash and
        # memory-efficient SDPA apply; outputs only, no LSE): the floor a
        # caller without this library would get at the frame shape.
        from torch.nn.attention import SDPBackend, sdpa_kernel
        own_floor = {}
        for be, tag in ((SDPBackend.FLASH_ATTENTION, "flash"),
                        (SDPBackend.EFFICIENT_ATTENTION, "efficient")):
            def sdpa_own(be=be):
                with sdpa_kernel([be]):
                    return torch.nn.functional.scaled_dot_product_attention(qf, kf, vf, scale=SM_SCALE)
            try:
                sdpa_own()
                ts = statistics.median(event_ms(sdpa_own, 5))
                ent = kernel_entry(W.attn_flops(S * 16, P, P - pts, 64), ts)
                ent["this_kernel_speedup"] = round(ts / t, 3)
                ent["backend"] = str(be)
                own_floor[f"torch_sdpa_unmasked_{tag}"] = ent
                log(f"[bench] own-frame shape, torch SDPA {tag}: {ts:.3f} ms")
            except RuntimeError as e:
                own_floor[f"torch_sdpa_unmasked_{tag}"] = {"error": str(e).splitlines()[0][:200]}
        kernels["attn_frame_own_3200bh_1374x1369"]["floor"] = own_floor
        del kf, vf
        qs = qf.view(1, S, 16, P, 64).permute(0, 2, 1, 3, 4).reshape(1, 16, S * P, 64)
        del qf
        ks = (torch.randn(1, 16, S * (pts + npool), 64, device=dev) / 8).bfloat16()
        vs = (torch.randn(1, 16, S * (pts + npool), 64, device=dev) / 8).bfloat16()
        bs = torch.zeros(1, 16, 1, S * (pts + npool), device=dev)
        bs[..., S * pts:] = torch.randint(1, 12, (1, 16, 1, S * npool), device=dev).float().log()
        bs = bs.bfloat16()
        fn = lambda: attention_keybias(qs, ks, vs, bs, SM_SCALE, return_lse=True)  # noqa: E731
        out_b, lse_b = fn()
        t = statistics.median(event_ms(fn, 5))
        kernels["attn_frame_shared_16h_274800x6000"] = kernel_entry(
            W.attn_flops(16, S * P, S * (pts + npool), 64), t)
        fn = lambda: combine_by_lse(out_a, lse_a, out_b, lse_b, S)  # noqa: E731
        fn()
        t = statistics.median(event_ms(fn, 5))
        nbytes = 3 * S * P * 16 * 64 * 2 + 2 * S * P * 16 * 4
        kernels["lse_combine_200f_16h_274800"] = {
            "ms": round(t, 4), "gbps": round(nbytes / (t * 1e-3) / 1e9, 1),
            "pct_hbm": round(100 * nbytes / (t * 1e-3) / HBM_BYTES_PER_S, 2), "bytes": nbytes}
        del qs, ks, vs, bs, out_a, lse_a, out_b, lse_b
        # Row f2: the pooled shared set at 200 frames: kp 8 (25 seeds per
        # frame, seeds in registers) and kp 4 (100 seeds, super-chunks of 64).
        kk = (torch.randn(1, 16, S * P, 64, device=dev) / 8).bfloat16()
        vv = (torch.randn(1, 16, S * P, 64, device=dev) / 8).bfloat16()
        for kp in (8, 4):
            fn = lambda: torch.ops.gpa.pool_shared(kk, vv, S, pts, 37, 37, kp, False)  # noqa: E731
            fn()
            t = statistics.median(event_ms(fn, 5))
            nbytes = 2 * 16 * S * (P - pts) * 64 * 2
            kernels[f"pool_shared_200f_16h_kp{kp}"] = {
                "ms": round(t, 4), "gbps": round(nbytes / (t * 1e-3) / 1e9, 1),
                "pct_hbm": round(100 * nbytes / (t * 1e-3) / HBM_BYTES_PER_S, 2), "bytes": nbytes,
                "seeds_per_frame": (-(-37 // kp)) ** 2}
        del kk, vv
        # Row f3: the merge front end (projection 1024 -> 128, normalise,
        # [dst | src] gather, bf16) on the fp32 norm1 output of 274,800 tokens.
        from merging.merge import _projection, dst_mask
        g = torch.Generator(device=dev)
        g.manual_seed(33)
        order = torch.argsort(dst_mask(S, 37, 37, 2, 2, pts, False, g, dev), stable=True)
        metric = torch.randn(1, S * P, 1024, device=dev)
        proj = _projection(dev, 1024, 128)
        fn = lambda: _native.merge_metric(metric, proj, order, 0)  # noqa: E731
        fn()
        t = statistics.median(event_ms(fn, 5))
        nbytes = S * P * (1024 * 4 + 128 * 2)
        kernels["merge_metric_200f_274800x1024_f32"] = {
            "ms": round(t, 4), "gbps": round(nbytes / (t * 1e-3) / 1e9, 1),
            "pct_hbm": round(100 * nbytes / (t * 1e-3) / HBM_BYTES_PER_S, 2), "bytes": nbytes}
        del metric, order
        # The fused qk LayerNorm + 2D RoPE + cast of every aggregator block
        # (vggt/layers/attention.py:210-220) at 200 frames: the bf16 QKV
        # projection [1, 274800, 3072] in, q and k [1, 16, 274800, 64] out
        # (bf16, and fp32 k as the merged blocks keep it for the K merge).
        import gpa_aggregator as A
        qkv = (torch.randn(1, S * P, 3 * 1024, device=dev)).bfloat16()
        ln_w = torch.ones(2, 64, device=dev)
        ln_b = torch.zeros(2, 64, device=dev)
        rope = A.Rope2D(100.0).table(A.frame_positions(37, pts, dev), 64)
        for k_f32, tag in ((False, "bf16"), (True, "k_f32")):
            fn = lambda: torch.ops.gpa.qk_norm_rope(qkv, ln_w, ln_b, 1e-5, rope.pos, rope.cs,  # noqa: E731
                                                    16, False, k_f32)
            fn()
            t = statistics.median(event_ms(fn, 5))
            nbytes = S * P * (2 * 1024 * 2 + 1024 * 2 + 1024 * (4 if k_f32 else 2))
            kernels[f"qk_norm_rope_200f_274800x16h_{tag}"] = {
                "ms": round(t, 4), "gbps": round(nbytes / (t * 1e-3) / 1e9, 1),
                "pct_hbm": round(100 * nbytes / (t * 1e-3) / HBM_BYTES_PER_S, 2), "bytes": nbytes}
        del qkv
        # The unprojected metric (metric_dim=0, D = 1024) at the 200-frame
        # shape: the 256 x 256-tile similarity kernel.
        s3, d3 = W.sim_inputs(m=207_955, n=66_845, out_dim=1024, seed=4, device=dev)
        fn = lambda: fused_similarity_argmax(s3, d3)  # noqa: E731
        fn()
        t = statistics.median(event_ms(fn, 3))
        kernels["sim_argmax_200f_207955x66845x1024"] = kernel_entry(
            W.sim_flops(1, 207_955, 66_845, 1024), t)
        del s3, d3
        # Head dims other than 64 (the reference kernel's HEAD_DIM is a
        # template constant): 128, 16 heads x 65,536 queries x 68,700 keys.
        qd = (torch.randn(1, 16, 65_536, 128, device=dev) / 8).bfloat16()
        kd = (torch.randn(1, 16, 68_700, 128, device=dev) / 8).bfloat16()
        vd = (torch.randn(1, 16, 68_700, 128, device=dev) / 8).bfloat16()
        bd = bias[..., :68_700]
        fn = lambda: attention_keybias(qd, kd, vd, bd, 128 ** -0.5)  # noqa: E731
        fn()
        t = statistics.median(event_ms(fn, 3))
        kernels["attn_keybias_d128_16h_65536x68700"] = kernel_entry(
            W.attn_flops(16, 65_536, 68_700, 128), t)
        del qd, kd, vd
        # ... and 256, 16 heads x 32,768 queries (the same FLOP count).
        qd = (torch.randn(1, 16, 32_768, 256, device=dev) / 8).bfloat16()
        kd = (torch.randn(1, 16, 68_700, 256, device=dev) / 8).bfloat16()
        vd = (torch.randn(1, 16, 68_700, 256, device=dev) / 8).bfloat16()
        fn = lambda: attention_keybias(qd, kd, vd, bd, 256 ** -0.5)  # noqa: E731
        fn()
        t = statistics.median(event_ms(fn, 3))
        kernels["attn_keybias_d256_16h_32768x68700"] = kernel_entry(
            W.attn_flops(16, 32_768, 68_700, 256), t)
        del qd, kd, vd, bd
        log("[bench] 200-frame shapes done")

    if not args.no_200f:
        # Row f4: the fp16 twins at the headline shapes (fp16 autocast stack).
        sh, dh = W.sim_inputs(m=75_000, n=25_000, seed=0, device=dev)
        sh, dh = sh.half(), dh.half()
        fn = lambda: fused_similarity_argmax(sh, dh)  # noqa: E731
        fn()
        t = statistics.median(event_ms(fn, 10))
        kernels["sim_argmax_f16_75000x25000x128"] = kernel_entry(f_sim, t)
        del sh, dh
        qh, kh, vh, bh = q.half(), k.half(), v.half(), bias.half()
        fn = lambda: attention_keybias(qh, kh, vh, bh, SM_SCALE)  # noqa: E731
        fn()
        t = statistics.median(event_ms(fn, 3))
        kernels["attn_keybias_f16_16h_274800x68700"] = kernel_entry(f_attn, t)
        del qh, kh, vh, bh
        log("[bench] fp16 shapes done")
        # Larger logits: q and k scaled up so the Cauchy-Schwarz score bound
        # sits above what the bound-certified softmax offset covers, and
        # waves take the tile-0 offset (verified after the loop) or the
        # lazily moved one (same workload otherwise).  x8 puts the features
        # at LayerNorm scale (unit variance, as the model's qk norm leaves
        # them), where fp16's 16-unit window no longer certifies most rows.
        # The shares come from the kernel's per-wave flags.
        for dt, scale in ((torch.bfloat16, 8.0), (torch.float16, 8.0), (torch.bfloat16, 40.0),
                          (torch.float16, 6.0), (torch.float16, 12.0)):
            qs, ks = (q.float() * scale).to(dt), (k.float() * scale).to(dt)
            vs, bs = v.to(dt), bias.to(dt)
            _, _, flags = _native.attn_keybias_offset_flags(qs, ks, vs, bs, SM_SCALE)
            fl = flags.view(q.shape[1], -1)[:, :-(-q.shape[2] // 64)]     # waves holding queries
            share = lambda bit: round(100 * float(((fl & bit) != 0).float().mean().item()), 2)  # noqa: E731
            fn = lambda: attention_keybias(qs, ks, vs, bs, SM_SCALE)  # noqa: E731
            fn()
            t = statistics.median(event_ms(fn, 3))
            tag = "bf16" if dt == torch.bfloat16 else "f16"
            entry = kernel_entry(f_attn, t)
            base = attn_ms if dt == torch.bfloat16 else \
                kernels["attn_keybias_f16_16h_274800x68700"]["ms"]
            entry.update({"qk_scale": scale,
                          "tile0_offset_waves_pct": share(_native.ATTN_FLAG_TILE0),
                          "lazy_waves_pct": share(_native.ATTN_FLAG_LAZY),
                          "recomputed_waves_pct": share(_native.ATTN_FLAG_RERUN),
                          "vs_certified": round(t / base, 3)})
            name = "lnscale" if scale == 8.0 else f"sharp_{tag}_x{int(scale)}"
            kernels[f"attn_keybias_{name}{'_' + tag if scale == 8.0 else ''}_16h_274800x68700"] = entry
            del qs, ks, vs, bs, flags, fl
        log("[bench] sharp-logit shapes done")

    # The MFMA rate this part sustains on random data under its power limit:
    # a plain hipBLASLt bf16 GEMM (torch.matmul, 16384^3, N(0,1) operands),
    # and the same GEMM on all-zero operands (the multipliers do not toggle,
    # so the clock stays high).  Context for the attention's fraction of the
    # nominal peak; not part of the step.
    ceiling = {}
    n = 16_384
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    for tag in ("randn", "zeros"):
        if tag == "zeros":
            a = torch.zeros(n, n, device=dev, dtype=torch.bfloat16)
            b = torch.zeros(n, n, device=dev, dtype=torch.bfloat16)
        else:
            a = torch.randn(n, n, generator=g, device=dev).bfloat16()
            b = torch.randn(n, n, generator=g, device=dev).bfloat16()
        fn = lambda: a @ b  # noqa: E731
        fn()
        t = statistics.median(event_ms(fn, 7))
        ceiling[f"hipblaslt_gemm_bf16_{n}_{tag}"] = kernel_entry(2.0 * n ** 3, t)
        del a, b
    torch.cuda.empty_cache()
    gemm_tf = ceiling[f"hipblaslt_gemm_bf16_{n}_randn"]["tflops"]
    log(f"[bench] hipBLASLt GEMM ceiling {gemm_tf:.0f} TFLOP/s on random data")
    ceiling.update(mix_ceiling(dev))
    mix_tf = ceiling.get("probe_attention_tile_mix_random", {}).get("tflops")
    if mix_tf:
        log(f"[bench] attention instruction mix, registers only: {mix_tf:.0f} TFLOP/s on random data")

    achieved = f_attn / (attn_ms * 1e-3) / 1e12
    traffic = None
    if TRAFFIC_FILE.exists():
        try:
            traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                "traffic": traffic, "kernel": "attn_main_kernel",
                "flops_per_launch": f_attn,
                "gemm_ceiling_tflops": gemm_tf, "frac_of_gemm_ceiling": round(achieved / gemm_tf, 4)}
    if mix_tf:
        roofline.update({"mix_ceiling_tflops": mix_tf,
                         "frac_of_mix_ceiling": round(achieved / mix_tf, 4)})

    e2e = None
    if not args.no_e2e:
        del q, k, v, bias
        torch.cuda.empty_cache()
        e2e = e2e_latency(dev)
        q, k, v, bias = W.attn_inputs(m=274_800, n=68_700, seed=0, device=dev)

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline ...")
        src_c, dst_c = W.sim_inputs(m=75_000, n=25_000, seed=0, device=dev)
        cpu = cpu_baseline(src_c, dst_c, q, k, v, bias, args.cpu_budget)
        log(f"[bench] CPU baseline {cpu['value']} TFLOP/s on {cpu['cores']} threads")

    line = {
        "metric": "ms + TFLOP/s (% bf16 MFMA peak) for sim-argmax and biased attn, 200 frames",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": ("sim-argmax [75000x128]x[25000x128] + biased attention 16 heads "
                                "x 274800 queries x 68700 merged keys x d64 (200 frames x 1374 tokens)"),
                   "sm_scale": SM_SCALE, "bias": "log(count), bf16, [1,16,1,N]"},
        "kernels": kernels,
        "attention_floor": floor,
        "mfma_ceiling": ceiling,
        "e2e": e2e,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
