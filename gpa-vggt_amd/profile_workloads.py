#!/usr/bin/env python3
"""Run each hot kernel a few times at its benchmark shape, for profilers.

    python3 gpa-vggt_amd/profile_workloads.py {sim|attn|merge|copy|all} [reps]

  sim    fused similarity-argmax, 75,000 x 25,000 x 128 (bf16)
  attn   biased attention, 16 heads x 274,800 queries x 68,700 keys x 64
  merge  deterministic K/V merge, [1,16,274800,64] fp32 rows into 66,845 slots
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
    if which not in ("sim", "attn", "merge", "copy", "all"):
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
    if which in ("merge", "all"):
        t, off, tok = W.merge_inputs(device=dev)
        for _ in range(reps):
            _native.merge_heads(t, off, tok, off.numel() - 1, True)
        torch.cuda.synchronize()
        print(f"merge [1,16,274800,64] f32 -> 66845 slots x {reps} done", flush=True)
        del t, off, tok
    if which in ("attn", "all"):
        q, k, v, b = W.attn_inputs(device=dev)
        for _ in range(reps):
            attention_keybias(q, k, v, b, 0.125)
        torch.cuda.synchronize()
        print(f"attn 16x274800x68700x64 x {reps} done", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
