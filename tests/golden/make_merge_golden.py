"""Write tests/golden/merge_golden.npz from the reference's own merge code.

Runs `token_merge_bipartite2d` of noheat61/GPA-VGGT (merging/merge.py, read
from /root/reference) on the CPU, where it takes its torch path
(`fast_similarity_chunks`), on small seeded inputs, and stores inputs and
outputs as plain arrays.  The reference itself never travels: only these
vectors are committed.  What the fixture pins and the invariants do not:
the dst-window layout and draw order (merge.py:119-163), the [unmerged | dst]
slot layout, and the assignment of every merged source token.

Each case records, per output slot, the number of tokens behind it
(`merge.size` and merge(ones, "sum")), the smallest and largest input token
position merged into it (merge(pos, "amin"/"amax")), and merge.heads(t,
"mean") of a float64 tensor.

    python tests/golden/make_merge_golden.py      # (re)writes the .npz
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

REFERENCE = Path("/root/reference")
OUT = Path(__file__).resolve().parent / "merge_golden.npz"

# name, frames, w, h, sx, sy, num_special, C, metric_dim, r, no_rand, seed
CASES = [
    ("all_merged", 4, 6, 6, 2, 2, 5, 48, 16, 10_000, False, 0),
    ("partial", 4, 6, 6, 2, 2, 5, 48, 16, 12, False, 1),
    ("no_rand", 3, 6, 6, 2, 2, 5, 48, 16, 10_000, True, 2),
    ("odd_grid_fulldim", 3, 7, 5, 2, 2, 5, 32, 0, 15, False, 3),
    ("grid3", 3, 7, 7, 3, 3, 1, 40, 24, 30, False, 4),
]
H, D = 2, 8


def main() -> int:
    sys.path.insert(0, str(REFERENCE))
    from merging.merge import token_merge_bipartite2d  # the reference implementation

    arrays = {}
    names = []
    for name, frames, w, h, sx, sy, ns, c, mdim, r, no_rand, seed in CASES:
        n = frames * (w * h + ns)
        g = torch.Generator().manual_seed(1000 + seed)
        metric = torch.randn(1, n, c, generator=g, dtype=torch.float32)
        t = torch.randn(1, H, n, D, generator=g, dtype=torch.float64)
        gen = torch.Generator().manual_seed(33)
        m = token_merge_bipartite2d(metric, w, h, sx, sy, r, no_rand, gen,
                                    metric_dim=mdim, num_special=ns)
        pos = torch.arange(n, dtype=torch.float64).view(1, n, 1)
        ones = torch.ones(1, n, 1, dtype=torch.float64)
        arrays[f"{name}/params"] = np.array([frames, w, h, sx, sy, ns, c, mdim, r, int(no_rand), seed])
        arrays[f"{name}/metric"] = metric.numpy()
        arrays[f"{name}/t"] = t.numpy()
        arrays[f"{name}/size"] = m.size.numpy()
        arrays[f"{name}/count"] = m(ones, "sum")[0, :, 0].numpy()
        arrays[f"{name}/pos_min"] = m(pos, "amin")[0, :, 0].numpy()
        arrays[f"{name}/pos_max"] = m(pos, "amax")[0, :, 0].numpy()
        arrays[f"{name}/heads_mean"] = m.heads(t, "mean").numpy()
        names.append(name)
    arrays["cases"] = np.array(names)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(names)} cases)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
