"""CPU oracle for the GPA-VGGT merging hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference's PyTorch path for the two
kernels and their caller (noheat61/GPA-VGGT):

  similarity.py  fast_similarity_chunks        merging/merge.py:13-36
                 fp64 brute-force sim-argmax   (pins the above)
  attention.py   SDPA with a per-key bias      vggt/layers/attention.py:259-276
                 + the attention_keybias dtype contract
                                               merging/fused_attention.py:139-160
                 log2 LSE                      merging/fused_attention.py:123-127
                 LSE split combine             vggt/layers/attention.py:166-176
                 fp64 closed form              (pins the above)
  merge.py       token_merge_bipartite2d       merging/merge.py:39-256
                 fp64 brute-force K/V mean     (pins merge.heads)

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import it, and only as the reference the results are
compared against or as the timed CPU baseline.
The product (`gpa-vggt_amd/merging`) never imports it and has no CPU path.

Every function here is pinned by a check in `tests/test_oracle_*.py`
(closed forms, invariants, brute force, or fixtures written by running the
reference's own Python on the CPU, `tests/golden/`).
"""
