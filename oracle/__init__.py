"""CPU oracle of the dense H3 attention path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only to check results against it. The product
(``h3_flash_amd``) never calls it and has no CPU fallback.

Modules, each citing the reference lines it restates:

* ``attention`` — SDPA math reference with LSE (dense and varlen), sampled
  rows, and the log-sum-exp merge of partial results.
* ``brute`` — float64 restatement for tiny shapes.
* ``qknorm_rope`` — the fused q/k RMSNorm + RoPE prologue.
* ``projection`` — the projection feeding that prologue (fused GEMM epilogue).
* ``relayout`` — the packed-Ulysses pack / merge movements and the exchange.
* ``fusions`` — the DiT block's row fusions.
* ``metrics`` — the reference's error metrics and the path's tolerances.

Every function is pinned by a CPU test under ``tests/test_oracle*.py``
(brute force, closed forms, golden fixtures, planted mistakes). The
reference publishes no numeric vectors for this path and its kernels (FA4,
Triton) cannot run here, so nothing is checked against the reference's own
outputs.
"""
