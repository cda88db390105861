"""CPU oracle of the dense H3 attention path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker (or, for the baseline,
as the timed reference CPU path). The product (``h3_flash_amd``) never calls
it and has no CPU fallback.

Contents and what each follows in the reference repo:

* ``attention.sdpa_reference`` — torch SDPA math backend in fp32 on BHSD
  transposes of BSHD inputs, exactly the reference's call form
  (benchmarks/benchmark_dense_fa4.py:70-77, packed_ulysses.py:202-209),
  chunked over query rows, plus LSE = logsumexp(scale * q k^T) in natural
  log; block-diagonal per segment for packed varlen inputs.
* ``brute.attention_fp64`` — independent float64 numpy restatement
  (max-subtracted exp / sum) for tiny shapes, used to pin the former.
* ``qknorm_rope.qknorm_rope_reference`` — fp32 restatement of the Triton
  ``_qknorm_partial_rope_kernel`` (src/h3_flash/runtime/kernels/fusions.py:126-175).
* ``attention.merge_reference`` — fp32 log-sum-exp combine of partial
  attention results over disjoint key ranges (the context-parallel merge).
* ``relayout`` — the packed-Ulysses pack / merge movements in two forms, the
  permute form of src/h3_flash/runtime/parallel/relayout.py:81-94,138-142 and
  the index arithmetic of its Triton kernels (:28-49, :56-67), plus the
  all-to-all's effect on the buffers of every rank.
* ``fusions`` — fp32 restatements of the Triton row fusions
  (src/h3_flash/runtime/kernels/fusions.py:23-123).
* ``metrics.error_metrics`` — max_abs / mean_abs / relative_l2 / cosine of
  src/h3_flash/runtime/kernels/transformer.py:16-29 and
  benchmarks/benchmark_dense_fa4.py:92-99.

How each function is pinned (the checks live in tests/test_oracle.py):

* sdpa_reference: against the float64 brute force, the golden fixtures in
  tests/golden/, and closed forms (single key -> v; equal keys -> mean(v) and
  LSE = ln S + scale q.k; key/value permutation invariance; scale identity;
  varlen = concatenation of per-segment dense results; row sampling = rows of
  the full result). Planted mistakes in the oracle fail these checks.
* attention_fp64: closed forms above, and softmax rows summing to 1.
* merge_reference: merging the oracle's attention over key chunks equals
  attention over all keys; empty parts and part order change nothing
  (tests/test_oracle_merge.py).
* relayout: the two forms agree on every shape tried, the simulated exchange
  reproduces the head shards, planted index mistakes fail
  (tests/test_oracle_relayout.py).
* fusions: against torch's rms_norm and silu, the reference's eager
  formulas (benchmarks/benchmark_transformer_fusions.py:76-105) and closed
  forms; planted mistakes fail (tests/test_oracle_fusions.py).
* qknorm_rope_reference: against torch.nn.functional.rms_norm (R = 0), the
  complex-multiplication form of rotate-half RoPE, rotation inversion and
  pair-norm preservation, and the golden fixtures.

Parity note: the reference publishes no numeric vectors for this path and
its kernels (FA4, Triton) cannot run here, so no function is checked
against the reference's own outputs; the checks above pin the restatements.
"""
