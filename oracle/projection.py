"""fp32 restatement of the attention block's projection step with the q/k
RMSNorm + RoPE applied to the projection's fp32 result — test
infrastructure only.

The reference computes, per token row of ``hidden_states``:

* the projection ``x @ W^T + b`` of ``attn.to_qkv`` / ``to_q`` / ``to_k`` /
  ``to_v`` (nn.Linear; src/h3_flash/runtime/attention/dense_fa4.py:123-128,
  src/h3_flash/runtime/kernels/transformer.py:146-152), split into heads of
  D (:129-131, :153-154);
* for q and k, ``fused_qknorm_rope(x, norm.weight, cos, sin, norm.eps)``
  (transformer.py:160-173; src/h3_flash/runtime/kernels/fusions.py:126-175,
  268-293), restated in :func:`oracle.qknorm_rope.qknorm_rope_reference`.

The reference rounds the projection to bf16 (the linear's output dtype)
before the norm; ``round_projection=True``, the default, follows that order,
as the fused launch does. ``round_projection=False`` feeds the fp32 product
straight into the norm (one bf16 rounding of q and k, at the end), so tests
can bound the difference between the two orders.
"""

from __future__ import annotations

import torch

from .qknorm_rope import qknorm_rope_reference

__all__ = ["projection_reference"]


def projection_reference(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    norm_weight: torch.Tensor | None = None,
    eps: float = 1e-6,
    cos: torch.Tensor | None = None,
    sin: torch.Tensor | None = None,
    seqlen: int | None = None,
    head_dim: int = 128,
    round_projection: bool = True,
) -> torch.Tensor:
    """(m, k) x (n, k) -> (m, n) bf16.

    Without ``norm_weight``: ``bf16(x @ W^T + b)`` from an fp32 product.
    With it: each head of ``head_dim`` features of the product (rounded to
    bf16 first when ``round_projection``) is normalised, weighted and
    rotated in fp32 (tables ``cos``/``sin`` of ``seqlen`` rows, token row
    ``i`` using row ``i % seqlen``; no tables: the norm alone), then rounded
    to bf16.
    """

    xf = x.detach().to("cpu", torch.float32)
    wf = weight.detach().to("cpu", torch.float32)
    acc = xf @ wf.T
    if bias is not None:
        acc = acc + bias.detach().to("cpu", torch.float32)
    if round_projection:
        acc = acc.to(torch.bfloat16).float()
    if norm_weight is None:
        return acc.to(torch.bfloat16)
    m, n = acc.shape
    heads = n // head_dim
    if cos is None:
        cos = torch.ones((1, 0))
        sin = torch.zeros((1, 0))
        seqlen = 1
    seqlen = seqlen if seqlen is not None else m
    rows = torch.arange(m) % seqlen
    c = cos.detach().to("cpu", torch.float32)[rows]
    s = sin.detach().to("cpu", torch.float32)[rows]
    # one "batch" of m tokens whose table rows are gathered per token
    out = qknorm_rope_reference(acc.view(1, m, heads, head_dim), norm_weight, c, s, eps)
    return out.view(m, n)
