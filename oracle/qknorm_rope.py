"""fp32 restatement of the reference's fused q/k RMSNorm + partial RoPE —
test infrastructure only.

Follows ``_qknorm_partial_rope_kernel`` (src/h3_flash/runtime/kernels/fusions.py:126-175)
and its wrapper ``fused_qknorm_rope`` (:268-293), per (token, head) row of D:

* value = x in fp32; variance = sum(value^2) / D                  (:145-146)
* normed = value * rsqrt(variance + eps) * weight                   (:147-148)
* partner = c + R/2 for c < R/2, c - R/2 for R/2 <= c < R            (:149-151)
* rotated = -normed[partner] (first half), +normed[partner] (second) (:152-159)
* out = normed * cos[s, c] + rotated * sin[s, c] for c < R, else normed (:160-170)
* stored once in x's dtype                                          (:171-175)

with s the token's sequence index (:141) and cos/sin fp32 (S, R) tables.
"""

from __future__ import annotations

import torch

__all__ = ["qknorm_rope_reference"]


def qknorm_rope_reference(
    x: torch.Tensor,
    weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    eps: float,
    out_dtype: torch.dtype | None = torch.bfloat16,
) -> torch.Tensor:
    """x (B, S, H, D) -> (B, S, H, D); fp32 if ``out_dtype`` is None."""

    B, S, H, D = x.shape
    R = cos.shape[-1]
    if R > D or R % 2:
        raise ValueError(
            "fused qknorm+rope requires an even rotary dimension no wider "
            f"than the head, got rotary_dim={R}, head_dim={D}"
        )
    value = x.detach().to("cpu", torch.float32)
    w = weight.detach().to("cpu", torch.float32)
    variance = (value * value).sum(dim=-1, keepdim=True) / D
    normed = value * torch.rsqrt(variance + eps) * w
    out = normed.clone()
    if R > 0:
        half = R // 2
        c = cos.detach().to("cpu", torch.float32).view(1, S, 1, R)
        s = sin.detach().to("cpu", torch.float32).view(1, S, 1, R)
        rotated = torch.cat((-normed[..., half:R], normed[..., :half]), dim=-1)
        out[..., :R] = normed[..., :R] * c + rotated * s
    return out if out_dtype is None else out.to(out_dtype)
