"""Run-time numeric gate of the fused q/k prologue, for the install record.

The reference records, on the first attention block it runs, how far its
fused q RMSNorm + RoPE kernel is from the eager composition (the module's
``norm_q`` then Diffusers' rotate-half ``_apply_rotary_emb``), under
``runtime["gate"]["qknorm_partial_rope"]``
(src/h3_flash/runtime/kernels/transformer.py:174-190), with the metrics of
``_error_metrics`` (:16-29). :func:`gate_qknorm_rope` does the same for the
HIP prologue; the eager side is torch's own ops on the device.
"""

from __future__ import annotations

import torch
from torch.nn import functional

__all__ = ["error_metrics", "eager_qknorm_rope", "gate_qknorm_rope"]


def error_metrics(actual: torch.Tensor, reference: torch.Tensor) -> dict[str, float]:
    """max/mean absolute difference, relative L2 (against the reference's
    norm, clamped at 1e-12) and cosine similarity, in fp32: the quantities of
    ``_error_metrics`` (src/h3_flash/runtime/kernels/transformer.py:16-29)."""

    a = actual.float()
    r = reference.float()
    delta = (a - r).abs()
    return {
        "max_abs": float(delta.max()),
        "mean_abs": float(delta.mean()),
        "relative_l2": float(delta.norm() / r.norm().clamp_min(1e-12)),
        "cosine": float(functional.cosine_similarity(a.flatten(), r.flatten(), dim=0)),
    }


def eager_qknorm_rope(normed: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE of already-normalised ``normed`` (B, S, H, D) with
    (S, R) tables over its first R columns (columns past R pass through),
    computed in fp32 and rounded once to ``normed``'s dtype."""

    R = cos.shape[-1]
    x = normed.float()
    head, tail = x[..., :R], x[..., R:]
    half = R // 2
    rotated = torch.cat((-head[..., half:], head[..., :half]), dim=-1)
    c = cos.float()[None, :, None, :]
    s = sin.float()[None, :, None, :]
    return torch.cat((head * c + rotated * s, tail), dim=-1).to(normed.dtype)


def gate_qknorm_rope(
    attn, hidden_states: torch.Tensor, query: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor
) -> dict[str, float]:
    """Metrics of the fused prologue's query against the eager composition on
    the same projection: ``attn.norm_q`` on the (B, S, H, D) query projection,
    then rotate-half RoPE."""

    with torch.no_grad():
        if attn.fused_projections:
            raw = attn.to_qkv(hidden_states).chunk(3, dim=-1)[0]
        else:
            raw = attn.to_q(hidden_states)
        reference = eager_qknorm_rope(attn.norm_q(raw.unflatten(-1, (attn.heads, -1))), cos, sin)
        return error_metrics(query, reference)
