"""Error metrics of the reference's numeric gates — test infrastructure only.

Same quantities as ``_error_metrics`` (src/h3_flash/runtime/kernels/transformer.py:16-29)
and the numerical block of benchmarks/benchmark_dense_fa4.py:92-99, computed in
fp32 (float64 accumulation for the norms).
"""

from __future__ import annotations

import torch
from torch.nn import functional

__all__ = ["error_metrics", "ATTN_MAX_ABS", "ATTN_MEAN_ABS", "LSE_MAX_ABS"]

# Tolerances of the path against an fp32-accumulated SDPA-math reference.
ATTN_MAX_ABS = 2e-2
ATTN_MEAN_ABS = 2e-3
LSE_MAX_ABS = 1e-3


def error_metrics(actual: torch.Tensor, reference: torch.Tensor) -> dict[str, float]:
    a = actual.detach().to("cpu", torch.float64)
    r = reference.detach().to("cpu", torch.float64)
    delta = (a - r).abs()
    finite = bool(torch.isfinite(a).all())
    return {
        "max_abs": float(delta.max()) if delta.numel() else 0.0,
        "mean_abs": float(delta.mean()) if delta.numel() else 0.0,
        "relative_l2": float(delta.norm() / r.norm().clamp_min(1e-12)),
        "cosine": float(functional.cosine_similarity(a.flatten(), r.flatten(), dim=0)) if a.numel() else 1.0,
        "finite": finite,
    }
