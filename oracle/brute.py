"""float64 numpy brute-force attention for tiny shapes — test infrastructure only.

Independent of torch's SDPA: scores, max-subtracted exponentials and their sum
are written out per (batch, head) in float64, so it can pin the fp32 oracle.
"""

from __future__ import annotations

import math

import numpy as np

__all__ = ["attention_fp64"]


def attention_fp64(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float | None = None):
    """q (B, Sq, H, D), k/v (B, Sk, H, D) -> out (B, Sq, H, D), lse (B, H, Sq)."""

    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Sq, H, D = q.shape
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    out = np.zeros((B, Sq, H, D))
    lse = np.full((B, H, Sq), -np.inf)
    if k.shape[1] == 0:
        return out, lse
    for b in range(B):
        for h in range(H):
            s = scale * (q[b, :, h, :] @ k[b, :, h, :].T)  # (Sq, Sk)
            m = s.max(axis=1, keepdims=True)
            e = np.exp(s - m)
            z = e.sum(axis=1, keepdims=True)
            out[b, :, h, :] = (e / z) @ v[b, :, h, :]
            lse[b, h, :] = (m + np.log(z))[:, 0]
    return out, lse
