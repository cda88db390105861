"""fp32 restatement of the DiT-block row fusions — test infrastructure only.

Follows the reference Triton kernels in src/h3_flash/runtime/kernels/fusions.py,
all arithmetic in fp32 and one rounding to the output dtype:

* ``rmsnorm_modulate_reference`` — ``_rmsnorm_modulate_kernel`` (:69-96):
  variance = sum(x^2) / C (:90), normed = x * rsqrt(variance + eps) (:91),
  out = normed * weight * (1 + scale[t]) + shift[t] (:95), t = index[row % n] (:88).
* ``residual_gate_rmsnorm_modulate_reference`` —
  ``_residual_gate_rmsnorm_modulate_kernel`` (:23-67): hidden = residual +
  gate[t] * branch (:50), stored (:51-55); the norm uses the fp32 hidden
  (:56-59); normed = hidden * rsqrt(var + eps) * weight, then
  * (1 + scale[t]) + shift[t] (:57-62).
* ``swiglu_reference`` — ``_swiglu_kernel`` (:98-123):
  out = value * (gate * sigmoid(gate)), value / gate the two halves of a row.

Table rows are clamped to the table, as the HIP kernels do.
"""

from __future__ import annotations

import torch

__all__ = [
    "residual_gate_rmsnorm_modulate_reference",
    "rmsnorm_modulate_reference",
    "swiglu_reference",
    "table_rows",
]


def table_rows(index: torch.Tensor, rows: int, n_table: int) -> torch.Tensor:
    """Table row of every token: index[row % len(index)], clamped to the table."""

    idx = index.reshape(-1).long().cpu()
    t = idx[torch.arange(rows) % idx.numel()]
    return t.clamp(0, n_table - 1)


def _norm(h: torch.Tensor, eps: float) -> torch.Tensor:
    variance = (h * h).sum(dim=-1, keepdim=True) / h.shape[-1]
    return h * torch.rsqrt(variance + eps)


def rmsnorm_modulate_reference(x, weight, scale, shift, index, eps, out_dtype=torch.bfloat16):
    C = x.shape[-1]
    h = x.reshape(-1, C).float().cpu()
    t = table_rows(index, h.shape[0], min(scale.shape[0], shift.shape[0]))
    out = _norm(h, eps) * weight.float().cpu() * (1.0 + scale.float().cpu()[t]) + shift.float().cpu()[t]
    out = out if out_dtype is None else out.to(out_dtype)
    return out.view(x.shape)


def residual_gate_rmsnorm_modulate_reference(
    residual, branch, gate, weight, scale, shift, index, eps, out_dtype=torch.bfloat16
):
    C = residual.shape[-1]
    r = residual.reshape(-1, C).float().cpu()
    b = branch.reshape(-1, C).float().cpu()
    t = table_rows(index, r.shape[0], min(gate.shape[0], scale.shape[0], shift.shape[0]))
    hidden = r + gate.float().cpu()[t] * b
    normed = _norm(hidden, eps) * weight.float().cpu()
    normed = normed * (1.0 + scale.float().cpu()[t]) + shift.float().cpu()[t]
    if out_dtype is not None:
        hidden, normed = hidden.to(out_dtype), normed.to(out_dtype)
    return hidden.view(residual.shape), normed.view(residual.shape)


def swiglu_reference(x, out_dtype=torch.bfloat16):
    C = x.shape[-1] // 2
    f = x.float().cpu()
    value, gate = f[..., :C], f[..., C:]
    out = value * (gate * torch.sigmoid(gate))
    return out if out_dtype is None else out.to(out_dtype)
