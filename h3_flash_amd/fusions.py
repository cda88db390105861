"""Row-wise fusions of the MiniMax H3 DiT block on MI355X (HIP, gfx950).

Same function names, arguments and return values as the reference's Triton
wrappers (src/h3_flash/runtime/kernels/fusions.py):

* :func:`fused_rmsnorm_modulate` (fusions.py:194-215)
* :func:`fused_residual_gate_rmsnorm_modulate` (fusions.py:218-248)
* :func:`fused_swiglu` (fusions.py:251-265)
* :func:`fused_qknorm_rope` (fusions.py:268-293), from :mod:`h3_flash_amd.prologue`

Activations are bf16 (the dtype the H3 block runs in); weights and
modulation tables may be bf16 or fp32, table indices int32 or int64. Table
indices outside the table are clamped to it (the reference reads out of
bounds there). Every call is one HIP launch on the current stream.
"""

from __future__ import annotations

import ctypes

import torch

from . import _ext
from .prologue import fused_qknorm_rope

__all__ = [
    "fused_qknorm_rope",
    "fused_residual_gate_rmsnorm_modulate",
    "fused_rmsnorm_modulate",
    "fused_swiglu",
]


def _raise(lib: ctypes.CDLL, rc: int) -> None:
    if rc != _ext.H3A_OK:
        message = _ext.last_error(lib)
        if rc == _ext.H3A_EINVAL:
            raise ValueError(message)
        raise RuntimeError(message)


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _rows(x: torch.Tensor, name: str, columns: int) -> torch.Tensor:
    """(N, columns) bf16 device view with a contiguous last dimension."""

    if x.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {x.dtype}")
    if not x.is_cuda:
        raise RuntimeError(f"{name} must be on a ROCm device, got {x.device}")
    flat = x.reshape(-1, columns)
    return flat if flat.stride(-1) == 1 else flat.contiguous()


def _vector(t: torch.Tensor, columns: int, device: torch.device, name: str) -> torch.Tensor:
    if t.shape[-1] != columns or t.numel() != columns:
        raise ValueError(f"{name} must have {columns} elements, got shape {tuple(t.shape)}")
    t = t.reshape(columns).to(device)
    if t.dtype not in (torch.bfloat16, torch.float32):
        t = t.float()
    return t if t.is_contiguous() else t.contiguous()


def _tables(tables: list[torch.Tensor], columns: int, device: torch.device) -> list[torch.Tensor]:
    out = []
    for t in tables:
        if t.dim() != 2 or t.shape[1] != columns:
            raise ValueError(f"modulation tables must be (rows, {columns}), got {tuple(t.shape)}")
        out.append(t.to(device))
    dtype = torch.bfloat16 if all(t.dtype == torch.bfloat16 for t in out) else torch.float32
    out = [t.to(dtype) for t in out]
    # _row_addressable (fusions.py:190-191): the last dimension must be
    # contiguous; broadcast rows (a row stride under the row, e.g. expand())
    # are written out, since the launch takes one row stride per table
    return [t if t.stride(-1) == 1 and t.stride(0) >= columns else t.contiguous() for t in out]


def _index(index: torch.Tensor, device: torch.device) -> torch.Tensor:
    index = index.reshape(-1).to(device)
    if index.numel() == 0:
        raise ValueError("index must not be empty")
    if index.dtype not in (torch.int32, torch.int64):
        index = index.long()
    return index if index.is_contiguous() else index.contiguous()


def _fill_common(args, weight, tables, index, eps) -> None:
    args.abi_version = _ext.ABI_VERSION
    args.weight = weight.data_ptr()
    args.w_dtype = _ext.H3A_DTYPE_F32 if weight.dtype == torch.float32 else _ext.H3A_DTYPE_BF16
    args.table_dtype = _ext.H3A_DTYPE_F32 if tables[0].dtype == torch.float32 else _ext.H3A_DTYPE_BF16
    args.table_rows = min(t.shape[0] for t in tables)
    args.index = index.data_ptr()
    args.index_dtype = _ext.H3A_DTYPE_I64 if index.dtype == torch.int64 else _ext.H3A_DTYPE_I32
    args.n_index = index.numel()
    args.eps = float(eps)


def fused_rmsnorm_modulate(x, weight, scale, shift, index, eps):
    """RMSNorm over the last dimension, times ``weight``, then
    ``* (1 + scale[t]) + shift[t]`` with ``t = index[row % len(index)]``."""

    columns = x.shape[-1]
    flat = _rows(x, "x", columns)
    weight = _vector(weight, columns, x.device, "weight")
    scale, shift = _tables([scale, shift], columns, x.device)
    index = _index(index, x.device)
    output = torch.empty((flat.shape[0], columns), dtype=x.dtype, device=x.device)
    args = _ext.RmsnormModulateArgs()
    _fill_common(args, weight, [scale, shift], index, eps)
    args.x, args.out = flat.data_ptr(), output.data_ptr()
    args.scale, args.shift = scale.data_ptr(), shift.data_ptr()
    args.scale_stride, args.shift_stride = scale.stride(0), shift.stride(0)
    args.rows, args.cols = flat.shape[0], columns
    args.x_stride, args.out_stride = flat.stride(0), output.stride(0)
    lib = _ext.load_library()
    with torch.cuda.device(x.device):
        _raise(lib, lib.h3a_rmsnorm_modulate(ctypes.byref(args), _stream(x.device)))
    return output.view(x.shape)


def fused_residual_gate_rmsnorm_modulate(residual, branch, gate, weight, scale, shift, index, eps):
    """``hidden = residual + gate[t] * branch``, then RMSNorm(hidden) * weight
    * (1 + scale[t]) + shift[t]; returns ``(hidden, normed)``."""

    columns = residual.shape[-1]
    if branch.shape != residual.shape:
        raise ValueError(f"residual {tuple(residual.shape)} and branch {tuple(branch.shape)} differ")
    residual_flat = _rows(residual, "residual", columns)
    branch_flat = _rows(branch, "branch", columns)
    if branch.device != residual.device:
        raise ValueError(f"residual and branch must be on one device, got {residual.device} and {branch.device}")
    weight = _vector(weight, columns, residual.device, "weight")
    gate, scale, shift = _tables([gate, scale, shift], columns, residual.device)
    index = _index(index, residual.device)
    hidden = torch.empty((residual_flat.shape[0], columns), dtype=residual.dtype, device=residual.device)
    normed = torch.empty_like(hidden)
    args = _ext.ResidualGateRmsnormModulateArgs()
    _fill_common(args, weight, [gate, scale, shift], index, eps)
    args.residual, args.branch = residual_flat.data_ptr(), branch_flat.data_ptr()
    args.hidden_out, args.normed_out = hidden.data_ptr(), normed.data_ptr()
    args.gate, args.scale, args.shift = gate.data_ptr(), scale.data_ptr(), shift.data_ptr()
    args.gate_stride, args.scale_stride, args.shift_stride = gate.stride(0), scale.stride(0), shift.stride(0)
    args.rows, args.cols = residual_flat.shape[0], columns
    args.residual_stride, args.branch_stride = residual_flat.stride(0), branch_flat.stride(0)
    args.hidden_stride, args.normed_stride = hidden.stride(0), normed.stride(0)
    lib = _ext.load_library()
    with torch.cuda.device(residual.device):
        _raise(lib, lib.h3a_residual_gate_rmsnorm_modulate(ctypes.byref(args), _stream(residual.device)))
    return hidden.view(residual.shape), normed.view(residual.shape)


def fused_swiglu(x):
    """``value * silu(gate)`` with ``value, gate = x.chunk(2, -1)``."""

    if x.shape[-1] % 2:
        raise ValueError(f"swiglu needs an even last dimension, got {x.shape[-1]}")
    columns = x.shape[-1] // 2
    flat = _rows(x, "x", x.shape[-1])
    output = torch.empty((flat.shape[0], columns), dtype=x.dtype, device=x.device)
    args = _ext.SwigluArgs()
    args.abi_version = _ext.ABI_VERSION
    args.x, args.out = flat.data_ptr(), output.data_ptr()
    args.rows, args.cols = flat.shape[0], columns
    args.x_stride, args.out_stride = flat.stride(0), output.stride(0)
    lib = _ext.load_library()
    with torch.cuda.device(x.device):
        _raise(lib, lib.h3a_swiglu(ctypes.byref(args), _stream(x.device)))
    return output.view(*x.shape[:-1], columns)
