"""Fused q/k RMSNorm + rotate-half RoPE in front of attention (HIP, gfx950).

``fused_qknorm_rope(x, weight, cos, sin, eps)`` keeps the signature, argument
meaning and ValueError of the reference's Triton wrapper
(src/h3_flash/runtime/kernels/fusions.py:268-293). ``fused_qk_norm_rope``
transforms q and k in a single launch, which is how the attention processor
calls it: the reference issues one launch per tensor
(src/h3_flash/runtime/kernels/transformer.py:160-173).
"""

from __future__ import annotations

import ctypes

import torch

from . import _ext

__all__ = ["fused_qknorm_rope", "fused_qk_norm_rope"]


def _check_rotary(head_dim: int, rotary_dim: int) -> None:
    if rotary_dim > head_dim or rotary_dim % 2:
        raise ValueError(
            "fused qknorm+rope requires an even rotary dimension no wider "
            f"than the head, got rotary_dim={rotary_dim}, head_dim={head_dim}"
        )


def _operand(x: torch.Tensor, name: str) -> torch.Tensor:
    if x.dim() != 4:
        raise ValueError(f"{name} must be 4-D (batch, seq, heads, head_dim), got {tuple(x.shape)}")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {x.dtype}")
    if x.device.type != "cuda":
        raise RuntimeError(f"{name} must be on a ROCm device, got {x.device}")
    ok = x.stride(-1) == 1 and all(s % 8 == 0 for s in x.stride()[:3]) and x.data_ptr() % 16 == 0
    return x if ok else x.contiguous()


def _weight(w: torch.Tensor, head_dim: int, device: torch.device) -> torch.Tensor:
    if w.shape != (head_dim,):
        raise ValueError(f"norm weight must have shape ({head_dim},), got {tuple(w.shape)}")
    if w.dtype not in (torch.bfloat16, torch.float32):
        w = w.float()
    w = w.to(device)
    return w if (w.is_contiguous() and w.data_ptr() % 16 == 0) else w.contiguous().clone()


def _table(t: torch.Tensor, seqlen: int, device: torch.device) -> torch.Tensor:
    if t.dim() != 2 or t.shape[0] != seqlen:
        raise ValueError(f"cos/sin tables must be (seq={seqlen}, rotary_dim), got {tuple(t.shape)}")
    t = t.to(device=device, dtype=torch.float32)
    # broadcast rows (a row stride under the row, e.g. expand()) are written
    # out: the launch reads row s at s * table_stride with table_stride >= R
    return t if t.stride(-1) == 1 and t.stride(0) >= t.shape[-1] else t.contiguous()


def _tables(cos: torch.Tensor, sin: torch.Tensor, seqlen: int, device: torch.device):
    """fp32 device cos/sin with one row stride between them (the launch
    takes a single table stride)."""
    cos, sin = _table(cos, seqlen, device), _table(sin, seqlen, device)
    if cos.stride(0) != sin.stride(0):
        cos, sin = cos.contiguous(), sin.contiguous()
    return cos, sin


def _launch(q, k, wq, wk, cos, sin, eps_q, eps_k, out_q, out_k) -> None:
    B, S, H, D = q.shape
    R = cos.shape[-1]
    args = _ext.QkNormRopeArgs()
    args.abi_version = _ext.ABI_VERSION
    args.xq, args.yq, args.wq = q.data_ptr(), out_q.data_ptr(), wq.data_ptr()
    if k is not None:
        args.xk, args.yk, args.wk = k.data_ptr(), out_k.data_ptr(), wk.data_ptr()
        args.xk_stride[:] = k.stride()[:3]
        args.yk_stride[:] = out_k.stride()[:3]
    args.w_dtype = _ext.H3A_DTYPE_F32 if wq.dtype == torch.float32 else _ext.H3A_DTYPE_BF16
    args.cos, args.sin = cos.data_ptr(), sin.data_ptr()
    args.table_stride = cos.stride(0)
    args.batch, args.seqlen, args.heads, args.head_dim, args.rotary_dim = B, S, H, D, R
    args.xq_stride[:] = q.stride()[:3]
    args.yq_stride[:] = out_q.stride()[:3]
    args.eps_q, args.eps_k = float(eps_q), float(eps_k)
    lib = _ext.load_library()
    stream = torch.cuda.current_stream(q.device).cuda_stream
    rc = lib.h3a_qknorm_rope(ctypes.byref(args), ctypes.c_void_p(stream))
    if rc != _ext.H3A_OK:
        message = _ext.last_error(lib)
        if rc == _ext.H3A_EINVAL:
            raise ValueError(message)
        raise RuntimeError(message)


def fused_qknorm_rope(
    x: torch.Tensor, weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, eps: float
) -> torch.Tensor:
    """RMSNorm over the head dim, times ``weight``, then rotate-half RoPE on
    the first ``cos.shape[-1]`` columns; returns a new (B, S, H, D) bf16 tensor.
    """

    B, S, H, D = x.shape
    _check_rotary(D, cos.shape[-1])
    x = _operand(x, "x")
    if sin.shape != cos.shape:
        raise ValueError("cos and sin must have the same shape")
    w = _weight(weight, D, x.device)
    cos, sin = _tables(cos, sin, S, x.device)
    out = torch.empty((B, S, H, D), dtype=x.dtype, device=x.device)
    _launch(x, None, w, None, cos, sin, eps, eps, out, None)
    return out


def fused_qk_norm_rope(
    q: torch.Tensor,
    k: torch.Tensor,
    weight_q: torch.Tensor,
    weight_k: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    eps_q: float,
    eps_k: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``fused_qknorm_rope`` on q and k in one launch (shared cos/sin row reads)."""

    if q.shape != k.shape:
        raise ValueError(f"q and k shapes differ: {tuple(q.shape)} vs {tuple(k.shape)}")
    B, S, H, D = q.shape
    _check_rotary(D, cos.shape[-1])
    if sin.shape != cos.shape:
        raise ValueError("cos and sin must have the same shape")
    q = _operand(q, "q")
    k = _operand(k, "k")
    if k.device != q.device:
        raise ValueError(f"q and k must be on one device, got {q.device} and {k.device}")
    wq = _weight(weight_q, D, q.device)
    wk = _weight(weight_k, D, q.device)
    if wq.dtype != wk.dtype:
        wq, wk = wq.float(), wk.float()
    cos, sin = _tables(cos, sin, S, q.device)
    out_q = torch.empty((B, S, H, D), dtype=q.dtype, device=q.device)
    out_k = torch.empty((B, S, H, D), dtype=k.dtype, device=k.device)
    _launch(q, k, wq, wk, cos, sin, eps_q, eps_k, out_q, out_k)
    return out_q, out_k
