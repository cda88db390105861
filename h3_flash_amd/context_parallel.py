"""Context-parallel pieces of the dense path on MI355X (HIP, gfx950).

Diffusers' context-parallel template calls a forward op per key/value chunk
with ``return_lse=True`` and combines the partial results by their
log-sum-exp (the reference's FA4 forward op refuses ``return_lse``,
src/h3_flash/runtime/attention/dense_fa4.py:72-73; :func:`hip_forward_op`
returns it). This module supplies the combine step as one HIP launch, and a
single-device form of the ring schedule built from it.
"""

from __future__ import annotations

import ctypes
from typing import Sequence

import torch

from . import _ext
from .attention import flash_attn_func

__all__ = ["chunked_attention", "merge_attention"]


def _raise(lib: ctypes.CDLL, rc: int) -> None:
    if rc != _ext.H3A_OK:
        message = _ext.last_error(lib)
        if rc == _ext.H3A_EINVAL:
            raise ValueError(message)
        raise RuntimeError(message)


def _dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return _ext.H3A_DTYPE_BF16
    if dtype == torch.float32:
        return _ext.H3A_DTYPE_F32
    raise TypeError(f"partial outputs must be bfloat16 or float32, got {dtype}")


def merge_attention(
    outs: Sequence[torch.Tensor],
    lses: Sequence[torch.Tensor],
    *,
    out: torch.Tensor | None = None,
    lse: torch.Tensor | None = None,
    out_dtype: torch.dtype | None = None,
    lse_layout: str = "bhs",
) -> tuple[torch.Tensor, torch.Tensor]:
    """Combine partial attention results over disjoint key ranges.

    ``outs[i]``: (B, S, H, D) bf16 or fp32. ``lses[i]``: fp32, laid out as
    ``lse_layout`` says: ``"bhs"`` (B, H, S), as :func:`flash_attn_func`
    returns it, or ``"bsh"`` (B, S, H), as :func:`hip_forward_op` returns it
    for Diffusers' context-parallel template. The layout is an explicit
    argument because the two shapes coincide when S == H. Returns
    ``(out, lse)`` with ``lse = logsumexp_i(lses[i])`` in the same layout and
    ``out = sum_i exp(lses[i] - lse) * outs[i]``. ``out``/``lse`` may be
    given, and may be ``outs[0]``/``lses[0]`` (in place).
    """

    if lse_layout not in ("bhs", "bsh"):
        raise ValueError(f"lse_layout must be 'bhs' or 'bsh', got {lse_layout!r}")
    if lse_layout == "bsh":
        # (B, S, H) views are (B, H, S) tensors transposed; the launch takes
        # the (B, H, S) form (a transposed view of a contiguous (B, H, S)
        # tensor goes back without a copy).
        for o, l in zip(outs, lses):
            if l.dim() != 3 or tuple(l.shape) != (o.shape[0], o.shape[1], o.shape[2]):
                raise ValueError(f"'bsh' LSEs must be (B, S, H) = {tuple(o.shape[:3])}, got {tuple(l.shape)}")
        if lse is not None and (lse.dim() != 3 or tuple(lse.shape) != tuple(outs[0].shape[:3])):
            raise ValueError(f"lse must be (B, S, H) = {tuple(outs[0].shape[:3])} with lse_layout='bsh'")
        direct = lse is not None and lse.transpose(1, 2).stride(-1) == 1
        o, l = merge_attention(
            outs,
            [x.transpose(1, 2) for x in lses],
            out=out,
            lse=lse.transpose(1, 2) if direct else None,
            out_dtype=out_dtype,
        )
        if lse is not None and not direct:
            lse.copy_(l.transpose(1, 2))  # a caller's contiguous (B, S, H) buffer
            return o, lse
        return o, l.transpose(1, 2)
    n = len(outs)
    if n == 0 or n != len(lses):
        raise ValueError("merge_attention needs as many LSEs as partial outputs, at least one")
    if n > _ext.H3A_MERGE_MAX_PARTS:
        # Merge the first 16 in fp32, then that result with the rest (in fp32:
        # parts of one call share a dtype), so nothing is rounded twice.
        k = _ext.H3A_MERGE_MAX_PARTS
        head = merge_attention(outs[:k], lses[:k], out_dtype=torch.float32)
        # the output dtype as a call with 16 parts or fewer picks it
        final_dtype = out_dtype or (out.dtype if out is not None else outs[0].dtype)
        return merge_attention(
            [head[0], *(o.float() for o in outs[k:])], [head[1], *lses[k:]],
            out=out, lse=lse, out_dtype=final_dtype,
        )
    ref = outs[0]
    if ref.dim() != 4 or not ref.is_cuda:
        raise ValueError(f"partial outputs must be (B, S, H, D) device tensors, got {tuple(ref.shape)}")
    B, S, H, D = ref.shape
    dtype = ref.dtype
    strides = ref.stride()
    parts = []
    for o in outs:
        if o.shape != ref.shape or o.dtype != dtype or o.device != ref.device:
            raise ValueError("partial outputs must share shape, dtype and device")
        parts.append(o if o.stride() == strides and o.stride(-1) == 1 else o.contiguous())
    if any(p.stride() != parts[0].stride() for p in parts):
        parts = [p.contiguous() for p in parts]
    lparts = []
    for l in lses:
        if l.shape != (B, H, S) or l.dtype != torch.float32 or l.device != ref.device:
            raise ValueError(f"LSEs must be fp32 (B, H, S) = {(B, H, S)} on {ref.device}")
        lparts.append(l if l.stride(-1) == 1 else l.contiguous())
    if any(l.stride() != lparts[0].stride() for l in lparts):
        lparts = [l.contiguous() for l in lparts]
    out_dtype = out_dtype or (out.dtype if out is not None else dtype)
    if out is None:
        out = torch.empty((B, S, H, D), dtype=out_dtype, device=ref.device)
    elif out.shape != (B, S, H, D) or out.dtype != out_dtype or out.stride(-1) != 1 or out.device != ref.device:
        raise ValueError(f"out must be (B, S, H, D) in the requested dtype on {ref.device} with a contiguous last dim")
    if lse is None:
        lse = torch.empty((B, H, S), dtype=torch.float32, device=ref.device)
    elif lse.shape != (B, H, S) or lse.dtype != torch.float32 or lse.stride(-1) != 1 or lse.device != ref.device:
        raise ValueError(f"lse must be fp32 (B, H, S) on {ref.device} with a contiguous last dim")
    args = _ext.AttnMergeArgs()
    args.abi_version = _ext.ABI_VERSION
    args.n_parts = n
    for i, (o, l) in enumerate(zip(parts, lparts)):
        args.o_parts[i] = o.data_ptr()
        args.lse_parts[i] = l.data_ptr()
    args.part_dtype = _dtype_code(dtype)
    args.o, args.out_dtype, args.lse = out.data_ptr(), _dtype_code(out_dtype), lse.data_ptr()
    args.batch, args.heads, args.seqlen, args.head_dim = B, H, S, D
    args.part_o_stride[:] = (parts[0].stride(0), parts[0].stride(1), parts[0].stride(2))
    args.part_lse_stride[:] = (lparts[0].stride(0), lparts[0].stride(1))
    args.o_stride[:] = (out.stride(0), out.stride(1), out.stride(2))
    args.lse_stride[:] = (lse.stride(0), lse.stride(1))
    lib = _ext.load_library()
    with torch.cuda.device(ref.device):
        stream = ctypes.c_void_p(torch.cuda.current_stream(ref.device).cuda_stream)
        _raise(lib, lib.h3a_attn_merge(ctypes.byref(args), stream))
    return out, lse


def chunked_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    chunks: int,
    softmax_scale: float | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Attention of q over k/v split into ``chunks`` contiguous key ranges,
    one :func:`flash_attn_func` call per range, merged by LSE: the ring
    schedule of context parallelism run on one device. Equal to
    ``flash_attn_func(q, k, v)`` up to the rounding of the partial outputs."""

    Sk = k.shape[1]
    if chunks < 1 or chunks > Sk:
        raise ValueError(f"chunks must be in [1, {Sk}], got {chunks}")
    bounds = [Sk * i // chunks for i in range(chunks + 1)]
    outs, lses = [], []
    for a, b in zip(bounds[:-1], bounds[1:]):
        o, l = flash_attn_func(q, k[:, a:b], v[:, a:b], softmax_scale=softmax_scale)
        outs.append(o)
        lses.append(l)
    return merge_attention(outs, lses, out_dtype=q.dtype)
