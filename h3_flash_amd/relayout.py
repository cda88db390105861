"""Packed-Ulysses relayouts on MI355X (HIP, gfx950): bit-exact data movement.

The functions keep the names, argument meaning and errors of the reference's
relayout module (src/h3_flash/runtime/parallel/relayout.py):

* :func:`pack_qkv_destination_major` (relayout.py:97-130) — q, k, v of shape
  (rows, heads, head_dim) into the destination-major send buffer
  (world, rows, heads/world, 3*head_dim) of the QKV all-to-all
  (src/h3_flash/runtime/parallel/packed_ulysses.py:85-108).
* :func:`merge_heads` (relayout.py:133-159) — (world, rows, hl, head_dim)
  after the output all-to-all into (rows, world*hl, head_dim)
  (packed_ulysses.py:111-128).
* :func:`can_pack_qkv` (relayout.py:70-78).

Two MI355X additions sit on the same boundary:

* :func:`qknorm_rope_pack_qkv` — the per-rank steps of packed_ulysses.py:177-200
  (RMSNorm + RoPE of q and k, then the pack) as one launch that writes the
  send buffer directly, so normalised q and k never round-trip through HBM.
* :func:`packed_qkv_attention` — the attention of packed_ulysses.py:201-209 on
  the exchanged buffer, read in place through strided q/k/v views.

The collectives themselves are not part of this single-GPU build.
"""

from __future__ import annotations

import ctypes

import torch

from . import _ext
from .attention import flash_attn_func
from .prologue import _check_rotary, _tables, _weight

__all__ = [
    "can_pack_qkv",
    "merge_heads",
    "pack_qkv_destination_major",
    "packed_qkv_attention",
    "qknorm_rope_pack_qkv",
]


def _raise(lib: ctypes.CDLL, rc: int) -> None:
    if rc != _ext.H3A_OK:
        message = _ext.last_error(lib)
        if rc == _ext.H3A_EINVAL:
            raise ValueError(message)
        raise RuntimeError(message)


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def can_pack_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
    """Whether :func:`pack_qkv_destination_major` takes these tensors
    (same predicate as relayout.py:70-78)."""

    return (
        q.is_cuda
        and q.ndim == 3
        and q.shape == k.shape == v.shape
        and q.dtype == k.dtype == v.dtype
        and q.device == k.device == v.device
        and q.stride(-1) == k.stride(-1) == v.stride(-1) == 1
    )


def pack_qkv_destination_major(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, world: int
) -> torch.Tensor:
    """Move q, k, v into destination-major order without arithmetic.

    Returns ``out`` of shape (world, rows, heads // world, 3 * head_dim) with
    ``out[d, r, j] = cat(q[r, d*hl + j], k[r, d*hl + j], v[r, d*hl + j])``.
    Raises ValueError when heads is not a multiple of ``world``.
    """

    if not can_pack_qkv(q, k, v):
        raise ValueError(
            "pack_qkv_destination_major needs three device tensors of one shape (rows, heads, head_dim), "
            "one dtype and a contiguous last dimension"
        )
    rows, heads, head_dim = q.shape
    if world <= 0 or heads % world:
        raise ValueError(f"heads ({heads}) must divide Ulysses degree ({world})")
    heads_local = heads // world
    out = torch.empty((world, rows, heads_local, 3 * head_dim), dtype=q.dtype, device=q.device)
    if out.numel() == 0:
        return out
    args = _ext.PackQkvArgs()
    args.abi_version = _ext.ABI_VERSION
    args.q, args.k, args.v, args.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    args.elem_bytes = q.element_size()
    args.rows, args.heads, args.head_dim, args.world = rows, heads, head_dim, world
    args.q_stride[:] = q.stride()[:2]
    args.k_stride[:] = k.stride()[:2]
    args.v_stride[:] = v.stride()[:2]
    lib = _ext.load_library()
    with torch.cuda.device(q.device):
        _raise(lib, lib.h3a_pack_qkv(ctypes.byref(args), _stream(q.device)))
    return out


def merge_heads(x: torch.Tensor) -> torch.Tensor:
    """Transpose source-rank and row dimensions without changing any value:
    (world, rows, hl, head_dim) -> (rows, world * hl, head_dim)."""

    if x.ndim != 4:
        raise ValueError(f"merge_heads expects (world, rows, heads_local, head_dim), got {tuple(x.shape)}")
    if not x.is_cuda:
        raise RuntimeError(f"merge_heads needs a ROCm device tensor, got {x.device}")
    world, rows, heads_local, head_dim = x.shape
    inner = heads_local * head_dim
    if x.stride(3) != 1 or (heads_local > 1 and x.stride(2) != head_dim):
        x = x.contiguous()  # the (heads_local, head_dim) block must be contiguous
    out = torch.empty((rows, world, heads_local, head_dim), dtype=x.dtype, device=x.device)
    if out.numel() == 0:
        return out.reshape(rows, world * heads_local, head_dim)
    args = _ext.MergeHeadsArgs()
    args.abi_version = _ext.ABI_VERSION
    args.x, args.out = x.data_ptr(), out.data_ptr()
    args.elem_bytes = x.element_size()
    args.world, args.rows, args.inner = world, rows, inner
    args.x_stride[:] = (x.stride(0), x.stride(1))
    lib = _ext.load_library()
    with torch.cuda.device(x.device):
        _raise(lib, lib.h3a_merge_heads(ctypes.byref(args), _stream(x.device)))
    return out.reshape(rows, world * heads_local, head_dim)


def _rows_operand(x: torch.Tensor, name: str) -> torch.Tensor:
    if x.dim() != 3:
        raise ValueError(f"{name} must be (rows, heads, head_dim), got {tuple(x.shape)}")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {x.dtype}")
    if not x.is_cuda:
        raise RuntimeError(f"{name} must be on a ROCm device, got {x.device}")
    ok = x.stride(-1) == 1 and x.stride(0) % 8 == 0 and x.stride(1) % 8 == 0 and x.data_ptr() % 16 == 0
    return x if ok else x.contiguous()


def qknorm_rope_pack_qkv(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    weight_q: torch.Tensor,
    weight_k: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    eps_q: float,
    eps_k: float,
    world: int,
) -> torch.Tensor:
    """RMSNorm + rotate-half RoPE of q and k (as :func:`fused_qknorm_rope`)
    and the destination-major pack of (q, k, v), in one launch.

    q, k, v: (rows, heads, head_dim) bf16; cos/sin: fp32 (rows, R). The
    result is bit-identical to ``pack_qkv_destination_major(fused_qknorm_rope(q),
    fused_qknorm_rope(k), v, world)``, for every even rotary width R <= D
    (the reference's prologue takes any, fusions.py:268-275; tables built as
    _official_rope builds them have R = 6 * len(inv_freq), e.g. 126).
    """

    if not (q.shape == k.shape == v.shape):
        raise ValueError(f"q, k, v shapes differ: {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    rows, heads, head_dim = q.shape
    R = cos.shape[-1]
    _check_rotary(head_dim, R)
    if sin.shape != cos.shape:
        raise ValueError("cos and sin must have the same shape")
    if world <= 0 or heads % world:
        raise ValueError(f"heads ({heads}) must divide Ulysses degree ({world})")
    q, k, v = _rows_operand(q, "q"), _rows_operand(k, "k"), _rows_operand(v, "v")
    wq = _weight(weight_q, head_dim, q.device)
    wk = _weight(weight_k, head_dim, q.device)
    if wq.dtype != wk.dtype:
        wq, wk = wq.float(), wk.float()
    cos, sin = _tables(cos, sin, rows, q.device)
    out = torch.empty((world, rows, heads // world, 3 * head_dim), dtype=q.dtype, device=q.device)
    if out.numel() == 0:
        return out
    args = _ext.QkNormRopePackArgs()
    args.abi_version = _ext.ABI_VERSION
    args.q, args.k, args.v, args.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    args.wq, args.wk = wq.data_ptr(), wk.data_ptr()
    args.w_dtype = _ext.H3A_DTYPE_F32 if wq.dtype == torch.float32 else _ext.H3A_DTYPE_BF16
    args.cos, args.sin, args.table_stride = cos.data_ptr(), sin.data_ptr(), cos.stride(0)
    args.rows, args.heads, args.head_dim, args.rotary_dim, args.world = rows, heads, head_dim, R, world
    args.q_stride[:] = q.stride()[:2]
    args.k_stride[:] = k.stride()[:2]
    args.v_stride[:] = v.stride()[:2]
    args.eps_q, args.eps_k = float(eps_q), float(eps_k)
    lib = _ext.load_library()
    with torch.cuda.device(q.device):
        _raise(lib, lib.h3a_qknorm_rope_pack(ctypes.byref(args), _stream(q.device)))
    return out


def packed_qkv_attention(
    packed: torch.Tensor, softmax_scale: float | None = None
) -> tuple[torch.Tensor, torch.Tensor]:
    """Dense attention over an exchanged (rows_full, heads_local, 3*head_dim)
    buffer, as packed_ulysses.py:201-209 runs it: q, k, v are read in place
    as strided views. Returns ``(out (rows_full, heads_local, head_dim),
    lse (heads_local, rows_full))``."""

    if packed.dim() != 3 or packed.shape[-1] % 3:
        raise ValueError(f"packed must be (rows, heads_local, 3*head_dim), got {tuple(packed.shape)}")
    head_dim = packed.shape[-1] // 3
    q, k, v = packed.unsqueeze(0).split(head_dim, dim=-1)
    out, lse = flash_attn_func(q, k, v, softmax_scale=softmax_scale)
    return out.squeeze(0), lse.squeeze(0)
