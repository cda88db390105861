"""Projection GEMMs of the H3 attention block on the HIP library (gfx950).

``h3a_proj_gemm`` computes ``x @ W^T + b`` for up to three output sections
in one launch, each section either stored as it is or, per 128-feature head,
RMS-normalised, scaled by the norm weight and rotated (rotate-half RoPE) in
the GEMM's epilogue. It takes the place of the reference's projection step
plus its separate q/k norm + RoPE:

* ``attn.to_qkv(hidden_states).chunk(3, dim=-1)`` or ``attn.to_q/to_k/to_v``
  (src/h3_flash/runtime/attention/dense_fa4.py:123-128,
  src/h3_flash/runtime/kernels/transformer.py:146-152), then
  ``norm_q/norm_k`` + ``_apply_rotary_emb`` or ``fused_qknorm_rope``
  (dense_fa4.py:132-140, transformer.py:155-173);
* ``attn.to_out[0](output)`` (dense_fa4.py:169) as one plain section.

The fused epilogue keeps the reference's rounding order: the projection is
rounded to bf16 (as the module's linear outputs it), then normalised and
rotated in fp32 and rounded once more. (Normalising the fp32 accumulator
instead, with a single rounding, moved the LSE of the attention that follows
by up to about 2e-3 against that order at 40 heads.) Any even rotary width
up to 128 is taken; RoPE tables in the rotate-half form (columns ``c`` and
``c + R/2`` equal, ``cos(cat(theta, theta))``) with R a multiple of 32 are
read at their first half only, others at every rotated column. Non-bf16
weights, a head size other than 128 or a call without RoPE (where the
reference applies the module's own norms) make :func:`qkv_projection`
return ``None``, with the reason, so the caller keeps the unfused path.
"""

from __future__ import annotations

import ctypes
import weakref
from typing import Any

import torch

from . import _ext

__all__ = ["Section", "proj_gemm", "qkv_projection", "out_projection", "rotate_half_tables"]

HEAD_DIM = 128
K_MULTIPLE = 128  # the launch's reduction length must be a multiple of this


class Section:
    """One output section: ``y = x @ weight^T + bias`` (then the q/k norm +
    RoPE when ``norm_weight`` is given). ``y`` is a (m, n) bf16 view with
    unit column stride."""

    __slots__ = ("weight", "bias", "y", "norm_weight", "eps")

    def __init__(self, weight, y, bias=None, norm_weight=None, eps=0.0):
        self.weight, self.y, self.bias, self.norm_weight, self.eps = weight, y, bias, norm_weight, float(eps)


def _ok2d(t: torch.Tensor) -> bool:
    return t.dim() == 2 and t.stride(1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0


def proj_gemm(
    x: torch.Tensor,
    sections: list[Section],
    cos: torch.Tensor | None = None,
    sin: torch.Tensor | None = None,
    seqlen: int | None = None,
    rotate_half: bool = True,
) -> None:
    """Launch ``h3a_proj_gemm`` on the current stream.

    ``x``: (m, k) bf16; each section's ``weight`` (n, k) bf16, ``y`` (m, n)
    bf16. ``cos``/``sin``: fp32 (seqlen, R) tables for the norm sections, R
    even (token row ``i`` of ``x`` uses table row ``i % seqlen``);
    ``rotate_half``: the caller's word that columns ``c`` and ``c + R/2``
    are equal, which lets the epilogue read the first half only (R a
    multiple of 32); ``False`` reads every rotated column.
    Raises ``ValueError`` for an argument the library rejects and
    ``RuntimeError`` for an unsupported one or a failed launch.
    """

    if not 1 <= len(sections) <= _ext.H3A_PROJ_MAX_SECTIONS:
        raise ValueError(f"1 to {_ext.H3A_PROJ_MAX_SECTIONS} sections, got {len(sections)}")
    args = _ext.ProjArgs()
    args.abi_version = _ext.ABI_VERSION
    args.x = x.data_ptr()
    args.x_stride = x.stride(0)
    args.m, args.k = x.shape
    args.head_dim = HEAD_DIM
    args.num_sections = len(sections)
    for i, s in enumerate(sections):
        d = args.sections[i]
        d.weight = s.weight.data_ptr()
        d.weight_stride = s.weight.stride(0)
        d.n = s.weight.shape[0]
        d.bias = s.bias.data_ptr() if s.bias is not None else None
        d.y = s.y.data_ptr()
        d.y_stride = s.y.stride(0)
        d.mode = _ext.H3A_PROJ_QKNORM_ROPE if s.norm_weight is not None else _ext.H3A_PROJ_PLAIN
        d.norm_weight = s.norm_weight.data_ptr() if s.norm_weight is not None else None
        d.eps = s.eps
    if cos is not None:
        args.cos, args.sin = cos.data_ptr(), sin.data_ptr()
        args.table_stride = cos.stride(0)
        args.rotary_dim = cos.shape[-1]
        args.seqlen = seqlen if seqlen is not None else cos.shape[0]
        args.rotate_half_tables = 1 if rotate_half else 0
    lib = _ext.load_library()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    rc = lib.h3a_proj_gemm(ctypes.byref(args), ctypes.c_void_p(stream))
    if rc != _ext.H3A_OK:
        message = _ext.last_error(lib)
        if rc == _ext.H3A_EINVAL:
            raise ValueError(message)
        raise RuntimeError(message)


# Attribute under which a cos table object remembers its last check: (a weak
# reference to the sin table it was checked with, both tables' versions, the
# answer). It lives on the tensor object itself, so a later table that reuses
# a freed table's memory (the caching allocator hands addresses out again,
# and a new tensor starts at version 0) never sees an earlier answer.
_HALF_ATTR = "_h3a_rotate_half"


def rotate_half_tables(cos: torch.Tensor, sin: torch.Tensor) -> bool:
    """Whether columns ``c`` and ``c + R/2`` of both tables are equal (one
    device comparison per pair of table objects and versions, then cached on
    the cos tensor)."""

    R = cos.shape[-1]
    if R % 2 or sin.shape != cos.shape:
        return False
    memo = getattr(cos, _HALF_ATTR, None)
    if memo is not None:
        sin_ref, cos_ver, sin_ver, hit = memo
        if sin_ref() is sin and cos_ver == cos._version and sin_ver == sin._version:
            return hit
    h = R // 2
    hit = bool(torch.equal(cos[..., :h], cos[..., h:]) and torch.equal(sin[..., :h], sin[..., h:]))
    setattr(cos, _HALF_ATTR, (weakref.ref(sin), cos._version, sin._version, hit))
    return hit


def _linear_parts(linear: Any) -> tuple[torch.Tensor, torch.Tensor | None] | None:
    w = getattr(linear, "weight", None)
    b = getattr(linear, "bias", None)
    if not isinstance(w, torch.Tensor) or w.dtype != torch.bfloat16 or not _ok2d(w):
        return None
    if b is not None and (b.dtype != torch.bfloat16 or b.stride(0) != 1 or b.data_ptr() % 8):
        return None
    return w, b


def qkv_projection(
    attn: Any,
    hidden_states: torch.Tensor,
    rotary_emb: tuple[torch.Tensor, torch.Tensor] | None,
    why: list[str] | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None:
    """q, k, v as (B, S, H, 128) bf16 views of one (B, S, 3*H*128) buffer, q
    and k normalised and rotated in the GEMM epilogue; ``None`` when the
    module or inputs are outside what the fused launch takes (then nothing
    was launched, and the reason is appended to ``why`` when given).

    Every even rotary width up to 128 is taken (the reference's prologue
    takes any, src/h3_flash/runtime/kernels/fusions.py:268-275; tables built
    as _official_rope builds them have R = 6 * len(inv_freq), e.g. 126,
    src/h3_flash/runtime/parallel/rank_local_io.py:74-80). Tables in the
    rotate-half form with R a multiple of 32 are read at their first half;
    others at every rotated column."""

    def no(reason: str):
        if why is not None:
            why.append(reason)
        return None

    x = hidden_states
    if x.dim() != 3 or x.dtype != torch.bfloat16 or x.device.type != "cuda":
        return no("hidden_states is not a 3-d bf16 GPU tensor")
    H = getattr(attn, "heads", None)
    if not isinstance(H, int):
        return no("the module has no integer heads")
    B, S, hidden = x.shape
    if hidden % 128 or not x.is_contiguous() or x.data_ptr() % 16 or B * S == 0:
        return no("hidden_states is empty, not contiguous, not 16-byte aligned or its width not a multiple of 128")
    nq, nk = getattr(attn, "norm_q", None), getattr(attn, "norm_k", None)
    wq_n, wk_n = getattr(nq, "weight", None), getattr(nk, "weight", None)
    if not (isinstance(wq_n, torch.Tensor) and isinstance(wk_n, torch.Tensor)):
        return no("norm_q / norm_k carry no weight")
    if getattr(nq, "eps", None) is None or getattr(nk, "eps", None) is None:
        return no("norm_q / norm_k carry no eps")
    if wq_n.shape != (HEAD_DIM,) or wk_n.shape != (HEAD_DIM,) or wq_n.dtype != torch.bfloat16 or wk_n.dtype != torch.bfloat16:
        return no("norm weights are not bf16 of head_dim 128")
    if attn.fused_projections:
        parts = _linear_parts(attn.to_qkv)
        if parts is None:
            return no("to_qkv is not a bf16 linear with 16-byte aligned rows")
        w, b = parts
        n = w.shape[0] // 3
        weights = (w[:n], w[n : 2 * n], w[2 * n :])
        biases = (None, None, None) if b is None else (b[:n], b[n : 2 * n], b[2 * n :])
    else:
        ps = [_linear_parts(m) for m in (attn.to_q, attn.to_k, attn.to_v)]
        if any(q is None for q in ps):
            return no("to_q / to_k / to_v are not bf16 linears with 16-byte aligned rows")
        weights = tuple(q[0] for q in ps)
        biases = tuple(q[1] for q in ps)
        n = weights[0].shape[0]
        if any(w.shape[0] != n for w in weights):
            return no("to_q / to_k / to_v differ in width")
    if n != H * HEAD_DIM or hidden % K_MULTIPLE or any(w.shape[1] != hidden for w in weights):
        return no("projection widths do not match heads * 128, or hidden is not a multiple of 128")
    if rotary_emb is None:
        # without RoPE the module's own norms apply (transformer.py:155-158)
        return no("no rotary_emb: the module's own norms apply")
    cos, sin = rotary_emb
    R = cos.shape[-1] if cos.dim() == 2 else -1
    if cos.dim() != 2 or cos.shape[0] != S or R % 2 or R > HEAD_DIM or sin.shape != cos.shape:
        return no(f"rotary tables of shape {tuple(cos.shape)} / {tuple(sin.shape)} for {S} tokens (even R <= 128 taken)")
    # Checked on the caller's own table objects (the conversions below may
    # make fresh temporaries); a dtype or layout change keeps the form.
    half_form = rotate_half_tables(cos, sin) if R % 32 == 0 and R > 0 else False
    cos = cos.to(device=x.device, dtype=torch.float32)
    sin = sin.to(device=x.device, dtype=torch.float32)
    if not (cos.is_contiguous() and sin.is_contiguous()):
        cos, sin = cos.contiguous(), sin.contiguous()
    wq_n, wk_n = (t.to(x.device) for t in (wq_n, wk_n))
    out = torch.empty((B, S, 3 * n), dtype=torch.bfloat16, device=x.device)
    y = out.view(B * S, 3 * n)
    sections = [
        Section(weights[0], y[:, :n], biases[0], wq_n, nq.eps),
        Section(weights[1], y[:, n : 2 * n], biases[1], wk_n, nk.eps),
        Section(weights[2], y[:, 2 * n :], biases[2]),
    ]
    proj_gemm(x.view(B * S, hidden), sections, cos, sin, S, rotate_half=half_form)
    q, k, v = out.chunk(3, dim=-1)
    return q.unflatten(-1, (H, HEAD_DIM)), k.unflatten(-1, (H, HEAD_DIM)), v.unflatten(-1, (H, HEAD_DIM))


def out_projection(linear: Any, x: torch.Tensor) -> torch.Tensor | None:
    """``linear(x)`` for a bf16 nn.Linear on (..., k) bf16 input through one
    plain section; ``None`` when the shapes are outside what the launch takes."""

    parts = _linear_parts(linear)
    if parts is None or x.dtype != torch.bfloat16 or x.device.type != "cuda":
        return None
    w, b = parts
    k = x.shape[-1]
    if w.shape[1] != k or w.shape[0] % 128 or k % K_MULTIPLE or not x.is_contiguous() or x.data_ptr() % 16:
        return None
    x2 = x.view(-1, k)
    y = torch.empty((x2.shape[0], w.shape[0]), dtype=torch.bfloat16, device=x.device)
    if x2.shape[0]:
        proj_gemm(x2, [Section(w, y, b)])
    return y.view(*x.shape[:-1], w.shape[0])
