"""Dense attention for MiniMax H3 blocks on MI355X, behind the reference's
dense-FA4 adapter interface.

Reference interface mirrored here (paths relative to the reference repo):

* ``flash_attn_func`` takes the FlashAttention call form the adapter uses,
  ``kernel(q, k, v, *, softmax_scale=None, causal=False)`` with BSHD bf16
  tensors (src/h3_flash/runtime/attention/dense_fa4.py:74-80,145), and returns
  ``(out, lse)`` like FA's ``return_lse`` form; LSE is fp32, natural log,
  shape (B, H, S).
* ``DenseMiniMaxH3Processor`` has the call signature, ``calls`` counter,
  ``kernel=`` injection seam and mask rejection of
  ``DenseFA4MiniMaxH3Processor`` (dense_fa4.py:88-170). Its q/k path is the
  fused ordering of src/h3_flash/runtime/kernels/transformer.py:146-202: with
  ``rotary_emb`` the q/k RMSNorm and RoPE run as one HIP launch, otherwise the
  module's own norms are applied.
* ``install_dense_hip`` mirrors ``install_dense_fa4`` (dense_fa4.py:173-194):
  one shared kernel on every H3 attention module and an audit record.
* ``hip_forward_op`` has the signature of ``_fa4_forward_op``
  (dense_fa4.py:53-81) and, unlike it, can return the LSE.

There is exactly one implementation: the gfx950 library bound in ``_ext``.
Nothing here falls back to another backend.
"""

from __future__ import annotations

import ctypes
import math
from collections.abc import Callable
from typing import Any

import torch

from . import _ext
from .audit import gate_qknorm_rope
from .projection import out_projection, qkv_projection
from .prologue import fused_qk_norm_rope

__all__ = [
    "flash_attn_func",
    "flash_attn_varlen_func",
    "load_kernel",
    "provenance",
    "hip_forward_op",
    "DenseMiniMaxH3Processor",
    "install_dense_hip",
]

HEAD_DIM = 128


def _strides3(t: torch.Tensor) -> tuple[int, int, int]:
    s = t.stride()
    return (s[0], s[1], s[2])


def _as_kernel_operand(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {t.dtype}")
    if t.dim() != 4:
        raise ValueError(f"{name} must be 4-D (batch, seq, heads, head_dim), got {tuple(t.shape)}")
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be on a ROCm device, got {t.device}")
    aligned = t.stride(-1) == 1 and all(s % 8 == 0 for s in t.stride()[:3]) and t.data_ptr() % 16 == 0
    return t if aligned else t.contiguous()


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def flash_attn_func(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    softmax_scale: float | None = None,
    causal: bool = False,
    *,
    cu_seqlens_q: torch.Tensor | None = None,
    cu_seqlens_k: torch.Tensor | None = None,
    max_seqlen_q: int | None = None,
    out: torch.Tensor | None = None,
    lse: torch.Tensor | None = None,
    split_tail: bool = True,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Non-causal attention forward on MI355X; returns ``(out, lse)``.

    ``q``: (B, Sq, H, 128) bf16; ``k``/``v``: (B, Sk, H, 128) bf16; any
    strides with a contiguous last dimension. ``softmax_scale`` defaults to
    1/sqrt(128). With ``cu_seqlens_q``/``cu_seqlens_k`` (int32, device,
    ``num_segments + 1`` offsets into the sequence dimension, batch 1) the
    attention is block-diagonal over the packed segments; ``max_seqlen_q``
    must be at least the longest query segment, as in FlashAttention's
    varlen call (query rows past it are not computed); when omitted it is
    read from ``cu_seqlens_q``, which synchronises the stream.
    ``out``/``lse`` may be passed pre-allocated (BSHD bf16 / (B, H, Sq)
    fp32).

    ``split_tail``: the tiles of the last round of a dense call run as
    key-range pieces (taken from a counter as CUs free up when there are
    more tiles than CUs; statically assigned when a single round would
    leave most CUs idle), merged by a second kernel; the workspace comes
    from torch's stream-ordered caching allocator. ``False`` runs every
    tile whole (results differ by rounding).

    Raises RuntimeError for semantics the dense path does not serve (causal,
    GQA) and for a missing library, mirroring dense_fa4.py:19-20,72-73.
    """

    if causal:
        raise RuntimeError("H3 dense HIP attention supports only non-causal attention")
    q = _as_kernel_operand(q, "q")
    k = _as_kernel_operand(k, "k")
    v = _as_kernel_operand(v, "v")
    B, Sq, H, D = q.shape
    if D != HEAD_DIM:
        raise ValueError(f"head_dim must be {HEAD_DIM}, got {D}")
    if k.shape != v.shape:
        raise ValueError(f"k and v shapes differ: {tuple(k.shape)} vs {tuple(v.shape)}")
    if k.shape[0] != B or k.shape[3] != D:
        raise ValueError(f"q {tuple(q.shape)} and k {tuple(k.shape)} are incompatible")
    if k.shape[2] != H:
        raise RuntimeError("H3 dense HIP attention does not support grouped-query attention")
    if not (q.device == k.device == v.device):
        raise ValueError("q, k and v must be on the same device")
    Sk = k.shape[1]
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)

    if out is None:
        out = torch.empty((B, Sq, H, D), dtype=torch.bfloat16, device=q.device)
    elif out.shape != (B, Sq, H, D) or out.dtype != torch.bfloat16 or out.stride(-1) != 1 or out.device != q.device:
        raise ValueError(f"out must be a bf16 (B, Sq, H, 128) tensor on {q.device} with a contiguous last dim")
    if lse is None:
        lse = torch.empty((B, H, Sq), dtype=torch.float32, device=q.device)
    elif lse.shape != (B, H, Sq) or lse.dtype != torch.float32 or lse.stride(-1) != 1 or lse.device != q.device:
        raise ValueError(f"lse must be an fp32 (B, H, Sq) tensor on {q.device} with a contiguous last dim")

    args = _ext.AttnArgs()
    args.abi_version = _ext.ABI_VERSION
    args.q, args.k, args.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    args.o, args.lse = out.data_ptr(), lse.data_ptr()
    args.batch, args.heads, args.seqlen_q, args.seqlen_k, args.head_dim = B, H, Sq, Sk, D
    args.q_stride[:] = _strides3(q)
    args.k_stride[:] = _strides3(k)
    args.v_stride[:] = _strides3(v)
    args.o_stride[:] = _strides3(out)
    args.lse_stride[:] = (lse.stride(0), lse.stride(1))
    args.softmax_scale = scale
    args.causal = 0
    if cu_seqlens_q is not None or cu_seqlens_k is not None:
        if cu_seqlens_q is None:
            raise ValueError("cu_seqlens_k given without cu_seqlens_q")
        if cu_seqlens_k is None:
            cu_seqlens_k = cu_seqlens_q
        for name, cu in (("cu_seqlens_q", cu_seqlens_q), ("cu_seqlens_k", cu_seqlens_k)):
            if cu.dtype != torch.int32 or cu.dim() != 1 or cu.device != q.device or not cu.is_contiguous():
                raise ValueError(f"{name} must be a contiguous 1-D int32 tensor on {q.device}")
        if cu_seqlens_q.numel() != cu_seqlens_k.numel() or cu_seqlens_q.numel() < 2:
            raise ValueError("cu_seqlens_q and cu_seqlens_k must have the same length >= 2")
        if B != 1:
            raise ValueError("packed varlen attention requires batch 1")
        if max_seqlen_q is None:
            # One host read of the offsets (synchronises the stream).
            max_seqlen_q = int((cu_seqlens_q[1:] - cu_seqlens_q[:-1]).max().item())
        args.cu_seqlens_q = cu_seqlens_q.data_ptr()
        args.cu_seqlens_k = cu_seqlens_k.data_ptr()
        args.num_segments = cu_seqlens_q.numel() - 1
        args.max_seqlen_q = int(max_seqlen_q)
        if args.max_seqlen_q <= 0:
            out.zero_()
            lse.fill_(float("-inf"))
            return out, lse
    lib = _ext.load_library()
    workspace = None
    with torch.cuda.device(q.device):
        need = lib.h3a_attn_fwd_workspace_size(ctypes.byref(args)) if split_tail else 0
        if need > 0:
            # Stream-ordered caching allocation: reused, not freed, after the call.
            workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
            args.workspace, args.workspace_bytes = workspace.data_ptr(), need
        rc = lib.h3a_attn_fwd(ctypes.byref(args), ctypes.c_void_p(_stream_handle(q.device)))
    if rc != _ext.H3A_OK:
        message = _ext.last_error(lib)
        if rc == _ext.H3A_EINVAL:
            raise ValueError(message)
        raise RuntimeError(message)
    return out, lse


def flash_attn_varlen_func(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int | None = None,
    max_seqlen_k: int | None = None,
    softmax_scale: float | None = None,
    causal: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """FA varlen call form on packed (total, H, D) tensors; returns
    ``(out (total, H, D), lse (H, total))``."""

    del max_seqlen_k
    o, lse = flash_attn_func(
        q.unsqueeze(0),
        k.unsqueeze(0),
        v.unsqueeze(0),
        softmax_scale=softmax_scale,
        causal=causal,
        cu_seqlens_q=cu_seqlens_q,
        cu_seqlens_k=cu_seqlens_k,
        max_seqlen_q=max_seqlen_q,
    )
    return o.squeeze(0), lse.squeeze(0)


def load_kernel() -> Callable[..., Any]:
    """Return the shared kernel callable; RuntimeError if the library is missing.

    Counterpart of ``load_fa4`` (dense_fa4.py:14-31).
    """

    _ext.load_library()
    return flash_attn_func


def provenance() -> dict[str, Any]:
    """Counterpart of ``fa4_provenance`` (dense_fa4.py:34-50)."""

    return {"distribution": "h3-flash-amd", **_ext.provenance()}


def hip_forward_op(
    _ctx: Any,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: Any = None,
    dropout_p: float = 0.0,
    is_causal: bool = False,
    scale: float | None = None,
    enable_gqa: bool = False,
    return_lse: bool = False,
    _save_ctx: bool = False,
    _parallel_config: Any = None,
    *,
    kernel: Callable[..., Any] = flash_attn_func,
) -> Any:
    """Forward op with the signature of ``_fa4_forward_op`` (dense_fa4.py:53-81).

    Rejects masks, dropout, GQA and causal attention with RuntimeError. With
    ``return_lse`` it returns ``(out, lse)`` where ``out`` is (B, S, H, D)
    and ``lse`` is fp32 **(B, S, H)**: the layout Diffusers' context-parallel
    template expects from a forward op (its ring merge broadcasts
    ``lse.unsqueeze(-1)`` against ``out``). The kernel's own (B, H, S) LSE
    is returned as a transposed view, so no copy is made;
    :func:`h3_flash_amd.context_parallel.merge_attention` takes it with
    ``lse_layout="bsh"``.
    """

    del _ctx, _save_ctx, _parallel_config
    if attention_mask is not None or dropout_p != 0.0 or enable_gqa or is_causal:
        raise RuntimeError("H3 dense HIP attention supports only unmasked non-causal inference attention")
    output = kernel(query, key, value, softmax_scale=scale, causal=False)
    if return_lse:
        out, lse = output
        return out, lse.transpose(1, 2)
    return output[0] if isinstance(output, tuple) else output


def _norm_params(norm: Any) -> tuple[torch.Tensor, float] | None:
    weight = getattr(norm, "weight", None)
    eps = getattr(norm, "eps", None)
    if not isinstance(weight, torch.Tensor) or eps is None:
        return None
    return weight, float(eps)


class DenseMiniMaxH3Processor:
    """Diffusers attention processor for ``MiniMaxH3Attention`` on one HIP path.

    Same protocol as ``DenseFA4MiniMaxH3Processor.__call__``
    (dense_fa4.py:112-170): projections -> (B, S, H, D) -> q/k norm + RoPE ->
    ``kernel(q, k, v, causal=False)`` -> ``to_out``. ``kernel`` defaults to
    :func:`flash_attn_func`; tests inject a fake through ``kernel=`` exactly
    as the reference's contract test does.
    """

    _attention_backend = None
    _parallel_config = None

    def __init__(
        self,
        *,
        kernel: Callable[..., Any] | None = None,
        fuse_projections: bool = False,
        fuse_out_projection: bool = False,
    ) -> None:
        self.kernel = load_kernel() if kernel is None else kernel
        self.calls = 0
        # fuse_projections: q/k/v come from one h3a_proj_gemm launch with the
        # q/k RMSNorm + RoPE in its epilogue (modules or inputs outside what
        # it takes keep the separate steps). Off by default: the module's
        # projections (hipBLASLt) followed by the HIP prologue keep the
        # reference's rounding order (projection rounded to bf16, then norm
        # and RoPE) and measured as fast or faster than the fused launch,
        # whose epilogue runs while the CU's matrix cores idle.
        # fuse_out_projection: to_out[0] runs on h3a_proj_gemm too; off by
        # default, hipBLASLt's GEMM is 1-4% faster there and there is no
        # epilogue to fold.
        self.fuse_projections = fuse_projections
        self.fuse_out_projection = fuse_out_projection
        # Set by install_dense_hip on the first module: the install record,
        # whose "gate" receives the fused prologue's error on the first call
        # (transformer.py:174-190).
        self._runtime: dict[str, Any] | None = None
        # Set by install_dense_hip on every module: the same record, whose
        # "projection_fallbacks" counts, per reason, the calls in which
        # fuse_projections was asked for and the separate steps ran.
        self._audit: dict[str, Any] | None = None

    def __call__(
        self,
        attn: Any,
        hidden_states: torch.Tensor,
        rotary_emb: tuple[torch.Tensor, torch.Tensor] | None = None,
        attention_mask: Any | None = None,
    ) -> torch.Tensor:
        if attention_mask is not None:
            raise RuntimeError("dense HIP attention requires the official padless sequence")
        if self._parallel_config is not None:
            raise RuntimeError(
                "dense HIP attention runs one GPU's head shard; context parallelism is not installed"
            )
        fused = None
        if self.fuse_projections:
            why: list[str] = []
            fused = qkv_projection(attn, hidden_states, rotary_emb, why)
            if fused is None and self._audit is not None:
                counts = self._audit.setdefault("projection_fallbacks", {})
                for reason in why:
                    counts[reason] = counts.get(reason, 0) + 1
        if fused is not None:
            query, key, value = fused
            if self._runtime is not None and "qknorm_partial_rope" not in self._runtime["gate"]:
                self._runtime["gate"]["qknorm_partial_rope"] = gate_qknorm_rope(attn, hidden_states, query, *rotary_emb)
        else:
            query, key, value = self._projections(attn, hidden_states, rotary_emb)
        output = self.kernel(query, key, value, causal=False)
        if isinstance(output, tuple):
            output = output[0]
        self.calls += 1
        output = output.flatten(2, 3).type_as(query)
        projected = out_projection(attn.to_out[0], output) if self.fuse_out_projection else None
        output = attn.to_out[0](output) if projected is None else projected
        return attn.to_out[1](output)

    def _projections(self, attn: Any, hidden_states: torch.Tensor, rotary_emb: Any):
        """The separate steps: projections, then the fused q/k prologue (or the
        module's norms without RoPE)."""

        if attn.fused_projections:
            query, key, value = attn.to_qkv(hidden_states).chunk(3, dim=-1)
        else:
            query = attn.to_q(hidden_states)
            key = attn.to_k(hidden_states)
            value = attn.to_v(hidden_states)
        query = query.unflatten(-1, (attn.heads, -1))
        key = key.unflatten(-1, (attn.heads, -1))
        value = value.unflatten(-1, (attn.heads, -1))
        if rotary_emb is None:
            query = attn.norm_q(query)
            key = attn.norm_k(key)
        else:
            nq, nk = _norm_params(attn.norm_q), _norm_params(attn.norm_k)
            if nq is None or nk is None:
                raise RuntimeError(
                    "dense HIP attention fuses q/k RMSNorm with RoPE and needs norm_q/norm_k "
                    "with .weight and .eps"
                )
            cos, sin = rotary_emb
            query, key = fused_qk_norm_rope(query, key, nq[0], nk[0], cos, sin, nq[1], nk[1])
            if self._runtime is not None and "qknorm_partial_rope" not in self._runtime["gate"]:
                self._runtime["gate"]["qknorm_partial_rope"] = gate_qknorm_rope(attn, hidden_states, query, cos, sin)
        return query, key, value


def install_dense_hip(
    transformer: Any,
    attention_class: type | None = None,
    *,
    fuse_projections: bool = False,
    fuse_out_projection: bool = False,
) -> dict[str, Any]:
    """Install one shared HIP kernel on every H3 attention module.

    Mirrors ``install_dense_fa4`` (dense_fa4.py:173-194). Modules are matched
    by ``attention_class`` when given, else by the class name
    ``MiniMaxH3Attention``. Raises RuntimeError when none is found or the
    library is missing.

    The returned record is live: its ``"gate"`` dict receives, on the first
    rotary call of the first module, the error metrics of the fused q/k
    RMSNorm + RoPE against the eager composition, as the reference's fused
    runtime records them (transformer.py:174-190); with
    ``fuse_projections``, its ``"projection_fallbacks"`` dict counts, per
    reason, the calls of any module that ran the separate projection steps
    instead of the fused projection GEMM.
    """

    kernel = load_kernel()
    processors = []
    for module in transformer.modules():
        matched = (
            isinstance(module, attention_class)
            if attention_class is not None
            else type(module).__name__ == "MiniMaxH3Attention"
        )
        if matched:
            processor = DenseMiniMaxH3Processor(
                kernel=kernel, fuse_projections=fuse_projections, fuse_out_projection=fuse_out_projection
            )
            processor._parallel_config = getattr(transformer, "_parallel_config", None)
            module.set_processor(processor)
            processors.append(processor)
    if not processors:
        raise RuntimeError("no MiniMax H3 attention modules found")
    transformer._h3_flash_dense_hip_processors = processors
    record = {
        "backend": "hip_gfx950",
        "semantics": "dense",
        "processor_count": len(processors),
        **provenance(),
        "fuse_projections": bool(fuse_projections),
        "gate": {},
        "projection_fallbacks": {},
    }
    processors[0]._runtime = record
    for processor in processors:
        processor._audit = record
    return record
