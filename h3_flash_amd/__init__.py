"""MI355X-native dense attention hot path of H3-Flash (gfx950 HIP kernels).

Public entry points:

* :func:`flash_attn_func` / :func:`flash_attn_varlen_func` — the attention
  kernel callable (bf16 BSHD in, bf16 out + fp32 LSE).
* :func:`fused_qknorm_rope` / :func:`fused_qk_norm_rope` — the fused q/k
  RMSNorm + RoPE prologue.
* :class:`DenseMiniMaxH3Processor` / :func:`install_dense_hip` — the
  Diffusers attention-processor adapter.
* :mod:`h3_flash_amd.relayout` — the packed-Ulysses pack / merge relayouts
  and the fused q/k prologue + pack.
* :mod:`h3_flash_amd.fusions` — the DiT block's row fusions
  (rmsnorm_modulate, residual_gate_rmsnorm_modulate, swiglu).
* :mod:`h3_flash_amd.context_parallel` — the LSE merge of partial attention
  results and the ring schedule on one device.
"""

from .attention import (
    DenseMiniMaxH3Processor,
    flash_attn_func,
    flash_attn_varlen_func,
    hip_forward_op,
    install_dense_hip,
    load_kernel,
    provenance,
)
from .context_parallel import chunked_attention, merge_attention
from .prologue import fused_qk_norm_rope, fused_qknorm_rope

__all__ = [
    "DenseMiniMaxH3Processor",
    "chunked_attention",
    "flash_attn_func",
    "flash_attn_varlen_func",
    "fused_qk_norm_rope",
    "fused_qknorm_rope",
    "hip_forward_op",
    "install_dense_hip",
    "load_kernel",
    "merge_attention",
    "provenance",
]
