"""MI355X-native dense attention hot path of H3-Flash (gfx950 HIP kernels).

The modules ``relayout``, ``fusions``, ``projection`` and
``context_parallel`` hold the rows around the attention call."""

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
