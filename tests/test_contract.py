"""CPU contract tests of the adapter and of the kernel callable's argument
checks.

The processor contract is the one the reference pins in
tests/test_dense_fa4.py:11-52: with an injected kernel, a (1, 7, 8) hidden
state over 2 heads reaches the kernel as three (1, 7, 2, 4) BSHD tensors with
exactly ``causal=False``, the block's output keeps the input shape, the
``calls`` counter advances by one, and a mask is refused with a "padless"
message. The fake module here is built for this file: a tiny projection
stack whose attribute names are the ones the processor protocol reads
(dense_fa4.py:123-133,169-170).
"""

from __future__ import annotations

from pathlib import Path

import pytest
import torch

from h3_flash_amd import _ext
from h3_flash_amd.attention import (
    DenseMiniMaxH3Processor,
    flash_attn_func,
    hip_forward_op,
    install_dense_hip,
)
from h3_flash_amd.prologue import fused_qk_norm_rope, fused_qknorm_rope

HIDDEN, HEADS = 8, 2


class TinyH3Block(torch.nn.Module):
    """Projection stack with the attributes the processor reads; no weights
    are checked, so they stay at their random initialisation."""

    def __init__(self, fused: bool = False) -> None:
        super().__init__()
        self.heads = HEADS
        self.fused_projections = fused
        if fused:
            self.to_qkv = torch.nn.Linear(HIDDEN, 3 * HIDDEN, bias=False)
        for name in ("to_q", "to_k", "to_v"):
            setattr(self, name, torch.nn.Linear(HIDDEN, HIDDEN, bias=False))
        self.norm_q, self.norm_k = torch.nn.Identity(), torch.nn.Identity()
        self.to_out = torch.nn.ModuleList([torch.nn.Linear(HIDDEN, HIDDEN, bias=False), torch.nn.Identity()])


class RecordingKernel:
    """Kernel stand-in: remembers what it was called with and hands back
    ``v`` (optionally with a dummy LSE, as FA's tuple form does)."""

    def __init__(self, with_lse: bool = False) -> None:
        self.with_lse = with_lse
        self.seen: list[tuple[tuple[torch.Size, ...], dict]] = []

    def __call__(self, q, k, v, **kwargs):
        self.seen.append(((q.shape, k.shape, v.shape), dict(kwargs)))
        if self.with_lse:
            return v, torch.zeros(q.shape[0], q.shape[2], q.shape[1])
        return v


def test_missing_library_is_rejected(tmp_path: Path) -> None:
    with pytest.raises(RuntimeError, match="library not found"):
        _ext.load_library(tmp_path / "libh3attn.so")


def test_dense_processor_preserves_shape_and_full_sequence() -> None:
    kernel = RecordingKernel()
    processor = DenseMiniMaxH3Processor(kernel=kernel)
    hidden = torch.randn(1, 7, HIDDEN)
    block_out = processor(TinyH3Block(), hidden)

    assert block_out.shape == hidden.shape == (1, 7, 8)
    [(shapes, kwargs)] = kernel.seen  # one kernel call over the whole sequence
    assert shapes == ((1, 7, 2, 4),) * 3
    assert kwargs == {"causal": False}
    assert processor.calls == 1


def test_dense_processor_takes_first_of_tuple_and_fused_projection() -> None:
    block = TinyH3Block(fused=True)
    processor = DenseMiniMaxH3Processor(kernel=RecordingKernel(with_lse=True))
    hidden = torch.randn(2, 5, HIDDEN)
    block_out = processor(block, hidden)
    # The kernel echoes v, so the block returns to_out applied to the v third
    # of the fused projection.
    value = block.to_qkv(hidden)[..., 2 * HIDDEN :]
    assert torch.allclose(block_out, block.to_out[0](value))
    assert processor.calls == 1


def test_dense_processor_rejects_masked_sequence() -> None:
    kernel = RecordingKernel()
    processor = DenseMiniMaxH3Processor(kernel=kernel)
    with pytest.raises(RuntimeError, match="padless"):
        processor(TinyH3Block(), torch.randn(1, 3, HIDDEN), attention_mask=torch.ones(1, 3, dtype=torch.bool))
    assert kernel.seen == [] and processor.calls == 0


def test_rotary_path_requires_rmsnorm_parameters() -> None:
    processor = DenseMiniMaxH3Processor(kernel=lambda q, k, v, **kw: v)
    cos = torch.ones(7, 4)
    with pytest.raises(RuntimeError, match="norm_q/norm_k"):
        processor(TinyH3Block(), torch.randn(1, 7, HIDDEN), rotary_emb=(cos, cos))


def test_context_parallel_is_refused() -> None:
    processor = DenseMiniMaxH3Processor(kernel=lambda q, k, v, **kw: v)
    processor._parallel_config = object()
    with pytest.raises(RuntimeError, match="head shard"):
        processor(TinyH3Block(), torch.randn(1, 7, HIDDEN))


def test_default_processor_loads_the_hip_kernel() -> None:
    processor = DenseMiniMaxH3Processor()
    assert processor.kernel is flash_attn_func


@pytest.mark.parametrize(
    "kwargs",
    [
        {"attention_mask": object()},
        {"dropout_p": 0.1},
        {"enable_gqa": True},
        {"is_causal": True},
    ],
)
def test_forward_op_rejects_unsupported_semantics(kwargs) -> None:
    with pytest.raises(RuntimeError, match="unmasked"):
        hip_forward_op(None, None, None, None, kernel=lambda *a, **k: None, **kwargs)


def test_forward_op_returns_lse_on_request() -> None:
    # The kernel's LSE is (B, H, S); the forward op hands Diffusers'
    # context-parallel template (B, S, H), a transposed view.
    lse_bhs = torch.arange(2 * 3 * 5, dtype=torch.float32).reshape(2, 3, 5)
    out = torch.zeros(2, 5, 3, 4)

    def kernel(q, k, v, softmax_scale=None, causal=False):
        return out, lse_bhs

    assert hip_forward_op(None, 1, 2, 3, kernel=kernel) is out
    o, lse = hip_forward_op(None, 1, 2, 3, return_lse=True, kernel=kernel)
    assert o is out
    assert lse.shape == (2, 5, 3)
    assert torch.equal(lse, lse_bhs.permute(0, 2, 1))
    assert lse.data_ptr() == lse_bhs.data_ptr()  # a view, no copy
    assert (out + lse.unsqueeze(-1)).shape == out.shape  # the template's broadcast


def test_kernel_callable_rejects_causal_and_host_tensors() -> None:
    q = torch.zeros(1, 4, 1, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="non-causal"):
        flash_attn_func(q, q, q, causal=True)
    with pytest.raises(RuntimeError, match="ROCm device"):
        flash_attn_func(q, q, q)
    with pytest.raises(TypeError, match="bfloat16"):
        flash_attn_func(q.float(), q, q)


def test_prologue_rejects_odd_or_wide_rotary_dim() -> None:
    x = torch.zeros(1, 3, 2, 128, dtype=torch.bfloat16)
    w = torch.ones(128)
    for R in (3, 130):
        table = torch.zeros(3, R)
        with pytest.raises(ValueError, match="even rotary dimension no wider than the head"):
            fused_qknorm_rope(x, w, table, table, 1e-5)
        with pytest.raises(ValueError, match="even rotary dimension no wider than the head"):
            fused_qk_norm_rope(x, x, w, w, table, table, 1e-5, 1e-5)


class FakeTransformer(torch.nn.Module):
    def __init__(self, n: int) -> None:
        super().__init__()

        class MiniMaxH3Attention(TinyH3Block):
            def set_processor(self, processor):
                self.processor = processor

        self.blocks = torch.nn.ModuleList([MiniMaxH3Attention() for _ in range(n)])


def test_install_sets_one_shared_kernel_on_every_module() -> None:
    transformer = FakeTransformer(3)
    record = install_dense_hip(transformer)
    assert record["backend"] == "hip_gfx950"
    assert record["semantics"] == "dense"
    assert record["processor_count"] == 3
    assert record["abi_version"] == _ext.ABI_VERSION
    kernels = {id(block.processor.kernel) for block in transformer.blocks}
    assert len(kernels) == 1
    # the first module's processor fills the record's gate on its first rotary call
    assert record["gate"] == {}
    assert transformer.blocks[0].processor._runtime is record
    assert all(b.processor._runtime is None for b in transformer.blocks[1:])
    assert transformer._h3_flash_dense_hip_processors == [b.processor for b in transformer.blocks]


def test_install_without_modules_is_rejected() -> None:
    with pytest.raises(RuntimeError, match="no MiniMax H3 attention modules"):
        install_dense_hip(torch.nn.Sequential(torch.nn.Linear(2, 2)))
