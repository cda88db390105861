"""CPU contract tests of the adapter, mirroring the reference's
tests/test_dense_fa4.py:11-52 (fake module + injected fake kernel) plus the
argument checks of the kernel callable and the prologue."""

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


class Attention(torch.nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.heads = 2
        self.fused_projections = False
        self.to_q = torch.nn.Linear(8, 8, bias=False)
        self.to_k = torch.nn.Linear(8, 8, bias=False)
        self.to_v = torch.nn.Linear(8, 8, bias=False)
        self.norm_q = torch.nn.Identity()
        self.norm_k = torch.nn.Identity()
        self.to_out = torch.nn.ModuleList([torch.nn.Linear(8, 8, bias=False), torch.nn.Identity()])


def test_missing_library_is_rejected(tmp_path: Path) -> None:
    with pytest.raises(RuntimeError, match="library not found"):
        _ext.load_library(tmp_path / "libh3attn.so")


def test_dense_processor_preserves_shape_and_full_sequence() -> None:
    seen = {}

    def kernel(q, k, v, **kwargs):
        seen["shapes"] = (q.shape, k.shape, v.shape)
        seen["kwargs"] = kwargs
        return v

    processor = DenseMiniMaxH3Processor(kernel=kernel)
    result = processor(Attention(), torch.randn(1, 7, 8))

    assert result.shape == (1, 7, 8)
    assert seen["shapes"] == ((1, 7, 2, 4),) * 3
    assert seen["kwargs"] == {"causal": False}
    assert processor.calls == 1


def test_dense_processor_takes_first_of_tuple_and_fused_projection() -> None:
    attn = Attention()
    attn.fused_projections = True
    attn.to_qkv = torch.nn.Linear(8, 24, bias=False)

    def kernel(q, k, v, **kwargs):
        return v, torch.zeros(q.shape[0], q.shape[2], q.shape[1])

    processor = DenseMiniMaxH3Processor(kernel=kernel)
    x = torch.randn(2, 5, 8)
    out = processor(attn, x)
    v = attn.to_qkv(x).chunk(3, dim=-1)[2]
    assert torch.allclose(out, attn.to_out[0](v))
    assert processor.calls == 1


def test_dense_processor_rejects_masked_sequence() -> None:
    processor = DenseMiniMaxH3Processor(kernel=lambda *args, **kwargs: None)
    with pytest.raises(RuntimeError, match="padless"):
        processor(None, None, attention_mask=object())


def test_rotary_path_requires_rmsnorm_parameters() -> None:
    processor = DenseMiniMaxH3Processor(kernel=lambda q, k, v, **kw: v)
    cos = torch.ones(7, 4)
    with pytest.raises(RuntimeError, match="norm_q/norm_k"):
        processor(Attention(), torch.randn(1, 7, 8), rotary_emb=(cos, cos))


def test_context_parallel_is_refused() -> None:
    processor = DenseMiniMaxH3Processor(kernel=lambda q, k, v, **kw: v)
    processor._parallel_config = object()
    with pytest.raises(RuntimeError, match="head shard"):
        processor(Attention(), torch.randn(1, 7, 8))


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
    def kernel(q, k, v, softmax_scale=None, causal=False):
        return v, "lse"

    assert hip_forward_op(None, 1, 2, 3, kernel=kernel) == 3
    assert hip_forward_op(None, 1, 2, 3, return_lse=True, kernel=kernel) == (3, "lse")


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

        class MiniMaxH3Attention(Attention):
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
    assert transformer._h3_flash_dense_hip_processors == [b.processor for b in transformer.blocks]


def test_install_without_modules_is_rejected() -> None:
    with pytest.raises(RuntimeError, match="no MiniMax H3 attention modules"):
        install_dense_hip(torch.nn.Sequential(torch.nn.Linear(2, 2)))
