"""The attention processor on the GPU: projections -> fused HIP q/k
RMSNorm + RoPE -> HIP attention -> output projection, against the same block
computed with the CPU oracle (fp32) from the same bf16 weights."""

from __future__ import annotations

import pytest
import torch

from h3_flash_amd import DenseMiniMaxH3Processor, install_dense_hip
from h3_flash_amd.rope import rope_3d_tables
from oracle.attention import sdpa_reference
from oracle.metrics import error_metrics
from oracle.qknorm_rope import qknorm_rope_reference

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


class MiniMaxH3Attention(torch.nn.Module):
    """Stand-in with the attributes the processor protocol reads."""

    def __init__(self, heads: int, head_dim: int = 128, fused: bool = False) -> None:
        super().__init__()
        hidden = heads * head_dim
        self.heads = heads
        self.fused_projections = fused
        g = torch.Generator().manual_seed(heads)
        init = lambda *shape: (torch.randn(shape, generator=g) / shape[-1] ** 0.5)  # noqa: E731
        if fused:
            self.to_qkv = torch.nn.Linear(hidden, 3 * hidden, bias=True)
            self.to_qkv.weight.data = init(3 * hidden, hidden)
        else:
            self.to_q = torch.nn.Linear(hidden, hidden, bias=True)
            self.to_k = torch.nn.Linear(hidden, hidden, bias=True)
            self.to_v = torch.nn.Linear(hidden, hidden, bias=True)
            for lin in (self.to_q, self.to_k, self.to_v):
                lin.weight.data = init(hidden, hidden)
        self.norm_q = torch.nn.RMSNorm(head_dim, eps=1e-6)
        self.norm_k = torch.nn.RMSNorm(head_dim, eps=1e-6)
        self.norm_q.weight.data = 1.0 + 0.1 * torch.randn(head_dim, generator=g)
        self.norm_k.weight.data = 1.0 + 0.1 * torch.randn(head_dim, generator=g)
        self.to_out = torch.nn.ModuleList([torch.nn.Linear(hidden, hidden, bias=True), torch.nn.Dropout(0.0)])
        self.processor = None

    def set_processor(self, processor):
        self.processor = processor

    def forward(self, hidden_states, rotary_emb=None, attention_mask=None):
        return self.processor(self, hidden_states, rotary_emb, attention_mask)


def eager_reference(attn: MiniMaxH3Attention, x: torch.Tensor, cos, sin) -> torch.Tensor:
    """The same block on the CPU: bf16 projections, oracle prologue + attention."""

    a = attn.to("cpu")
    x = x.cpu()
    if a.fused_projections:
        q, k, v = a.to_qkv(x).chunk(3, dim=-1)
    else:
        q, k, v = a.to_q(x), a.to_k(x), a.to_v(x)
    q, k, v = (t.unflatten(-1, (a.heads, -1)) for t in (q, k, v))
    q = qknorm_rope_reference(q, a.norm_q.weight, cos.cpu(), sin.cpu(), a.norm_q.eps)
    k = qknorm_rope_reference(k, a.norm_k.weight, cos.cpu(), sin.cpu(), a.norm_k.eps)
    o, _ = sdpa_reference(q, k, v)
    o = o.to(torch.bfloat16).flatten(2, 3)
    return a.to_out[1](a.to_out[0](o)).float()


@pytest.mark.parametrize("fused", [False, True])
def test_processor_block_matches_eager_reference(fused):
    heads, grid = 2, (2, 10, 13)
    S = grid[0] * grid[1] * grid[2]
    attn = MiniMaxH3Attention(heads, fused=fused).to(torch.bfloat16)
    x = torch.randn((1, S, heads * 128), generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    cos, sin = rope_3d_tables(grid)
    ref = eager_reference(attn, x, cos, sin)
    attn = attn.to(DEV)
    processor = DenseMiniMaxH3Processor()
    attn.set_processor(processor)
    with torch.no_grad():
        out = attn(x.to(DEV), rotary_emb=(cos.to(DEV), sin.to(DEV)))
    torch.cuda.synchronize()
    assert processor.calls == 1
    m = error_metrics(out.float(), ref)
    # the output projection adds bf16 rounding of both paths on top of attention
    assert m["relative_l2"] < 1e-2 and m["cosine"] > 0.9999, m


def test_install_and_run_every_module():
    class Transformer(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.blocks = torch.nn.ModuleList([MiniMaxH3Attention(1) for _ in range(2)])

    t = Transformer().to(torch.bfloat16).to(DEV)
    record = install_dense_hip(t)
    assert record["processor_count"] == 2
    cos, sin = (z.to(DEV) for z in rope_3d_tables((1, 8, 8)))
    x = torch.randn((1, 64, 128), device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        for blk in t.blocks:
            x = blk(x, rotary_emb=(cos, sin))
    torch.cuda.synchronize()
    assert torch.isfinite(x.float()).all()
    assert [b.processor.calls for b in t.blocks] == [1, 1]
    # the install record carries the fused prologue's first-block gate
    # (transformer.py:174-190): the HIP q against norm_q then eager RoPE,
    # which rounds once more (after the norm), so up to about two bf16 ulps
    gate = record["gate"]["qknorm_partial_rope"]
    assert set(gate) == {"max_abs", "mean_abs", "relative_l2", "cosine"}
    assert gate["max_abs"] <= 0.05 and gate["mean_abs"] <= 2e-3, gate
    assert gate["relative_l2"] <= 1e-2 and gate["cosine"] > 0.9999, gate
    with torch.no_grad():
        t.blocks[0](x, rotary_emb=(cos, sin))
    assert record["gate"]["qknorm_partial_rope"] is gate  # measured once
