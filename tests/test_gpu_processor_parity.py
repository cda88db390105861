"""The attention processor at the path's tolerance, against an oracle that
follows the reference's order.

The reference's processor (src/h3_flash/runtime/attention/dense_fa4.py:123-145,
and the fused ordering of src/h3_flash/runtime/kernels/transformer.py:146-173)
projects hidden_states with the module's linears (bf16 output), normalises
and rotates q and k (fp32 arithmetic, one bf16 rounding), then calls the
kernel. The oracle here does the same on the CPU: the projection as an fp32
product rounded to bf16, ``qknorm_rope_reference`` on it, then the fp32 SDPA
oracle on seeded rows.

A kernel wrapper records what the processor hands the kernel (q, k, v) and
what the kernel returns (out, LSE). Out and LSE must meet the path's bar
against the oracle (max abs <= 2e-2, mean abs <= 2e-3, |dLSE| <= 1e-3), for
the processor as constructed by default (hipBLASLt projections + the HIP
prologue), for the fused projection GEMM (its epilogue rounds the
projection to bf16 before the norm, as the reference does; rounding once,
from the fp32 accumulator, measured LSE errors of 1.9-2.1e-3 here), for both
projection layouts (to_qkv and to_q/to_k/to_v), with the 44/42/42 3D tables
and with tables built as _official_rope builds them (21 shared frequencies,
R = 126).
The q/k the processor produced must lie within the bound that rounding the
projection first sets on the CPU (tests/test_oracle_projection.py: 2^-4 at
most, 2^-8 on average).

Shape: 40 heads, hidden 5,120, the 6,240 tokens of one 8-way rank at 480p/5s
(latent grid 4 x 30 x 52).
"""

from __future__ import annotations

import pytest
import torch

from h3_flash_amd import DenseMiniMaxH3Processor, flash_attn_func
from h3_flash_amd.rope import rope_3d_tables
from oracle.attention import sdpa_rows
from oracle.metrics import ATTN_MAX_ABS, ATTN_MEAN_ABS, LSE_MAX_ABS, error_metrics
from oracle.projection import projection_reference
from oracle.qknorm_rope import qknorm_rope_reference

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
HEADS, D, GRID = 40, 128, (4, 30, 52)
HIDDEN = HEADS * D
S = GRID[0] * GRID[1] * GRID[2]


class H3Attention(torch.nn.Module):
    """The attributes the processor protocol reads (dense_fa4.py:123-133,169-170)."""

    def __init__(self, fused: bool, seed: int) -> None:
        super().__init__()
        self.heads = HEADS
        self.fused_projections = fused
        g = torch.Generator().manual_seed(seed)

        def linear(n_in, n_out):
            lin = torch.nn.Linear(n_in, n_out, bias=True)
            lin.weight.data = torch.randn((n_out, n_in), generator=g) / n_in**0.5
            lin.bias.data = 0.1 * torch.randn(n_out, generator=g)
            return lin

        if fused:
            self.to_qkv = linear(HIDDEN, 3 * HIDDEN)
        else:
            self.to_q, self.to_k, self.to_v = (linear(HIDDEN, HIDDEN) for _ in range(3))
        self.norm_q = torch.nn.RMSNorm(D, eps=1e-6)
        self.norm_k = torch.nn.RMSNorm(D, eps=1e-6)
        self.norm_q.weight.data = 1.0 + 0.1 * torch.randn(D, generator=g)
        self.norm_k.weight.data = 1.0 + 0.1 * torch.randn(D, generator=g)
        self.to_out = torch.nn.ModuleList([linear(HIDDEN, HIDDEN), torch.nn.Dropout(0.0)])

    def weights(self):
        """(weight, bias) of q, k, v as bf16 CPU tensors."""
        if self.fused_projections:
            w, b = self.to_qkv.weight.detach().cpu(), self.to_qkv.bias.detach().cpu()
            return [(w[i * HIDDEN : (i + 1) * HIDDEN], b[i * HIDDEN : (i + 1) * HIDDEN]) for i in range(3)]
        return [(m.weight.detach().cpu(), m.bias.detach().cpu()) for m in (self.to_q, self.to_k, self.to_v)]


class RecordingKernel:
    """The processor's kernel: HIP attention, keeping its inputs and outputs."""

    def __init__(self) -> None:
        self.record = None

    def __call__(self, q, k, v, causal=False):
        out, lse = flash_attn_func(q, k, v, causal=causal)
        self.record = tuple(t.detach().clone() for t in (q, k, v, out, lse))
        return out, lse


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 values at |x| (8 significand bits)."""
    e = torch.floor(torch.log2(x.abs().clamp_min(2.0**-126)))
    return 2.0 ** (e - 7)


def reference_order(attn: H3Attention, x: torch.Tensor, cos, sin):
    """q, k, v in the reference's order: bf16 projection, then the q/k
    norm + RoPE oracle on it (fp32, one rounding)."""

    x2 = x.detach().cpu().view(S, HIDDEN)
    (wq, bq), (wk, bk), (wv, bv) = attn.weights()
    q, k, v = (projection_reference(x2, w, b).view(1, S, HEADS, D) for w, b in ((wq, bq), (wk, bk), (wv, bv)))
    q = qknorm_rope_reference(q, attn.norm_q.weight.detach().cpu(), cos, sin, attn.norm_q.eps)
    k = qknorm_rope_reference(k, attn.norm_k.weight.detach().cpu(), cos, sin, attn.norm_k.eps)
    return q, k, v


def official_rope_tables(grid, n_freq: int = 21, base: float = 10000.0):
    """Tables built as _official_rope builds them (rank_local_io.py:74-80):
    one inv_freq of n_freq entries for every axis, angles cat(t f, h f, w f)
    repeated, so R = 6 * n_freq (126 for 21 frequencies)."""

    inv = 1.0 / base ** (torch.arange(0, 2 * n_freq, 2, dtype=torch.float32) / (2 * n_freq))
    T, Hp, Wp = grid
    n = torch.arange(T * Hp * Wp)
    pos = torch.stack((n // (Hp * Wp), (n // Wp) % Hp, n % Wp), dim=-1).float()
    theta = torch.cat([pos[:, a : a + 1] * inv[None, :] for a in range(3)], dim=-1)
    theta = torch.cat((theta, theta), dim=-1)
    return theta.cos(), theta.sin()


@pytest.mark.parametrize(
    "fused_module,fuse_projections,tables",
    [(True, None, "3d"), (False, None, "3d"), (True, True, "3d"), (False, True, "3d"), (True, True, "r126"),
     (False, None, "r126")],
    ids=["to_qkv-default", "to_q_k_v-default", "to_qkv-fused-gemm", "to_q_k_v-fused-gemm", "to_qkv-fused-gemm-R126",
         "to_q_k_v-default-R126"],
)
def test_processor_attention_meets_the_path_tolerance(fused_module, fuse_projections, tables):
    attn = H3Attention(fused_module, seed=31 + fused_module).to(torch.bfloat16)
    g = torch.Generator().manual_seed(7)
    x = torch.randn((1, S, HIDDEN), generator=g).to(torch.bfloat16)
    cos, sin = rope_3d_tables(GRID) if tables == "3d" else official_rope_tables(GRID)
    q_ref, k_ref, v_ref = reference_order(attn, x, cos, sin)

    kernel = RecordingKernel()
    kw = {} if fuse_projections is None else {"fuse_projections": fuse_projections}
    processor = DenseMiniMaxH3Processor(kernel=kernel, **kw)
    processor._audit = {}
    attn = attn.to(DEV)
    with torch.no_grad():
        block = processor(attn, x.to(DEV), (cos.to(DEV), sin.to(DEV)))
    torch.cuda.synchronize()
    assert processor._audit.get("projection_fallbacks", {}) == {}  # the fused launch ran when asked for
    assert processor.calls == 1 and kernel.record is not None
    assert block.shape == (1, S, HIDDEN) and torch.isfinite(block.float()).all()
    q, k, v, out, lse = (t.cpu() for t in kernel.record)
    tag = (fused_module, fuse_projections, tables, cos.shape[-1])

    # what reached the kernel: v is the bf16 projection (hipBLASLt, which may
    # round the product before adding the bias, or the GEMM's plain section)
    # against an fp32 product rounded once: at most one bf16 step of values
    # under 8; q and k within the rounding-order bound
    dv = (v.float() - v_ref.float()).abs()
    print(tag, "v", float(dv.max()), float(dv.mean()), float((dv == 0).float().mean()))
    assert dv.max() <= 2.0**-5 and dv.mean() <= 2.0**-10, (tag, float(dv.max()), float(dv.mean()))
    for name, got, ref in (("q", q, q_ref), ("k", k, k_ref)):
        d = (got.float() - ref.float()).abs()
        print(tag, name, float(d.max()), float(d.mean()))
        assert d.max() <= 2.0**-4 and d.mean() <= 2.0**-8, (tag, name, float(d.max()), float(d.mean()))

    # what the kernel returned, on seeded rows against all keys
    rows = torch.randperm(S, generator=torch.Generator().manual_seed(11))[:640].sort().values
    ref_o, ref_l = sdpa_rows(q_ref, k_ref, v_ref, rows)
    m = error_metrics(out[:, rows].float(), ref_o)
    lse_err = (lse[:, :, rows].double() - ref_l.double()).abs().max().item()
    print(tag, "attention", m, "lse", lse_err)
    assert m["finite"], tag
    assert m["max_abs"] <= ATTN_MAX_ABS, (tag, m)
    assert m["mean_abs"] <= ATTN_MEAN_ABS, (tag, m)
    assert lse_err <= LSE_MAX_ABS, (tag, lse_err)


def test_default_processor_keeps_the_reference_order():
    # the processor as constructed: projections on the module's linears,
    # then the fused HIP prologue, so q and k are the prologue applied to the
    # bf16 projection, exactly as the prologue oracle bounds it (one bf16
    # ulp of the oracle on every element)
    attn = H3Attention(True, seed=5).to(torch.bfloat16)
    x = torch.randn((1, S, HIDDEN), generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    cos, sin = rope_3d_tables(GRID)
    kernel = RecordingKernel()
    processor = DenseMiniMaxH3Processor(kernel=kernel)
    assert processor.fuse_projections is False
    attn = attn.to(DEV)
    with torch.no_grad():
        processor(attn, x.to(DEV), (cos.to(DEV), sin.to(DEV)))
        proj_q = attn.to_qkv(x.to(DEV)).chunk(3, dim=-1)[0].unflatten(-1, (HEADS, D))
    torch.cuda.synchronize()
    q = kernel.record[0].cpu().float()
    want = qknorm_rope_reference(proj_q.cpu(), attn.norm_q.weight.detach().cpu(), cos, sin, attn.norm_q.eps).float()
    bound = torch.maximum(bf16_ulp(want) * 1.0001, torch.full_like(want, 2e-6))
    assert torch.all((q - want).abs() <= bound)
