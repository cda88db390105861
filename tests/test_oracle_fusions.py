"""Pins the row-fusion oracle (CPU) against what fixes it independently:
torch's own rms_norm / silu, the eager formulas the reference gates its
Triton kernels against (benchmarks/benchmark_transformer_fusions.py:76-105),
closed forms, and planted mistakes that must fail."""

from __future__ import annotations

import pytest
import torch
from torch.nn import functional

from oracle.fusions import (
    residual_gate_rmsnorm_modulate_reference,
    rmsnorm_modulate_reference,
    swiglu_reference,
    table_rows,
)


def _setup(rows=37, hidden=96, n_table=9, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((1, rows, hidden), generator=g)
    branch = torch.randn((1, rows, hidden), generator=g)
    weight = torch.randn(hidden, generator=g)
    wide = torch.randn((n_table, 6 * hidden), generator=g)
    shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, _ = wide.chunk(6, -1)
    index = torch.arange(rows) % n_table
    return x, branch, weight, shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, index


def test_rmsnorm_modulate_matches_eager_formula():
    x, _, weight, shift, scale, _, _, _, index = _setup()
    eps = 1e-5
    eager = functional.rms_norm(x, (x.shape[-1],), weight, eps) * (
        1.0 + scale.index_select(0, index)
    ) + shift.index_select(0, index)
    ours = rmsnorm_modulate_reference(x, weight, scale, shift, index, eps, out_dtype=None)
    torch.testing.assert_close(ours, eager, rtol=2e-6, atol=2e-6)


def test_residual_chain_matches_eager_formula():
    x, branch, weight, _, _, gate, shift, scale, index = _setup(seed=1)
    eps = 1e-6
    updated = x + gate.index_select(0, index) * branch
    normed = functional.rms_norm(updated, (x.shape[-1],), weight, eps)
    normed = normed * (1.0 + scale.index_select(0, index)) + shift.index_select(0, index)
    hidden, ours = residual_gate_rmsnorm_modulate_reference(
        x, branch, gate, weight, scale, shift, index, eps, out_dtype=None
    )
    torch.testing.assert_close(hidden, updated, rtol=0, atol=1e-6)
    torch.testing.assert_close(ours, normed, rtol=2e-6, atol=2e-6)


def test_swiglu_matches_silu():
    x = torch.randn((5, 7, 2 * 64), generator=torch.Generator().manual_seed(2)) * 4
    value, gate = x.chunk(2, -1)
    torch.testing.assert_close(swiglu_reference(x, out_dtype=None), value * functional.silu(gate), rtol=1e-6, atol=1e-6)


def test_closed_forms():
    x, branch, _, _, _, _, _, _, index = _setup(rows=11, hidden=64, seed=3)
    ones = torch.ones(64)
    zeros = torch.zeros((9, 64))
    # unit weight, no modulation: every row has mean square 1 / (1 + eps / ms)
    out = rmsnorm_modulate_reference(x, ones, zeros, zeros, index, 0.0, out_dtype=None)
    torch.testing.assert_close((out * out).mean(-1), torch.ones(1, 11), rtol=1e-5, atol=1e-5)
    # scale = -1 cancels the norm: the output is the shift row exactly
    shift = torch.randn((9, 64), generator=torch.Generator().manual_seed(4))
    out = rmsnorm_modulate_reference(x, ones, -torch.ones((9, 64)), shift, index, 1e-5, out_dtype=None)
    assert torch.equal(out.reshape(11, 64), shift[index])
    # gate 0: hidden is the residual; gate 1 and branch -residual: hidden 0, normed = shift
    hidden, _ = residual_gate_rmsnorm_modulate_reference(x, branch, zeros, ones, zeros, zeros, index, 1e-5, None)
    assert torch.equal(hidden, x)
    hidden, normed = residual_gate_rmsnorm_modulate_reference(
        x, -x, torch.ones((9, 64)), ones, zeros, shift, index, 1e-5, None
    )
    assert torch.count_nonzero(hidden) == 0
    assert torch.equal(normed.reshape(11, 64), shift[index])
    # swiglu: gate 0 gives 0, large gate gives value
    v = torch.randn((3, 8), generator=torch.Generator().manual_seed(5))
    assert torch.count_nonzero(swiglu_reference(torch.cat([v, torch.zeros(3, 8)], -1), None)) == 0
    torch.testing.assert_close(swiglu_reference(torch.cat([v, torch.full((3, 8), 40.0)], -1), None), v * 40.0)


def test_index_wraps_and_clamps():
    assert table_rows(torch.tensor([2, 0, 1]), 7, 3).tolist() == [2, 0, 1, 2, 0, 1, 2]
    assert table_rows(torch.tensor([5, -2], dtype=torch.int32), 4, 3).tolist() == [2, 0, 2, 0]


def _planted(x, weight, scale, shift, index, eps, mistake):
    C = x.shape[-1]
    h = x.reshape(-1, C).float()
    t = index[torch.arange(h.shape[0]) % index.numel()]
    if mistake == "sum_not_mean":
        n = h * torch.rsqrt((h * h).sum(-1, keepdim=True) + eps)
    elif mistake == "eps_outside":
        n = h * (torch.rsqrt((h * h).mean(-1, keepdim=True)) + eps)
    else:
        n = h * torch.rsqrt((h * h).mean(-1, keepdim=True) + eps)
    if mistake == "no_one_plus":
        return n * weight * scale[t] + shift[t]
    if mistake == "index_no_wrap":
        t = index.repeat(h.shape[0] // index.numel() + 1)[: h.shape[0]].flip(0)
    return n * weight * (1 + scale[t]) + shift[t]


@pytest.mark.parametrize("mistake", ["sum_not_mean", "eps_outside", "no_one_plus", "index_no_wrap"])
def test_planted_mistakes_fail(mistake):
    x, _, weight, shift, scale, _, _, _, index = _setup(seed=6)
    good = rmsnorm_modulate_reference(x, weight, scale, shift, index, 1e-2, out_dtype=None).reshape(-1, x.shape[-1])
    bad = _planted(x, weight, scale, shift, index, 1e-2, mistake)
    assert not torch.allclose(good, bad, rtol=1e-3, atol=1e-3)
