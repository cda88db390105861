"""GPU parity of the DiT-block row fusions against the fp32 oracle.

Both sides compute in fp32 and round once to bf16; the summation order of
the row norm and FMA contraction move an fp32 value by a few ulp, which
flips the bf16 rounding only near a rounding midpoint. Bar: every element
within one bf16 ulp of the oracle's bf16 result (or 1e-5 absolute where
terms cancel below bf16 resolution), and at least 99% bit-identical.
Shapes follow the reference's microbenchmark defaults
(benchmarks/benchmark_transformer_fusions.py:56-73: 257 rows, hidden 5376,
ffn 14336, 9 modulation rows indexed by arange % 9) and one Ulysses rank's
share of the 480p/5s sequence.
"""

from __future__ import annotations

import pytest
import torch

from h3_flash_amd.fusions import fused_residual_gate_rmsnorm_modulate, fused_rmsnorm_modulate, fused_swiglu
from oracle.fusions import (
    residual_gate_rmsnorm_modulate_reference,
    rmsnorm_modulate_reference,
    swiglu_reference,
)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    a = x.float().abs().clamp_min(2.0**-126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


def assert_parity(actual, expect, tag="", exact_min=0.99):
    a = actual.detach().float().cpu()
    e = expect.detach().float().cpu()
    assert a.shape == e.shape, (tag, a.shape, e.shape)
    diff = (a - e).abs()
    bound = torch.maximum(bf16_ulp(e) * 1.0001, torch.full_like(e, 1e-5))
    assert torch.all(diff <= bound), (tag, (diff / bound).max().item())
    exact = (diff == 0).float().mean().item()
    assert exact >= exact_min, (tag, exact)


def _inputs(rows, hidden, n_table=9, table_dtype=torch.bfloat16, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((1, rows, hidden), generator=g).to(torch.bfloat16)
    branch = torch.randn((1, rows, hidden), generator=g).to(torch.bfloat16)
    weight = torch.randn(hidden, generator=g).to(torch.bfloat16)
    wide = torch.randn((n_table, 6 * hidden), generator=g).to(table_dtype)
    return x, branch, weight, wide.chunk(6, -1)


@pytest.mark.parametrize(
    "rows, hidden, table_dtype, wdtype, idtype",
    [
        (257, 5376, torch.bfloat16, torch.bfloat16, torch.int64),  # reference microbenchmark shape
        (6240, 5376, torch.bfloat16, torch.bfloat16, torch.int64),  # one Ulysses rank at 480p/5s
        (33, 1000, torch.float32, torch.float32, torch.int32),
        (17, 1001, torch.bfloat16, torch.float32, torch.int64),  # odd width: element path
        (5, 20000, torch.bfloat16, torch.bfloat16, torch.int64),  # wider than the vector path
        (64, 8, torch.float32, torch.bfloat16, torch.int32),
        # vector path at other vector counts per lane (2048 columns per vector
        # step): a last vector held by one lane only, full steps, the widest
        (9, 2056, torch.bfloat16, torch.float32, torch.int64),
        (5, 6144, torch.float32, torch.float32, torch.int32),
        (4, 14344, torch.float32, torch.bfloat16, torch.int64),
        (3, 16384, torch.bfloat16, torch.bfloat16, torch.int32),
        # one wave per row (bf16 tables, 512 columns per vector step): one
        # full vector, the widest (11 per lane), one column step past it
        (6, 512, torch.bfloat16, torch.bfloat16, torch.int32),
        (5, 8, torch.bfloat16, torch.bfloat16, torch.int64),  # one vector, on lane 0 only
        (3, 24, torch.bfloat16, torch.float32, torch.int32),
        (10, 5632, torch.bfloat16, torch.float32, torch.int64),
        (7, 5640, torch.bfloat16, torch.bfloat16, torch.int32),
    ],
)
def test_rmsnorm_modulate(rows, hidden, table_dtype, wdtype, idtype):
    x, _, weight, (shift, scale, _, _, _, _) = _inputs(rows, hidden, table_dtype=table_dtype, seed=rows)
    weight = weight.to(wdtype)
    index = (torch.arange(rows) % 9).to(idtype)
    got = fused_rmsnorm_modulate(x.to(DEV), weight.to(DEV), scale.to(DEV), shift.to(DEV), index.to(DEV), 1e-5)
    assert got.shape == x.shape and got.dtype == torch.bfloat16
    assert_parity(got, rmsnorm_modulate_reference(x, weight, scale, shift, index, 1e-5), "rmsnorm_modulate")


@pytest.mark.parametrize(
    "rows, hidden, table_dtype, wdtype",
    [
        (257, 5376, torch.bfloat16, torch.bfloat16),
        (6240, 5376, torch.bfloat16, torch.bfloat16),
        (19, 1000, torch.float32, torch.bfloat16),
        (9, 1003, torch.bfloat16, torch.bfloat16),
        (7, 2056, torch.float32, torch.float32),
        (3, 16384, torch.bfloat16, torch.float32),
        (6, 4104, torch.bfloat16, torch.float32),  # one wave per row, last vector on one lane
        (9, 16, torch.bfloat16, torch.bfloat16),
        (5, 5632, torch.bfloat16, torch.bfloat16),
    ],
)
def test_residual_gate_rmsnorm_modulate(rows, hidden, table_dtype, wdtype):
    x, branch, weight, (_, _, gate, shift, scale, _) = _inputs(rows, hidden, table_dtype=table_dtype, seed=2 * rows)
    weight = weight.to(wdtype)
    index = torch.arange(rows) % 9
    hidden_out, normed = fused_residual_gate_rmsnorm_modulate(
        x.to(DEV), branch.to(DEV), gate.to(DEV), weight.to(DEV), scale.to(DEV), shift.to(DEV), index.to(DEV), 1e-6
    )
    ref_hidden, ref_normed = residual_gate_rmsnorm_modulate_reference(
        x, branch, gate, weight, scale, shift, index, 1e-6
    )
    assert_parity(hidden_out, ref_hidden, "hidden")
    assert_parity(normed, ref_normed, "normed")


def test_strided_rows_and_clamped_index():
    rows, hidden = 40, 2048
    base = torch.randn((rows, hidden + 64), generator=torch.Generator().manual_seed(7)).to(torch.bfloat16)
    x = base[:, :hidden]  # row stride hidden + 64
    _, _, weight, (shift, scale, _, _, _, _) = _inputs(rows, hidden, seed=8)
    index = torch.tensor([0, 3, 8, 12, -1], dtype=torch.int64)  # 12 and -1 lie outside the 9-row table
    got = fused_rmsnorm_modulate(x.to(DEV), weight.to(DEV), scale.to(DEV), shift.to(DEV), index.to(DEV), 1e-5)
    assert_parity(got, rmsnorm_modulate_reference(x, weight, scale, shift, index, 1e-5), "strided")


@pytest.mark.parametrize("hidden", [5120, 1001])
def test_edge_magnitudes(hidden):
    # rows of zeros, tiny values, large ones and ones whose squares overflow
    # fp32 (the norm factor goes to 0), on the vector and the element paths
    rows = 6
    x, branch, weight, (shift, scale, gate, _, _, _) = _inputs(rows, hidden, seed=12)
    x[0, 0] = 0.0
    x[0, 1] *= 1e-30
    x[0, 2] *= 1e17
    x[0, 3] *= 1e30
    branch[0, 4] = 0.0
    index = torch.arange(rows, dtype=torch.int64) % 9
    expect = rmsnorm_modulate_reference(x, weight, scale, shift, index, 1e-6)
    assert torch.isfinite(expect.float()).all()
    got = fused_rmsnorm_modulate(x.to(DEV), weight.to(DEV), scale.to(DEV), shift.to(DEV), index.to(DEV), 1e-6)
    assert_parity(got, expect, ("edge", hidden))
    residual = x * 1e-3
    rh, rn = residual_gate_rmsnorm_modulate_reference(residual, branch, gate, weight, scale, shift, index, 1e-6)
    h, n = fused_residual_gate_rmsnorm_modulate(
        residual.to(DEV), branch.to(DEV), gate.to(DEV), weight.to(DEV), scale.to(DEV), shift.to(DEV), index.to(DEV), 1e-6
    )
    assert_parity(h, rh, ("edge hidden", hidden))
    assert_parity(n, rn, ("edge normed", hidden))


def test_broadcast_table_rows():
    # modulation tables whose rows are one row broadcast on the device
    # (expand: row stride 0)
    rows, hidden = 24, 2048
    x, branch, weight, (shift, scale, gate, _, _, _) = _inputs(rows, hidden, seed=9)
    one = lambda t: t[:1].expand(9, hidden)  # noqa: E731
    dev1 = lambda t: t[:1].to(DEV).expand(9, hidden)  # noqa: E731
    assert dev1(scale).stride(0) == 0
    index = torch.arange(rows, dtype=torch.int64) % 9
    got = fused_rmsnorm_modulate(x.to(DEV), weight.to(DEV), dev1(scale), dev1(shift), index.to(DEV), 1e-5)
    assert_parity(got, rmsnorm_modulate_reference(x, weight, one(scale), one(shift), index, 1e-5), "broadcast")
    h, n = fused_residual_gate_rmsnorm_modulate(
        x.to(DEV), branch.to(DEV), dev1(gate), weight.to(DEV), dev1(scale), dev1(shift), index.to(DEV), 1e-5
    )
    rh, rn = residual_gate_rmsnorm_modulate_reference(x, branch, one(gate), weight, one(scale), one(shift), index, 1e-5)
    assert_parity(h, rh, "broadcast hidden")
    assert_parity(n, rn, "broadcast normed")


@pytest.mark.parametrize("rows, ffn", [(257, 14336), (6240, 14336), (7, 1000), (5, 1001)])
def test_swiglu(rows, ffn):
    x = (torch.randn((rows, 2 * ffn), generator=torch.Generator().manual_seed(ffn)) * 3).to(torch.bfloat16)
    got = fused_swiglu(x.to(DEV))
    assert got.shape == (rows, ffn)
    assert_parity(got, swiglu_reference(x), "swiglu")


def test_swiglu_batched_and_empty():
    x = torch.randn((2, 3, 2 * 64), generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    got = fused_swiglu(x.to(DEV))
    assert got.shape == (2, 3, 64)
    assert_parity(got, swiglu_reference(x), "batched")
    empty = torch.zeros((0, 128), dtype=torch.bfloat16, device=DEV)
    assert fused_swiglu(empty).shape == (0, 64)


def test_errors():
    x = torch.zeros((4, 64), dtype=torch.bfloat16, device=DEV)
    w = torch.ones(64, device=DEV)
    t = torch.zeros((2, 64), device=DEV)
    with pytest.raises(TypeError):
        fused_rmsnorm_modulate(x.float(), w, t, t, torch.zeros(1, dtype=torch.long, device=DEV), 1e-5)
    with pytest.raises(ValueError):
        fused_rmsnorm_modulate(x, torch.ones(32, device=DEV), t, t, torch.zeros(1, dtype=torch.long, device=DEV), 1e-5)
    with pytest.raises(ValueError):
        fused_rmsnorm_modulate(x, w, t, t, torch.zeros(0, dtype=torch.long, device=DEV), 1e-5)
    with pytest.raises(ValueError):
        fused_swiglu(torch.zeros((2, 63), dtype=torch.bfloat16, device=DEV))
