"""GPU parity of the fused q/k RMSNorm + RoPE kernel against the fp32 oracle.

Both compute in fp32 and round once to bf16, so the bar is: every element
within one bf16 ulp of the oracle's bf16 result (or within 2e-6 absolute,
the fp32 cancellation error of n*cos - n'*sin for |n| up to ~8, where the
result is far below bf16 resolution at unit scale) and at least 99.9% of
elements bit-identical. Summation order of the row norm and FMA contraction
move an fp32 value by about one fp32 ulp, which flips the bf16 rounding only
for values within that distance of a rounding midpoint.
"""

from __future__ import annotations

import pytest
import torch

from h3_flash_amd.prologue import fused_qk_norm_rope, fused_qknorm_rope
from h3_flash_amd.rope import rope_3d_tables
from h3_flash_amd.synth import WORKLOADS, make_raw
from oracle.qknorm_rope import qknorm_rope_reference
from tests._golden import bf16, f32, golden

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    a = x.float().abs().clamp_min(2.0**-126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


def assert_rounding_parity(actual: torch.Tensor, expect_bf16: torch.Tensor, tag=""):
    a = actual.detach().cpu().float()
    e = expect_bf16.detach().cpu().float()
    diff = (a - e).abs()
    bound = torch.maximum(bf16_ulp(e) * 1.0001, torch.full_like(e, 2e-6))
    assert torch.all(diff <= bound), (tag, (diff / bound).max().item())
    exact = (diff == 0).float().mean().item()
    assert exact >= 0.999, (tag, exact)


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def test_golden_tables():
    g = golden()
    x, w = bf16("rope_x"), bf16("rope_w")
    for R in (96, 128):
        cos, sin = f32(f"rope{R}_cos"), f32(f"rope{R}_sin")
        y = fused_qknorm_rope(x.to(DEV), w.to(DEV), cos.to(DEV), sin.to(DEV), float(g["rope_eps"]))
        assert_rounding_parity(y, f32(f"rope{R}_out").to(torch.bfloat16), R)


@pytest.mark.parametrize("D,R", [(128, 128), (128, 96), (128, 0), (128, 42), (128, 44), (128, 2), (64, 64), (256, 128)])
@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
def test_widths_and_weight_dtypes(D, R, wdtype):
    B, S, H = 2, 37, 3
    x = _rand((B, S, H, D), D + R, 2.0)
    w = torch.randn(D, generator=torch.Generator().manual_seed(R)).to(wdtype)
    ang = torch.randn((S, R), generator=torch.Generator().manual_seed(7))
    cos, sin = ang.cos(), ang.sin()
    y = fused_qknorm_rope(x.to(DEV), w.to(DEV), cos.to(DEV), sin.to(DEV), 1e-5)
    assert_rounding_parity(y, qknorm_rope_reference(x, w, cos, sin, 1e-5), (D, R, wdtype))


@pytest.mark.parametrize("H", [1, 8, 9, 40])
def test_head_counts_around_the_chunk_size(H):
    # heads are walked in chunks of 8 per token
    B, S, D = 1, 50, 128
    q, k = _rand((B, S, H, D), 30 + H), _rand((B, S, H, D), 60 + H)
    wq = torch.randn(D, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    wk = torch.randn(D, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    cos, sin = rope_3d_tables((2, 5, 5))
    oq, ok = fused_qk_norm_rope(q.to(DEV), k.to(DEV), wq.to(DEV), wk.to(DEV), cos.to(DEV), sin.to(DEV), 1e-5, 1e-6)
    assert_rounding_parity(oq, qknorm_rope_reference(q, wq, cos, sin, 1e-5), ("q", H))
    assert_rounding_parity(ok, qknorm_rope_reference(k, wk, cos, sin, 1e-6), ("k", H))


@pytest.mark.parametrize("R", [128, 96, 42])
def test_edge_magnitudes(R):
    # rows of zeros (r = rsqrt(eps)), of tiny values (squares underflow), of
    # large ones whose squares still sum finitely, and of ones whose squares
    # overflow fp32 (r = 0): the fused and generic kernels against the fp32
    # oracle, which computes the same quantities
    B, S, H, D = 1, 8, 4, 128
    x = _rand((B, S, H, D), 40 + R)
    x[0, 0] = 0.0
    x[0, 1] = x[0, 1] * 1e-30
    x[0, 2] = x[0, 2] * 1e17
    x[0, 3] = x[0, 3] * 1e30
    x[0, 4, 1] = 0.0
    x[0, 4, 2] = 3.0e38
    w = torch.randn(D, generator=torch.Generator().manual_seed(41)).to(torch.bfloat16)
    ang = torch.randn((S, R), generator=torch.Generator().manual_seed(42))
    cos, sin = ang.cos(), ang.sin()
    expect = qknorm_rope_reference(x, w, cos, sin, 1e-6)
    assert torch.isfinite(expect.float()).all()
    y = fused_qknorm_rope(x.to(DEV), w.to(DEV), cos.to(DEV), sin.to(DEV), 1e-6)
    assert_rounding_parity(y, expect, ("edge", R))


def test_q_and_k_in_one_launch_equals_two_launches():
    B, S, H, D = 1, 300, 5, 128
    q, k = _rand((B, S, H, D), 1).to(DEV), _rand((B, S, H, D), 2).to(DEV)
    wq = torch.randn(D, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(DEV)
    wk = torch.randn(D, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(DEV)
    cos, sin = (t.to(DEV) for t in rope_3d_tables((3, 10, 10)))
    oq, ok = fused_qk_norm_rope(q, k, wq, wk, cos, sin, 1e-5, 1e-6)
    assert torch.equal(oq, fused_qknorm_rope(q, wq, cos, sin, 1e-5))
    assert torch.equal(ok, fused_qknorm_rope(k, wk, cos, sin, 1e-6))


def test_strided_input():
    qkv = _rand((1, 50, 2, 3 * 128), 5).to(DEV)
    q = qkv[..., :128]
    cos, sin = (t.to(DEV) for t in rope_3d_tables((2, 5, 5)))
    w = torch.ones(128, dtype=torch.bfloat16, device=DEV)
    y = fused_qknorm_rope(q, w, cos, sin, 1e-5)
    assert_rounding_parity(y, qknorm_rope_reference(q.cpu(), w.cpu(), cos.cpu(), sin.cpu(), 1e-5), "strided")


def test_cos_and_sin_with_different_row_strides():
    # sin as a column slice of a wider table, cos contiguous: one table stride
    # is passed to the launch, so the wrapper must give both the same stride
    B, S, H, D, R = 1, 40, 2, 128, 96
    x = _rand((B, S, H, D), 8)
    w = torch.ones(D, dtype=torch.bfloat16)
    ang = torch.randn((S, R), generator=torch.Generator().manual_seed(9))
    cos = ang.cos()
    wide = torch.zeros((S, 2 * R))
    wide[:, R:] = ang.sin()
    sin = wide[:, R:]
    assert sin.stride(0) != cos.stride(0)
    expect = qknorm_rope_reference(x, w, cos, ang.sin(), 1e-5)
    y = fused_qknorm_rope(x.to(DEV), w.to(DEV), cos.to(DEV), sin.to(DEV), 1e-5)
    assert_rounding_parity(y, expect, "single")
    oq, ok = fused_qk_norm_rope(x.to(DEV), x.to(DEV), w.to(DEV), w.to(DEV), cos.to(DEV), sin.to(DEV), 1e-5, 1e-5)
    assert_rounding_parity(oq, expect, "q")
    assert_rounding_parity(ok, expect, "k")


def test_broadcast_table_rows():
    # one table row broadcast over the sequence on the device (expand: row
    # stride 0), as a caller may pass for a single position
    B, S, H, D, R = 1, 24, 2, 128, 64
    x = _rand((B, S, H, D), 10)
    w = torch.ones(D, dtype=torch.bfloat16)
    ang = torch.randn((1, R), generator=torch.Generator().manual_seed(11))
    cos_d, sin_d = ang.cos().to(DEV).expand(S, R), ang.sin().to(DEV).expand(S, R)
    assert cos_d.stride(0) == 0
    expect = qknorm_rope_reference(x, w, ang.cos().expand(S, R), ang.sin().expand(S, R), 1e-5)
    y = fused_qknorm_rope(x.to(DEV), w.to(DEV), cos_d, sin_d, 1e-5)
    assert_rounding_parity(y, expect, "broadcast")


@pytest.mark.parametrize("name", ["c2", "c5"])
def test_full_size_workload(name):
    raw = make_raw(WORKLOADS[name])
    oq, ok = fused_qk_norm_rope(
        raw["q_raw"].to(DEV), raw["k_raw"].to(DEV), raw["w_q"], raw["w_k"], raw["cos"], raw["sin"], raw["eps"], raw["eps"]
    )
    torch.cuda.synchronize()
    for got, x in ((oq, raw["q_raw"]), (ok, raw["k_raw"])):
        ref = qknorm_rope_reference(x, raw["w_q"], raw["cos"], raw["sin"], raw["eps"])
        assert_rounding_parity(got, ref, name)
