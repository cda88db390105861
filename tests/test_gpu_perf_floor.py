"""Throughput floors that catch a structural slowdown: of the attention
kernel on the C2 shard (B=1 H=5 S=49,920) and the packed two-segment batch
(49,920 + 1,296 tokens), at least 900 TFLOP/s each. Boxes measure
1,150-1,317 TFLOP/s on both, so the floor sits well below box-to-box
variation; a contiguous per-XCD tile order once ran the packed batch at
~620 TFLOP/s, which this catches. Inputs are N(0,1) (no prologue: the
kernel's speed does not depend on it). Also the fused projection GEMM and a
row fusion, below."""

from __future__ import annotations

import pytest
import torch

from h3_flash_amd import flash_attn_func

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
FLOOR_TFLOPS = 900.0


@pytest.mark.parametrize("segments", [(49920,), (49920, 1296)], ids=["dense", "two-segments"])
def test_attention_throughput_floor(segments):
    S, H, D = sum(segments), 5, 128
    g = torch.Generator(device=DEV).manual_seed(5)
    q, k, v = (torch.randn((1, S, H, D), device=DEV, generator=g).to(torch.bfloat16) for _ in range(3))
    out = torch.empty_like(q)
    lse = torch.empty((1, H, S), device=DEV)
    kw = {}
    if len(segments) > 1:
        cu = torch.tensor([0, *torch.tensor(segments).cumsum(0).tolist()], dtype=torch.int32, device=DEV)
        kw = {"cu_seqlens_q": cu, "cu_seqlens_k": cu, "max_seqlen_q": max(segments)}
    for _ in range(8):  # the clock settles over the first launches
        flash_attn_func(q, k, v, out=out, lse=lse, **kw)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(10):
        flash_attn_func(q, k, v, out=out, lse=lse, **kw)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / 10
    tflops = 4 * D * H * sum(s * s for s in segments) / (ms * 1e-3) / 1e12
    assert tflops >= FLOOR_TFLOPS, f"{segments}: {tflops:.0f} TFLOP/s ({ms:.3f} ms per launch)"


def _ms_per_call(fn, warmup=5, reps=10):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def test_fused_projection_throughput_floor():
    # q/k/v of one 8-way rank at 480p/5s (6,240 tokens, hidden 5,120, 40
    # heads) with the q/k norm + RoPE epilogue: boxes measure 1,190-1,400
    # TFLOP/s; a floor of 900 catches a structural slowdown
    from h3_flash_amd.projection import Section, proj_gemm

    m, hidden = 6240, 5120
    g = torch.Generator(device=DEV).manual_seed(3)
    x = torch.randn((m, hidden), device=DEV, generator=g).to(torch.bfloat16)
    w = (torch.randn((3 * hidden, hidden), device=DEV, generator=g) / hidden**0.5).to(torch.bfloat16)
    nw = torch.ones(128, device=DEV, dtype=torch.bfloat16)
    theta = torch.rand((m, 64), device=DEV, generator=g) * 6.0
    theta = torch.cat((theta, theta), dim=1)
    cos, sin = theta.cos(), theta.sin()
    y = torch.empty((m, 3 * hidden), device=DEV, dtype=torch.bfloat16)
    secs = [
        Section(w[:hidden], y[:, :hidden], None, nw, 1e-6),
        Section(w[hidden : 2 * hidden], y[:, hidden : 2 * hidden], None, nw, 1e-6),
        Section(w[2 * hidden :], y[:, 2 * hidden :]),
    ]
    ms = _ms_per_call(lambda: proj_gemm(x, secs, cos, sin, m))
    tflops = 2.0 * m * 3 * hidden * hidden / (ms * 1e-3) / 1e12
    assert tflops >= 900.0, f"{tflops:.0f} TFLOP/s ({ms:.3f} ms per launch)"


def test_row_fusion_bandwidth_floor():
    # rmsnorm_modulate over the whole 480p/5s sequence (49,920 x 5,120, 1 GB
    # moved): boxes measure 5.9-6.1 TB/s; a floor of 4 TB/s catches a
    # structural slowdown
    from h3_flash_amd.fusions import fused_rmsnorm_modulate

    rows, hidden = 49920, 5120
    g = torch.Generator(device=DEV).manual_seed(4)
    x = torch.randn((1, rows, hidden), device=DEV, generator=g).to(torch.bfloat16)
    weight = torch.randn(hidden, device=DEV, generator=g).to(torch.bfloat16)
    table = torch.randn((9, 2 * hidden), device=DEV, generator=g).to(torch.bfloat16)
    shift, scale = table.chunk(2, -1)
    idx = torch.arange(rows, device=DEV) % 9
    ms = _ms_per_call(lambda: fused_rmsnorm_modulate(x, weight, scale, shift, idx, 1e-5))
    tbs = 2 * rows * hidden * 2 / (ms * 1e-3) / 1e12
    assert tbs >= 4.0, f"{tbs:.2f} TB/s ({ms:.3f} ms per launch)"
