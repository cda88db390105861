"""Throughput floors that catch a structural slowdown of the attention
kernel: the C2 shard (B=1 H=5 S=49,920) and the packed two-segment batch
(49,920 + 1,296 tokens), at least 900 TFLOP/s each. Boxes measure
1,150-1,317 TFLOP/s on both, so the floor sits well below box-to-box
variation; a contiguous per-XCD tile order once ran the packed batch at
~620 TFLOP/s, which this catches. Inputs are N(0,1) (no prologue: the
kernel's speed does not depend on it)."""

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
