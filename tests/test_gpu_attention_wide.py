"""GPU parity of attention on views that span 2 GiB or more.

The reference's seam hands the kernel ``to_qkv(...).chunk(3)`` views of any
length (src/h3_flash/runtime/attention/dense_fa4.py:123-131,145). Views whose
rows span 2^31 bytes or more take the kernel's wide form, whose K / V buffer
resources are rebased at every key tile they load. The narrow form runs the same
tiles in the same order on a contiguous copy, so both must give the same
bits; sampled rows are also checked against the CPU oracle.
"""

from __future__ import annotations

import pytest
import torch

from h3_flash_amd import flash_attn_func
from oracle.attention import sdpa_rows
from oracle.metrics import ATTN_MAX_ABS, ATTN_MEAN_ABS, LSE_MAX_ABS, error_metrics

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _check_rows(q, k, v, out, lse, rows, cu=None, tag=""):
    ref_o, ref_l = sdpa_rows(q.cpu(), k.cpu(), v.cpu(), rows, cu_seqlens=cu)
    idx = rows.to(DEV)
    m = error_metrics(out[:, idx].float().cpu(), ref_o)
    lse_err = (lse[:, :, idx].cpu().double() - ref_l.double()).abs().max().item()
    assert m["finite"] and m["max_abs"] <= ATTN_MAX_ABS and m["mean_abs"] <= ATTN_MEAN_ABS, (tag, m)
    assert lse_err <= LSE_MAX_ABS, (tag, lse_err)


def test_fused_projection_views_of_40_heads_past_2gib():
    """to_qkv output chunked into q/k/v views at 40 heads and S = 72,003: each
    view spans 72,003 rows x 30,720 bytes = 2.21 GB (dynamic tail, ragged
    last query and key tiles)."""

    S, H, D = 72_003, 40, 128
    print(f"case: to_qkv views S={S} H={H}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(41)
    qkv = torch.randn((1, S, 3 * H * D), device=DEV, generator=g).to(torch.bfloat16)
    q, k, v = (t.unflatten(-1, (H, D)) for t in qkv.chunk(3, dim=-1))
    assert q.stride(1) * 2 * S >= 2**31
    out, lse = flash_attn_func(q, k, v)
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    del qkv
    out_c, lse_c = flash_attn_func(qc, kc, vc)
    torch.cuda.synchronize()
    assert torch.equal(out, out_c) and torch.equal(lse, lse_c)
    rows = torch.tensor([0, 1, 255, 256, 40_000, S - 258, S - 3, S - 2, S - 1])
    _check_rows(qc, kc, vc, out, lse, rows, tag="to_qkv views")


def test_views_past_4gib_dense_split_and_varlen():
    """One head each of q, k and v as column slices of a (40,000, 65,536)
    buffer: 128 KiB rows, a 5.24 GB span (offsets past 2^32 bytes). The dense
    launch has 157 tiles on the chip (key-range split); the varlen launch has
    a segment starting at key row 17,001."""

    S, W, D = 40_000, 1 << 16, 128
    print(f"case: column views S={S} row stride {W}", flush=True)
    buf = torch.empty((1, S, 1, W), dtype=torch.bfloat16, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(43)
    buf[..., : 3 * D] = torch.randn((1, S, 1, 3 * D), device=DEV, generator=g).to(torch.bfloat16)
    q, k, v = buf[..., :D], buf[..., D : 2 * D], buf[..., 2 * D : 3 * D]
    assert q.stride(1) * 2 * S >= 2**32
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()

    out, lse = flash_attn_func(q, k, v)
    out_c, lse_c = flash_attn_func(qc, kc, vc)
    torch.cuda.synchronize()
    assert torch.equal(out, out_c) and torch.equal(lse, lse_c)
    _check_rows(qc, kc, vc, out, lse, torch.tensor([0, 17_000, 33_333, S - 1]), tag="dense")

    cu = torch.tensor([0, 17_001, S], dtype=torch.int32, device=DEV)
    kw = {"cu_seqlens_q": cu, "cu_seqlens_k": cu, "max_seqlen_q": S - 17_001}
    out, lse = flash_attn_func(q, k, v, **kw)
    out_c, lse_c = flash_attn_func(qc, kc, vc, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out, out_c) and torch.equal(lse, lse_c)
    _check_rows(qc, kc, vc, out, lse, torch.tensor([0, 17_000, 17_001, 30_000, S - 1]), cu=cu.cpu(), tag="varlen")


def test_short_key_views_past_2gib_token_major_v():
    """Eight heads of q, k and v as column slices of a (12,000, 8, 16,384)
    buffer: 256 KiB rows, a 3.15 GB span. Under 16,384 keys the kernel reads
    V token-major (no d-major copy), so this is the wide form's other V
    layout; 376 tiles: one whole round on the chip, the rest as key-range
    pieces from the counter."""

    S, H, W, D = 12_000, 8, 1 << 14, 128
    print(f"case: token-major V column views S={S} H={H} row stride {H * W}", flush=True)
    buf = torch.empty((1, S, H, W), dtype=torch.bfloat16, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(47)
    buf[..., : 3 * D] = torch.randn((1, S, H, 3 * D), device=DEV, generator=g).to(torch.bfloat16)
    q, k, v = buf[..., :D], buf[..., D : 2 * D], buf[..., 2 * D : 3 * D]
    assert q.stride(1) * 2 * S >= 2**31
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    out, lse = flash_attn_func(q, k, v)
    out_c, lse_c = flash_attn_func(qc, kc, vc)
    torch.cuda.synchronize()
    assert torch.equal(out, out_c) and torch.equal(lse, lse_c)
    del buf, q, k, v
    _check_rows(qc, kc, vc, out, lse, torch.tensor([0, 255, 256, 6_000, S - 33, S - 1]), tag="token-major V")


@pytest.mark.parametrize(
    "S, H, W",
    [(40_000, 1, 1 << 16), (12_000, 8, 1 << 14)],
    ids=["d-major-V-5GB-rows", "token-major-V-3GB-rows"],
)
def test_wide_forms_on_extreme_scores(S, H, W):
    """The softmax's offset raise and overflow recompute in the wide forms
    (whose overflow path reloads K through a resource at the tile's first
    row): random scores at softmax_scale 12, and one key 100 log2 units
    above the rest, on column views whose rows span 3 GB and more, bit-equal
    to the narrow form on contiguous copies and within the extreme-scale
    bounds of the oracle on sampled rows."""

    import numpy as np

    D = 128
    buf = torch.empty((1, S, H, W), dtype=torch.bfloat16, device=DEV)
    q, k, v = buf[..., :D], buf[..., D : 2 * D], buf[..., 2 * D : 3 * D]
    assert q.stride(1) * 2 * S >= 2**31
    g = torch.Generator(device=DEV).manual_seed(53)
    rows = torch.unique(torch.cat((torch.randperm(S, generator=torch.Generator().manual_seed(54))[:96],
                                   torch.tensor([0, 255, 256, S - 1]))))
    excess = 100.0
    far = excess / (88.5 * 1.4426950408889634)
    c = np.float32(np.float32(far) * np.float32(1.4426950408889634))
    assert abs(float(np.float32(np.float32(88.5) * c)) - excess) < 1e-3
    for mode, scale in (("random", 12.0), ("far key", far)):
        print(f"case: wide S={S} H={H} row stride {H * W} {mode}", flush=True)
        if mode == "random":
            buf[..., : 3 * D] = torch.randn((1, S, H, 3 * D), device=DEV, generator=g).to(torch.bfloat16)
        else:
            buf[..., : 2 * D] = 0
            buf[..., 0] = 1.0  # every query is e0
            buf[:, S // 3, :, D] = 88.5  # one key far above the rest
        qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
        out, lse = flash_attn_func(q, k, v, softmax_scale=scale)
        out_c, lse_c = flash_attn_func(qc, kc, vc, softmax_scale=scale)
        torch.cuda.synchronize()
        assert torch.equal(out, out_c) and torch.equal(lse, lse_c), mode
        ref_o, ref_l = sdpa_rows(qc.cpu(), kc.cpu(), vc.cpu(), rows, scale)
        idx = rows.to(DEV)
        m = error_metrics(out[:, idx].float().cpu(), ref_o)
        peak = max(ref_o.abs().max().item(), 1.0)
        l = lse[:, :, idx].double().cpu()
        lse_err = ((l - ref_l.double()).abs() - 1e-6 * ref_l.double().abs()).max().item()
        assert m["finite"], mode
        assert m["max_abs"] <= max(ATTN_MAX_ABS, 2**-6 * peak), (mode, m)
        assert lse_err <= LSE_MAX_ABS, (mode, lse_err)
        if mode == "random":
            assert m["relative_l2"] <= 4e-3 and m["cosine"] >= 0.99999, (mode, m)
        del qc, kc, vc
