"""The softmax's rare paths in the production form of the kernel.

Sequences of 16,384 keys or more read V from the d-major copy, with the K
rows of every 16-key group in the bit-swapped order that form needs; the
masking of a ragged last key tile, the power-of-two raise of the softmax
offset and the recompute of a tile whose exp2 overflows all index keys
through that order. Normalised inputs (the C2-C5 workloads) rarely reach
those paths, and the tests that drive them on purpose elsewhere use
shorter sequences (the token-major form). Here they run at 16,411 keys and
4 heads: 260 query tiles, so one whole round on a 256-CU part and a
dynamic tail of graded key-range pieces (3/8, 3/8, 1/8, 1/8 of 257 key
tiles), with a ragged last query tile and a ragged last key tile. Both the
split launch (d-major V) and whole tiles without a workspace (token-major
V) are checked against the CPU oracle on seeded query rows, with the bounds
of the shorter extreme-scale tests.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from h3_flash_amd import flash_attn_func
from oracle.attention import sdpa_rows
from oracle.metrics import ATTN_MAX_ABS, ATTN_MEAN_ABS, LSE_MAX_ABS, error_metrics

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
S, H, D = 16_411, 4, 128


def _rand(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16)


def _rows(seed: int) -> torch.Tensor:
    """Seeded rows plus the edges: first and last rows of a tile, rows of
    the ragged last query tile (head 3's last tiles are tail pieces)."""

    g = torch.Generator().manual_seed(seed)
    pick = torch.randperm(S, generator=g)[:160]
    edges = torch.tensor([0, 255, 256, 15_615, 15_616, 16_128, S - 2, S - 1])
    return torch.unique(torch.cat((pick, edges)))


def test_the_launch_takes_the_d_major_form_and_the_tail():
    # the workspace this shape asks for on a 256-CU part: the dynamic tail's
    # 4 x 4 pieces of 256 rows (bf16 O, fp32 LSE) and counter, then the
    # d-major V (128 rows of 16,448 keys per head)
    import ctypes

    from h3_flash_amd import _ext

    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the plan is stated for a 256-CU part")
    a = _ext.AttnArgs()
    a.abi_version = _ext.ABI_VERSION
    a.q = a.k = a.v = a.o = 1 << 20
    a.batch, a.heads, a.seqlen_q, a.seqlen_k, a.head_dim = 1, H, S, S, D
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        getattr(a, name)[:] = (S * H * D, H * D, D)
    a.lse_stride[:] = (H * S, S)
    a.softmax_scale = 0.088
    split = 4 * 4 * 256 * (128 * 2 + 4) + 256
    vt = H * 128 * ((S + 63) // 64 * 64) * 2
    assert _ext.load_library().h3a_attn_fwd_workspace_size(ctypes.byref(a)) == (split + 255) // 256 * 256 + vt


@pytest.mark.parametrize("scale", [2.0, 12.0, 60.0])
def test_extreme_scales_on_random_data(scale):
    q, k, v = (_rand((1, S, H, D), 120 + i) for i in range(3))
    rows = _rows(int(scale * 10))
    ref_o, ref_l = sdpa_rows(q, k, v, rows, scale)
    peak = max(ref_o.abs().max().item(), 1.0)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    for split in (True, False):
        print(f"case: S={S} H={H} scale={scale} split_tail={split}", flush=True)
        out, lse = flash_attn_func(qd, kd, vd, softmax_scale=scale, split_tail=split)
        torch.cuda.synchronize()
        idx = rows.to(DEV)
        m = error_metrics(out[:, idx].float().cpu(), ref_o)
        l = lse[:, :, idx].double().cpu()
        lse_err = ((l - ref_l.double()).abs() - 1e-6 * ref_l.double().abs()).max().item()
        tag = (scale, split)
        assert m["finite"], tag
        assert m["max_abs"] <= max(ATTN_MAX_ABS, 2**-6 * peak), (tag, m)
        assert m["relative_l2"] <= 4e-3 and m["cosine"] >= 0.99999, (tag, m)
        assert lse_err <= LSE_MAX_ABS, (tag, lse_err)


@pytest.mark.parametrize("excess", [63.5, 100.0, 127.9986, 140.0])
def test_one_key_far_above_the_rest(excess):
    # Every query is e0; every key is zero except key pos = 88.5 * e0, which
    # scores fl32(88.5 * c) = `excess` log2 units above the others (c =
    # fl32(scale * log2 e), as the library computes it): 63.5 takes the
    # power-of-two raise of the offset, 100 and up the recompute against the
    # tile's exact max, 127.9986 a p finite in fp32 that rounds to inf in
    # bf16, 140 an fp32 overflow. The key sits in a middle key tile (inside
    # the second graded piece of a tail tile) or in the ragged last one.
    scale = excess / (88.5 * 1.4426950408889634)
    c = np.float32(np.float32(scale) * np.float32(1.4426950408889634))
    assert abs(float(np.float32(np.float32(88.5) * c)) - excess) < 1e-3
    q = torch.zeros((1, S, H, D), dtype=torch.bfloat16)
    q[..., 0] = 1.0
    v = _rand((1, S, H, D), 131)
    qd, vd = q.to(DEV), v.to(DEV)
    for pos in (9_000, S - 3):
        k = torch.zeros((1, S, H, D), dtype=torch.bfloat16)
        k[0, pos, :, 0] = 88.5
        ref_o, ref_l = sdpa_rows(q, k, v, torch.tensor([0]), scale)  # every row is the same
        peak = max(ref_o.abs().max().item(), 1.0)
        kd = k.to(DEV)
        for split in (True, False):
            print(f"case: excess={excess} pos={pos} split_tail={split}", flush=True)
            out, lse = flash_attn_func(qd, kd, vd, softmax_scale=scale, split_tail=split)
            torch.cuda.synchronize()
            o = out.float().cpu()
            m = error_metrics(o, ref_o.expand(1, S, H, D))
            lse_err = (lse.double().cpu() - ref_l.double().expand(1, H, S)).abs().max().item()
            tag = (excess, pos, split)
            assert m["finite"], tag
            assert m["max_abs"] <= max(ATTN_MAX_ABS, 2**-7 * peak), (tag, m)
            assert lse_err <= LSE_MAX_ABS, (tag, lse_err)


@pytest.mark.parametrize("mode", ["random scale 12", "far key"])
def test_planned_varlen_on_extreme_scores(mode):
    """The planned packed launch in the d-major V form (segments of 20,000
    and 5,000 rows at 4 heads: the device-built work list, a dynamic tail of
    key-range pieces for the long segment's last-round tiles, the short
    segment's V at its padded offset in the d-major copy) on random scores
    at softmax_scale 12, and with one key 100 log2 units above the rest in
    each segment (the overflow recompute reloads K from the segment's own
    rows), against the oracle on sampled rows of both segments."""

    lens = (20_000, 5_000)
    St = sum(lens)
    cu = torch.tensor([0, lens[0], St], dtype=torch.int32)
    if mode == "random scale 12":
        scale = 12.0
        q, k, v = (_rand((1, St, H, D), 140 + i) for i in range(3))
    else:
        scale = 100.0 / (88.5 * 1.4426950408889634)
        q = torch.zeros((1, St, H, D), dtype=torch.bfloat16)
        q[..., 0] = 1.0
        k = torch.zeros((1, St, H, D), dtype=torch.bfloat16)
        k[0, 7_777, :, 0] = 88.5  # segment 0, a middle key tile
        k[0, lens[0] + 3_001, :, 0] = 88.5  # segment 1
        v = _rand((1, St, H, D), 143)
    g = torch.Generator().manual_seed(144)
    rows = torch.unique(torch.cat((torch.randperm(St, generator=g)[:160],
                                   torch.tensor([0, lens[0] - 1, lens[0], lens[0] + 255, St - 1]))))
    ref_o, ref_l = sdpa_rows(q, k, v, rows, scale, cu_seqlens=cu)
    peak = max(ref_o.abs().max().item(), 1.0)
    kw = dict(cu_seqlens_q=cu.to(DEV), cu_seqlens_k=cu.to(DEV), max_seqlen_q=max(lens), softmax_scale=scale)
    print(f"case: planned varlen {lens} H={H} {mode}", flush=True)
    out, lse = flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), **kw)
    torch.cuda.synchronize()
    idx = rows.to(DEV)
    m = error_metrics(out[:, idx].float().cpu(), ref_o)
    l = lse[:, :, idx].double().cpu()
    lse_err = ((l - ref_l.double()).abs() - 1e-6 * ref_l.double().abs()).max().item()
    assert m["finite"], mode
    assert m["max_abs"] <= max(ATTN_MAX_ABS, 2**-6 * peak), (mode, m)
    assert lse_err <= LSE_MAX_ABS, (mode, lse_err)
    if mode == "random scale 12":
        assert m["relative_l2"] <= 4e-3 and m["cosine"] >= 0.99999, (mode, m)


@pytest.mark.parametrize(
    "B, Sq, Sk, Hh",
    [(2, 300, 17_000, 3), (1, 5_000, 16_500, 2), (2, 16_448, 16_448, 2)],
    ids=["cross-batch2", "cross-longer-keys", "self-batch2"],
)
def test_d_major_form_cross_and_batched(B, Sq, Sk, Hh):
    """The d-major V copy per (batch, head) block (batch stride heads x 128
    rows) and its key padding when the query and key lengths differ: batch 2,
    few query tiles against 17,000 keys (statically split pieces), and batch
    2 of 16,448 rows (a dynamic tail), against the oracle on sampled rows,
    with whole tiles on V as given (no workspace) alongside."""

    q = _rand((B, Sq, Hh, D), 150)
    k = _rand((B, Sk, Hh, D), 151)
    v = _rand((B, Sk, Hh, D), 152)
    g = torch.Generator().manual_seed(153)
    rows = torch.unique(torch.cat((torch.randperm(Sq, generator=g)[:128], torch.tensor([0, Sq - 1]))))
    ref_o, ref_l = sdpa_rows(q, k, v, rows)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    for split in (True, False):
        print(f"case: B={B} Sq={Sq} Sk={Sk} H={Hh} split_tail={split}", flush=True)
        out, lse = flash_attn_func(qd, kd, vd, split_tail=split)
        torch.cuda.synchronize()
        idx = rows.to(DEV)
        m = error_metrics(out[:, idx].float().cpu(), ref_o)
        lse_err = (lse[:, :, idx].double().cpu() - ref_l.double()).abs().max().item()
        tag = (B, Sq, Sk, Hh, split)
        assert m["finite"] and m["max_abs"] <= ATTN_MAX_ABS and m["mean_abs"] <= ATTN_MEAN_ABS, (tag, m)
        assert lse_err <= LSE_MAX_ABS, (tag, lse_err)
