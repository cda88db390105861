"""GPU parity of the packed-Ulysses relayouts (through the C ABI).

Movement is bit-exact: every output is compared with the oracle's on the raw
bits. The fused prologue + pack is bit-identical to the unfused HIP launches
(same arithmetic) and within the prologue's rounding bar of the fp32 oracle.
The single-GPU Ulysses simulation mirrors the equality gate of
benchmarks/check_packed_ulysses.py:65-140: exchanged q/k/v and the merged
attention output are bit-identical to the plain head-sliced path.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from h3_flash_amd import flash_attn_func
from h3_flash_amd.prologue import fused_qk_norm_rope
from h3_flash_amd.relayout import (
    can_pack_qkv,
    merge_heads,
    pack_qkv_destination_major,
    packed_qkv_attention,
    qknorm_rope_pack_qkv,
)
from h3_flash_amd.rope import rope_3d_tables
from oracle.qknorm_rope import qknorm_rope_reference
from oracle.relayout import merge_heads_permute, pack_qkv_permute
from tests.test_gpu_prologue import assert_rounding_parity

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

_BITS = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(_BITS[t.element_size()]).cpu().numpy()


def _random(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    size = torch.empty((), dtype=dtype).element_size()
    raw = torch.randint(-(2**15), 2**15, shape, generator=g, dtype=torch.int32)
    if size == 1:
        return (raw & 0xFF).to(torch.uint8).view(dtype)
    if size == 2:
        return raw.to(torch.int16).view(dtype)
    if size == 4:
        return (raw * 65599 + 7).view(dtype)
    return (raw.to(torch.int64) * 1_000_003 + 11).view(dtype)


@pytest.mark.parametrize(
    "rows, heads, head_dim, world, dtype",
    [
        (1, 1, 128, 1, torch.bfloat16),
        (37, 8, 128, 2, torch.bfloat16),
        (25, 56, 128, 8, torch.bfloat16),
        (6240, 40, 128, 8, torch.bfloat16),
        (13, 6, 96, 3, torch.bfloat16),
        (9, 4, 3, 2, torch.bfloat16),  # 6-byte rows: byte path
        (11, 8, 64, 4, torch.float32),
        (7, 4, 16, 2, torch.uint8),
        (5, 6, 32, 3, torch.float64),
        # wide rows: lane groups of 128 and 256 lanes
        (6, 4, 1024, 4, torch.bfloat16),
        (5, 4, 2048, 2, torch.bfloat16),
        (3, 2, 512, 2, torch.float32),
    ],
)
def test_pack_bit_exact(rows, heads, head_dim, world, dtype):
    q, k, v = (_random((rows, heads, head_dim), dtype, s) for s in (1, 2, 3))
    out = pack_qkv_destination_major(q.to(DEV), k.to(DEV), v.to(DEV), world)
    torch.cuda.synchronize()
    expect = pack_qkv_permute(_bits(q), _bits(k), _bits(v), world)
    assert out.shape == (world, rows, heads // world, 3 * head_dim)
    assert np.array_equal(_bits(out), expect)


def test_pack_strided_views():
    rows, heads, D, world = 53, 16, 128, 4
    # q, k, v as views of a fused projection output (rows, 3, heads, D)
    fused = _random((rows, 3, heads, D), torch.bfloat16, 5).to(DEV)
    q, k, v = fused[:, 0], fused[:, 1], fused[:, 2]
    out = pack_qkv_destination_major(q, k, v, world)
    expect = pack_qkv_permute(_bits(q), _bits(k), _bits(v), world)
    assert np.array_equal(_bits(out), expect)
    # head stride 2D and a row stride that is not a 16-byte multiple (byte path)
    wide = _random((rows, heads * 2 * D + 4), torch.bfloat16, 6).to(DEV)
    x = wide[:, : heads * 2 * D].view(rows, heads, 2 * D)[..., :D]
    assert x.stride() == (heads * 2 * D + 4, 2 * D, 1)
    out = pack_qkv_destination_major(x, q, x, world)
    assert np.array_equal(_bits(out), pack_qkv_permute(_bits(x), _bits(q), _bits(x), world))


def test_pack_errors_and_predicate():
    q = torch.zeros((4, 6, 128), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match=r"heads \(6\) must divide Ulysses degree \(4\)"):
        pack_qkv_destination_major(q, q, q, 4)
    assert can_pack_qkv(q, q, q)
    assert not can_pack_qkv(q, q, q.float())
    assert not can_pack_qkv(q, q, q.transpose(1, 2).contiguous().transpose(1, 2))
    assert not can_pack_qkv(q.cpu(), q.cpu(), q.cpu())
    with pytest.raises(ValueError):
        pack_qkv_destination_major(q, q, q[:2], 2)
    empty = torch.zeros((0, 8, 128), dtype=torch.bfloat16, device=DEV)
    assert pack_qkv_destination_major(empty, empty, empty, 4).shape == (4, 0, 2, 384)


@pytest.mark.parametrize(
    "world, rows, hl, head_dim, dtype",
    [
        (1, 9, 3, 128, torch.bfloat16),
        (8, 6240, 5, 128, torch.bfloat16),
        (4, 23, 14, 128, torch.bfloat16),
        (3, 7, 2, 3, torch.bfloat16),  # byte path
        (2, 17, 4, 32, torch.float32),
    ],
)
def test_merge_bit_exact(world, rows, hl, head_dim, dtype):
    x = _random((world, rows, hl, head_dim), dtype, world + rows)
    out = merge_heads(x.to(DEV))
    assert out.shape == (rows, world * hl, head_dim)
    assert np.array_equal(_bits(out), merge_heads_permute(_bits(x)))


def test_merge_strided_input():
    world, rows, hl, D = 4, 19, 5, 128
    big = _random((world, rows + 7, hl, D), torch.bfloat16, 9).to(DEV)
    x = big[:, 3 : 3 + rows]  # row stride unchanged, world stride larger than rows * inner
    out = merge_heads(x)
    assert np.array_equal(_bits(out), merge_heads_permute(_bits(x)))
    # non-contiguous inner block: made contiguous first, same values
    y = _random((world, rows, D, hl), torch.bfloat16, 10).to(DEV).transpose(2, 3)
    assert y.stride(3) != 1
    assert np.array_equal(_bits(merge_heads(y)), merge_heads_permute(_bits(y)))


@pytest.mark.parametrize("R", [128, 96, 0, 42, 126, 2])
@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("heads, world", [(40, 8), (6, 3), (7, 7)])  # whole and partial head chunks
def test_fused_prologue_pack_equals_unfused(R, wdtype, heads, world):
    rows, D = 211, 128
    fused = (torch.randn((rows, 3, heads, D), generator=torch.Generator().manual_seed(R)) * 1.5).to(torch.bfloat16)
    fused = fused.to(DEV)
    q, k, v = fused[:, 0], fused[:, 1], fused[:, 2]
    g = torch.Generator().manual_seed(100 + R)
    wq = (1 + 0.1 * torch.randn(D, generator=g)).to(wdtype)
    wk = (1 + 0.1 * torch.randn(D, generator=g)).to(wdtype)
    ang = torch.randn((rows, R), generator=g)
    cos, sin = ang.cos(), ang.sin()
    tc, ts = cos, sin
    if R == 96:
        # device tables with rows of 98 floats (not 16-byte rows), read in
        # place: the element-wise kernel in the pack layout
        tc, ts = torch.zeros((rows, 98), device=DEV), torch.zeros((rows, 98), device=DEV)
        tc[:, :R], ts[:, :R] = cos.to(DEV), sin.to(DEV)
        tc, ts = tc[:, :R], ts[:, :R]
        assert tc.stride(0) == 98
    packed = qknorm_rope_pack_qkv(q, k, v, wq, wk, tc, ts, 1e-5, 1e-6, world)
    qn, kn = fused_qk_norm_rope(
        q.unsqueeze(0), k.unsqueeze(0), wq.to(DEV), wk.to(DEV), cos.to(DEV), sin.to(DEV), 1e-5, 1e-6
    )
    unfused = pack_qkv_destination_major(qn.squeeze(0), kn.squeeze(0), v, world)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(packed), _bits(unfused))
    # and against the fp32 oracle: q/k slots within the prologue bar, v slot exact
    rq = qknorm_rope_reference(q.cpu().unsqueeze(0), wq, cos, sin, 1e-5).squeeze(0)
    rk = qknorm_rope_reference(k.cpu().unsqueeze(0), wk, cos, sin, 1e-6).squeeze(0)
    hl = heads // world
    got = packed.cpu()
    for dest in range(world):
        sl = slice(dest * hl, (dest + 1) * hl)
        assert_rounding_parity(got[dest, :, :, :D], rq[:, sl], f"q{dest}")
        assert_rounding_parity(got[dest, :, :, D : 2 * D], rk[:, sl], f"k{dest}")
        assert torch.equal(got[dest, :, :, 2 * D :].view(torch.int16), v[:, sl].cpu().view(torch.int16))


@pytest.mark.parametrize("world, heads, base_rows", [(4, 8, 19), (8, 40, 1560)])
def test_single_gpu_ulysses_equality_gate(world, heads, base_rows):
    """Per-rank prologue + pack, simulated all-to-all, attention on the
    exchanged buffer, output exchange and merge: bit-identical to the
    head-sliced path on the full sequence."""

    D = 128
    hl = heads // world
    counts = [base_rows + (world - r) for r in range(world)]  # deliberately uneven
    S = sum(counts)
    offs = np.concatenate([[0], np.cumsum(counts)])
    g = torch.Generator().manual_seed(world * 1000 + heads)
    raw = [torch.randn((S, heads, D), generator=g).to(torch.bfloat16).to(DEV) for _ in range(3)]
    w = torch.ones(D, dtype=torch.bfloat16, device=DEV)
    cos, sin = rope_3d_tables((1, 1, S))
    cos, sin = cos.to(DEV), sin.to(DEV)

    # each rank: its rows, all heads -> destination-major send buffer
    send = [
        qknorm_rope_pack_qkv(
            *(t[offs[r] : offs[r + 1]] for t in raw), w, w, cos[offs[r] : offs[r + 1]], sin[offs[r] : offs[r + 1]],
            1e-5, 1e-5, world,
        )
        for r in range(world)
    ]
    recv = [torch.cat([send[src][dst] for src in range(world)], dim=0) for dst in range(world)]
    outs = [packed_qkv_attention(recv[r])[0] for r in range(world)]
    merged = [merge_heads(torch.stack([outs[r][offs[s] : offs[s + 1]] for r in range(world)], 0)) for s in range(world)]

    # reference: prologue on the full sequence, attention per head shard
    qn, kn = fused_qk_norm_rope(raw[0].unsqueeze(0), raw[1].unsqueeze(0), w, w, cos, sin, 1e-5, 1e-5)
    full_out = torch.empty((S, heads, D), dtype=torch.bfloat16, device=DEV)
    for r in range(world):
        sl = slice(r * hl, (r + 1) * hl)
        q_ref = qn[:, :, sl].contiguous()
        k_ref = kn[:, :, sl].contiguous()
        v_ref = raw[2][:, sl].unsqueeze(0).contiguous()
        assert torch.equal(recv[r][..., :D].view(torch.int16), q_ref.squeeze(0).view(torch.int16))
        assert torch.equal(recv[r][..., D : 2 * D].view(torch.int16), k_ref.squeeze(0).view(torch.int16))
        assert torch.equal(recv[r][..., 2 * D :].view(torch.int16), v_ref.squeeze(0).view(torch.int16))
        o_ref, _ = flash_attn_func(q_ref, k_ref, v_ref)
        full_out[:, sl] = o_ref.squeeze(0)
    torch.cuda.synchronize()
    for s in range(world):
        assert torch.equal(merged[s].view(torch.int16), full_out[offs[s] : offs[s + 1]].view(torch.int16)), s
