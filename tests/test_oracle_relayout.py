"""Pins the relayout oracle (CPU): the permute form and the kernel-index form
of each movement agree, the simulated exchange reproduces the head shards of
benchmarks/check_packed_ulysses.py:20-62, and planted index mistakes fail."""

from __future__ import annotations

import numpy as np
import pytest

from oracle.relayout import (
    exchange_output,
    exchange_qkv,
    merge_heads_indexed,
    merge_heads_permute,
    pack_qkv_indexed,
    pack_qkv_permute,
)


def _ids(shape, offset=0):
    # every element distinct, so a misplaced value is always visible
    return (np.arange(int(np.prod(shape)), dtype=np.int64) + offset).reshape(shape)


@pytest.mark.parametrize(
    "rows, heads, head_dim, world",
    [(1, 1, 1, 1), (3, 4, 2, 2), (5, 8, 3, 4), (7, 6, 4, 3), (2, 8, 5, 8), (4, 56, 2, 8), (6, 40, 3, 8)],
)
def test_pack_forms_agree(rows, heads, head_dim, world):
    q, k, v = (_ids((rows, heads, head_dim), o) for o in (0, 10**6, 2 * 10**6))
    a = pack_qkv_permute(q, k, v, world)
    b = pack_qkv_indexed(q, k, v, world)
    assert a.shape == (world, rows, heads // world, 3 * head_dim)
    assert np.array_equal(a, b)
    # every source element appears exactly once
    assert np.array_equal(np.sort(a.reshape(-1)), np.sort(np.concatenate([q.ravel(), k.ravel(), v.ravel()])))


def test_pack_layout_closed_form():
    rows, heads, head_dim, world = 3, 6, 2, 3
    q, k, v = (_ids((rows, heads, head_dim), o) for o in (0, 1000, 2000))
    out = pack_qkv_permute(q, k, v, world)
    hl = heads // world
    for dest in range(world):
        for r in range(rows):
            for lh in range(hl):
                h = dest * hl + lh
                assert np.array_equal(out[dest, r, lh], np.concatenate([q[r, h], k[r, h], v[r, h]]))


@pytest.mark.parametrize("world, heads", [(4, 6), (3, 8), (8, 5)])
def test_pack_rejects_indivisible_heads(world, heads):
    q = _ids((2, heads, 4))
    with pytest.raises(ValueError, match=rf"heads \({heads}\) must divide Ulysses degree \({world}\)"):
        pack_qkv_permute(q, q, q, world)
    with pytest.raises(ValueError, match="must divide Ulysses degree"):
        pack_qkv_indexed(q, q, q, world)


@pytest.mark.parametrize("world, rows, hl, head_dim", [(1, 3, 2, 2), (2, 5, 1, 3), (4, 3, 2, 4), (8, 2, 7, 2)])
def test_merge_forms_agree(world, rows, hl, head_dim):
    x = _ids((world, rows, hl, head_dim))
    a = merge_heads_permute(x)
    b = merge_heads_indexed(x)
    assert a.shape == (rows, world * hl, head_dim)
    assert np.array_equal(a, b)
    for s in range(world):
        assert np.array_equal(a[:, s * hl : (s + 1) * hl], x[s])


def test_exchange_round_trip_reproduces_head_shards():
    # uneven rows per rank, as the reference's 8-rank gate uses (19 + world - rank)
    world, heads, head_dim = 4, 8, 3
    hl = heads // world
    counts = [19 + (world - r) for r in range(world)]
    full = [_ids((sum(counts), heads, head_dim), o) for o in (0, 10**6, 2 * 10**6)]
    offsets = np.concatenate([[0], np.cumsum(counts)])
    shards = [[t[offsets[r] : offsets[r + 1]] for t in full] for r in range(world)]
    send = [pack_qkv_permute(*shards[r], world) for r in range(world)]
    recv = exchange_qkv(send)
    for r in range(world):
        assert recv[r].shape == (sum(counts), hl, 3 * head_dim)
        for i in range(3):
            assert np.array_equal(recv[r][..., i * head_dim : (i + 1) * head_dim], full[i][:, r * hl : (r + 1) * hl])
    # output path: each rank's "attention" returns its q slot; after the
    # output exchange and merge, rank s holds q of its own rows, all heads
    outputs = [recv[r][..., :head_dim] for r in range(world)]
    back = exchange_output(outputs, counts)
    for s in range(world):
        assert np.array_equal(merge_heads_permute(back[s]), shards[s][0])


def _pack_swapped(q, k, v, world):
    # planted mistake: destination and local head swapped in the index math
    rows, heads, head_dim = q.shape
    hl = heads // world
    out = np.empty((world, rows, hl, 3 * head_dim), dtype=q.dtype)
    for dest in range(world):
        for r in range(rows):
            for lh in range(hl):
                h = lh * world + dest
                out[dest, r, lh] = np.concatenate([q[r, h], k[r, h], v[r, h]])
    return out


def _merge_transposed(x):
    # planted mistake: rows taken in source-major order
    world, rows, hl, head_dim = x.shape
    return x.reshape(rows, world * hl, head_dim)


def test_planted_mistakes_are_caught():
    q, k, v = (_ids((3, 8, 2), o) for o in (0, 1000, 2000))
    assert not np.array_equal(_pack_swapped(q, k, v, 4), pack_qkv_indexed(q, k, v, 4))
    x = _ids((4, 3, 2, 2))
    assert not np.array_equal(_merge_transposed(x), merge_heads_indexed(x))
