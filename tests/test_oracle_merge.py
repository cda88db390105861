"""Pins the LSE-merge oracle (CPU): merging the oracle's own attention over
disjoint key chunks reproduces attention over all keys (softmax over a union
of key ranges), parts with no keys weigh nothing, part order does not
matter, and planted mistakes fail."""

from __future__ import annotations

import pytest
import torch

from oracle.attention import merge_reference, sdpa_reference


def _qkv(B=2, S=40, Sk=53, H=3, D=16, seed=0):
    g = torch.Generator().manual_seed(seed)
    return tuple((torch.randn(shape, generator=g) * 2).to(torch.bfloat16) for shape in
                 ((B, S, H, D), (B, Sk, H, D), (B, Sk, H, D)))


@pytest.mark.parametrize("bounds", [[0, 53], [0, 20, 53], [0, 1, 2, 30, 53], [0, 13, 26, 39, 52, 53]])
def test_merge_of_key_chunks_equals_full_attention(bounds):
    q, k, v = _qkv()
    full_o, full_l = sdpa_reference(q, k, v)
    parts = [sdpa_reference(q, k[:, a:b], v[:, a:b]) for a, b in zip(bounds[:-1], bounds[1:])]
    o, l = merge_reference([p[0] for p in parts], [p[1] for p in parts])
    torch.testing.assert_close(o, full_o, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(l, full_l, rtol=1e-6, atol=1e-5)


def test_empty_parts_and_order():
    q, k, v = _qkv(seed=1)
    a = sdpa_reference(q, k[:, :30], v[:, :30])
    b = sdpa_reference(q, k[:, 30:], v[:, 30:])
    empty = (torch.randn_like(a[0]), torch.full_like(a[1], float("-inf")))
    o1, l1 = merge_reference([a[0], b[0]], [a[1], b[1]])
    o2, l2 = merge_reference([b[0], empty[0], a[0]], [b[1], empty[1], a[1]])
    torch.testing.assert_close(o1, o2, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(l1, l2, rtol=1e-6, atol=1e-6)
    o, l = merge_reference([empty[0]], [empty[1]])
    assert torch.count_nonzero(o) == 0 and torch.all(l == float("-inf"))
    o, l = merge_reference([a[0]], [a[1]])
    torch.testing.assert_close(o, a[0].float(), rtol=0, atol=0)


def test_planted_mistakes_fail():
    q, k, v = _qkv(seed=2)
    full_o, full_l = sdpa_reference(q, k, v)
    a = sdpa_reference(q, k[:, :25], v[:, :25])
    b = sdpa_reference(q, k[:, 25:], v[:, 25:])
    mean_o = (a[0] + b[0]) / 2  # plain average instead of LSE weights
    assert not torch.allclose(mean_o, full_o, rtol=1e-3, atol=1e-3)
    max_l = torch.maximum(a[1], b[1])  # max instead of logsumexp
    assert not torch.allclose(max_l, full_l, rtol=1e-3, atol=1e-3)
