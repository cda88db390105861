"""Seeded sweep of the attention kernel over random shapes against the
oracle: batch, heads, query and key lengths (1 to 1,500, so partial tiles
and every split-tail decision occur), softmax scales, strided views (packed
q|k|v rows, padded head dimensions) and packed varlen segmentations with
empty segments. Same tolerance as the other attention tests."""

from __future__ import annotations

import math
import random

import pytest
import torch

from h3_flash_amd import flash_attn_func
from oracle.attention import sdpa_reference
from tests.test_gpu_attention import assert_parity

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
D = 128


def _case(i: int) -> dict:
    rng = random.Random(7000 + i)
    kind = rng.choice(["dense", "dense", "cross", "varlen"])
    B = rng.choice([1, 2, 3]) if kind != "varlen" else 1
    Sq = rng.randint(1, 1500)
    Sk = rng.randint(1, 1500) if kind == "cross" else Sq
    return {
        "kind": kind,
        "B": B,
        "H": rng.randint(1, 6),
        "Sq": Sq,
        "Sk": Sk,
        "scale": rng.choice([None, 0.05, 0.2, 1 / math.sqrt(D)]),
        "layout": rng.choice(["contiguous", "padded_heads"] + (["packed_qkv"] if Sq == Sk else [])),
        "split_tail": rng.choice([True, False]),
        "seed": rng.randrange(1 << 30),
    }


CASES = [_case(i) for i in range(40)]


def _tensors(c):
    g = torch.Generator().manual_seed(c["seed"])
    B, H, Sq, Sk = c["B"], c["H"], c["Sq"], c["Sk"]
    if c["layout"] == "packed_qkv":
        base = torch.randn((B, Sq, 3, H, D), generator=g).to(torch.bfloat16).to(DEV)
        return base[:, :, 0], base[:, :, 1], base[:, :, 2]
    if c["layout"] == "padded_heads":
        pad = lambda S: torch.randn((B, S, H + 2, D), generator=g).to(torch.bfloat16).to(DEV)[:, :, 1 : H + 1]
        return pad(Sq), pad(Sk), pad(Sk)
    mk = lambda S: torch.randn((B, S, H, D), generator=g).to(torch.bfloat16).to(DEV)
    return mk(Sq), mk(Sk), mk(Sk)


def _segments(S, seed):
    rng = random.Random(seed)
    cuts = sorted(rng.randint(0, S) for _ in range(rng.randint(1, 5)))
    return torch.tensor([0, *cuts, S], dtype=torch.int32)


@pytest.mark.parametrize("c", CASES, ids=[f"{i}-{c['kind']}-{c['layout']}" for i, c in enumerate(CASES)])
def test_random_shapes_against_oracle(c):
    q, k, v = _tensors(c)
    kw = {"softmax_scale": c["scale"], "split_tail": c["split_tail"]}
    cu = None
    if c["kind"] == "varlen":
        cu = _segments(c["Sq"], c["seed"])
        kw.update(cu_seqlens_q=cu.to(DEV), cu_seqlens_k=cu.to(DEV))
    out, lse = flash_attn_func(q, k, v, **kw)
    torch.cuda.synchronize()
    ref_out, ref_lse = sdpa_reference(q.cpu(), k.cpu(), v.cpu(), scale=c["scale"], cu_seqlens=cu)
    assert_parity(out.cpu(), lse.cpu(), ref_out, ref_lse, str(c))
