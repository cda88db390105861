"""Pins for oracle.projection.projection_reference (CPU): a float64 brute
force written from the definition, closed forms (identity weights reduce it
to the pinned q/k prologue reference; plain sections are nn.Linear), and
planted mistakes that these checks must catch."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.projection import projection_reference
from oracle.qknorm_rope import qknorm_rope_reference


def brute_fp64(x, w, b, nw, eps, cos, sin, seqlen, head_dim=128, round_projection=True):
    """Loops in float64: product, bias, (the projection rounded to bf16, as
    the linear outputs it), per-head RMSNorm, weight, rotate-half."""

    x, w = x.double().numpy(), w.double().numpy()
    m, n = x.shape[0], w.shape[0]
    acc = np.zeros((m, n))
    for i in range(m):
        for f in range(n):
            acc[i, f] = float(np.dot(x[i], w[f])) + (float(b[f]) if b is not None else 0.0)
    if nw is None:
        return acc
    if round_projection:
        acc = torch.from_numpy(acc).to(torch.bfloat16).double().numpy()
    nw = nw.double().numpy()
    R = 0 if cos is None else cos.shape[1]
    out = np.zeros_like(acc)
    for i in range(m):
        s = i % seqlen
        for h in range(n // head_dim):
            seg = acc[i, h * head_dim : (h + 1) * head_dim]
            r = 1.0 / math.sqrt(float(np.mean(seg * seg)) + eps)
            nrm = seg * r * nw
            for c in range(head_dim):
                if c < R:
                    partner = nrm[c + R // 2] if c < R // 2 else nrm[c - R // 2]
                    rot = -partner if c < R // 2 else partner
                    out[i, h * head_dim + c] = nrm[c] * float(cos[s, c]) + rot * float(sin[s, c])
                else:
                    out[i, h * head_dim + c] = nrm[c]
    return out


def bf16_ulp(v: torch.Tensor) -> torch.Tensor:
    a = v.abs().clamp_min(1e-30)
    return 2.0 ** (torch.floor(torch.log2(a)) - 7)


def rotate_half_tables(seqlen: int, R: int, seed: int = 0):
    g = torch.Generator().manual_seed(seed)
    theta = torch.rand((seqlen, R // 2), generator=g) * 6.0
    theta = torch.cat((theta, theta), dim=1)
    return theta.cos(), theta.sin()


def case(m=5, k=32, heads=2, R=64, seqlen=3, seed=0, bias=True):
    g = torch.Generator().manual_seed(seed)
    n = heads * 128
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    w = (torch.randn((n, k), generator=g) / k**0.5).to(torch.bfloat16)
    b = (0.1 * torch.randn(n, generator=g)).to(torch.bfloat16) if bias else None
    nw = (1 + 0.2 * torch.randn(128, generator=g)).to(torch.bfloat16)
    cos, sin = rotate_half_tables(seqlen, R, seed) if R else (None, None)
    return x, w, b, nw, cos, sin


def assert_within_one_ulp(got: torch.Tensor, exact: np.ndarray):
    exact_t = torch.from_numpy(exact).float()
    d = (got.float() - exact_t).abs()
    assert (d <= bf16_ulp(exact_t) + 1e-30).all(), float((d / bf16_ulp(exact_t)).max())


@pytest.mark.parametrize("R, seqlen, bias", [(64, 3, True), (128, 5, False), (0, 1, True), (32, 2, True)])
@pytest.mark.parametrize("round_projection", [True, False])
def test_matches_float64_brute_force(R, seqlen, bias, round_projection):
    x, w, b, nw, cos, sin = case(R=R, seqlen=seqlen, bias=bias)
    got = projection_reference(x, w, b, nw, 1e-6, cos, sin, seqlen, round_projection=round_projection)
    assert_within_one_ulp(got, brute_fp64(x, w, b, nw, 1e-6, cos, sin, seqlen, round_projection=round_projection))


def test_default_order_is_the_rounded_projection():
    # the default follows the reference: bf16 projection, then the prologue
    # oracle on it (transformer.py:146-173)
    x, w, b, nw, cos, sin = case(m=9, k=64, heads=2, R=64, seqlen=9, seed=3)
    proj = torch.nn.functional.linear(x.float(), w.float(), b.float()).to(torch.bfloat16)
    want = qknorm_rope_reference(proj.view(1, 9, 2, 128), nw, cos, sin, 1e-6).view(9, 256)
    assert torch.equal(projection_reference(x, w, b, nw, 1e-6, cos, sin, 9), want)


def test_plain_section_is_an_fp32_linear():
    x, w, b, _, _, _ = case(m=7, k=64, heads=1, R=0)
    got = projection_reference(x, w, b)
    want = torch.nn.functional.linear(x.float(), w.float(), b.float()).to(torch.bfloat16)
    assert torch.equal(got, want)
    assert_within_one_ulp(got, brute_fp64(x, w, b, None, 0, None, None, 1))


def test_identity_weights_reduce_to_the_prologue_reference():
    g = torch.Generator().manual_seed(3)
    m, heads, R = 6, 2, 128
    x = torch.randn((m, heads * 128), generator=g).to(torch.bfloat16)
    eye = torch.eye(heads * 128).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16)
    cos, sin = rotate_half_tables(m, R, 3)
    got = projection_reference(x, eye, None, nw, 1e-5, cos, sin, m)
    want = qknorm_rope_reference(x.view(1, m, heads, 128), nw, cos, sin, 1e-5).view(m, heads * 128)
    assert torch.equal(got, want)


def test_table_rows_wrap_per_sequence():
    # token rows of a batch of 2 sequences use table rows i % seqlen
    x, w, b, nw, cos, sin = case(m=6, R=64, seqlen=3)
    got = projection_reference(x, w, b, nw, 1e-6, cos, sin, 3)
    assert torch.equal(got[3:], projection_reference(x[3:], w, b, nw, 1e-6, cos, sin, 3))


def test_single_rounding_differs_from_the_rounded_projection_by_the_projection_rounding():
    # rounding the projection first (the reference's order) moves a
    # normalised value (RMS 1 per head) by about one bf16 step of its inputs:
    # at most one bf16 step of the largest outputs (2^-4 at |y| < 8), 2^-8 on
    # average, on a minority of elements
    x, w, b, nw, cos, sin = case(m=64, k=256, R=128, seqlen=64, seed=4)
    once = projection_reference(x, w, b, nw, 1e-6, cos, sin, 64, round_projection=False).float()
    twice = projection_reference(x, w, b, nw, 1e-6, cos, sin, 64, round_projection=True).float()
    d = (once - twice).abs()
    assert 0 < (once != twice).float().mean() < 0.5
    assert d.max() <= 2.0**-4 and d.mean() <= 2.0**-8, (float(d.max()), float(d.mean()))


@pytest.mark.parametrize("mistake", ["no_bias", "transposed_weight", "unwrapped_rows", "rotation_sign", "no_weight"])
def test_planted_mistakes_fail_the_brute_force(mistake):
    x, w, b, nw, cos, sin = case(m=6, k=128, heads=1, R=64, seqlen=4, seed=9)
    exact = brute_fp64(x, w, b, nw, 1e-6, cos, sin, 4)
    if mistake == "no_bias":
        bad = projection_reference(x, w, None, nw, 1e-6, cos, sin, 4)
    elif mistake == "transposed_weight":
        bad = projection_reference(x, w.T.contiguous(), b, nw, 1e-6, cos, sin, 4)
    elif mistake == "unwrapped_rows":
        c6 = torch.cat((cos, rotate_half_tables(2, 64, 11)[0]))
        s6 = torch.cat((sin, rotate_half_tables(2, 64, 11)[1]))
        bad = projection_reference(x, w, b, nw, 1e-6, c6, s6, 6)
    elif mistake == "rotation_sign":
        bad = projection_reference(x, w, b, nw, 1e-6, cos, -sin, 4)
    else:
        bad = projection_reference(x, w, b, torch.ones(128, dtype=torch.bfloat16), 1e-6, cos, sin, 4)
    with pytest.raises(AssertionError):
        assert_within_one_ulp(bad, exact)
