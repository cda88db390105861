"""Pins the CPU oracle before it is trusted as the parity checker.

Attention (oracle.attention) is checked against an independent float64 brute
force, the golden fixtures and closed forms; the q/k RMSNorm + RoPE
restatement (oracle.qknorm_rope) against torch's rms_norm, the complex
multiplication form of rotate-half RoPE, rotation inversion and the golden
fixtures. Each check set is also run on oracles with one planted mistake,
which it must reject.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from torch.nn import functional

import oracle.attention as oa
import oracle.qknorm_rope as oq
from oracle.brute import attention_fp64
from tests._golden import bf16, f32, golden

D = 128


def _rand(shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype)


# ---------------------------------------------------------------- attention


def attention_checks(attn) -> list[str]:
    """Run every attention pin on ``attn(q, k, v, scale, cu_seqlens)``; return the failed ones."""

    failed = []

    def check(name, fn):
        try:
            fn()
        except Exception:  # an exception is a failed pin
            failed.append(name)

    def brute():
        for seed, (B, Sq, Sk, H) in enumerate([(1, 37, 37, 2), (2, 5, 70, 1), (1, 130, 9, 3)]):
            q, k, v = _rand((B, Sq, H, D), seed), _rand((B, Sk, H, D), seed + 10), _rand((B, Sk, H, D), seed + 20)
            o, l = attn(q, k, v, None, None)
            ro, rl = attention_fp64(q.numpy(), k.numpy(), v.numpy())
            assert np.abs(o.numpy() - ro).max() < 1e-5
            assert np.abs(l.numpy() - rl).max() < 1e-5

    def golden_cases():
        g = golden()
        for case in ("dense", "cross"):
            o, l = attn(bf16(f"{case}_q"), bf16(f"{case}_k"), bf16(f"{case}_v"), float(g["scale"]), None)
            assert (o - f32(f"{case}_out")).abs().max() < 1e-5
            assert (l - f32(f"{case}_lse")).abs().max() < 1e-5
        cu = torch.from_numpy(g["varlen_cu"])
        o, l = attn(bf16("dense_q"), bf16("dense_k"), bf16("dense_v"), float(g["scale"]), cu)
        assert (o - f32("varlen_out")).abs().max() < 1e-5
        assert (l - f32("varlen_lse")).abs().max() < 1e-5

    def single_key():
        q, k, v = _rand((1, 9, 2, D), 1), _rand((1, 1, 2, D), 2), _rand((1, 1, 2, D), 3)
        o, l = attn(q, k, v, None, None)
        assert torch.allclose(o, v.expand_as(o), atol=1e-6)
        dots = torch.einsum("bshd,bhd->bhs", q, k[:, 0]) / math.sqrt(D)
        assert torch.allclose(l, dots, atol=1e-5)

    def equal_keys():
        S = 50
        q, v = _rand((1, 11, 2, D), 4), _rand((1, S, 2, D), 5)
        k = _rand((1, 1, 2, D), 6).expand(1, S, 2, D).contiguous()
        o, l = attn(q, k, v, None, None)
        assert torch.allclose(o, v.mean(dim=1, keepdim=True).expand_as(o), atol=1e-5)
        dots = torch.einsum("bshd,bhd->bhs", q, k[:, 0]) / math.sqrt(D)
        assert torch.allclose(l, dots + math.log(S), atol=1e-5)

    def permutation():
        q, k, v = _rand((1, 21, 2, D), 7), _rand((1, 40, 2, D), 8), _rand((1, 40, 2, D), 9)
        perm = torch.randperm(40, generator=torch.Generator().manual_seed(0))
        o1, l1 = attn(q, k, v, None, None)
        o2, l2 = attn(q, k[:, perm], v[:, perm], None, None)
        assert torch.allclose(o1, o2, atol=1e-5) and torch.allclose(l1, l2, atol=1e-5)

    def scale_identity():
        q, k, v = _rand((1, 13, 1, D), 10), _rand((1, 30, 1, D), 11), _rand((1, 30, 1, D), 12)
        o1, l1 = attn(q, k, v, 0.3, None)
        o2, l2 = attn(q * 3.0, k, v, 0.1, None)
        assert torch.allclose(o1, o2, atol=1e-5) and torch.allclose(l1, l2, atol=1e-5)

    def varlen_concat():
        q, k, v = _rand((1, 60, 2, D), 13), _rand((1, 60, 2, D), 14), _rand((1, 60, 2, D), 15)
        cu = torch.tensor([0, 7, 7, 41, 60], dtype=torch.int32)
        o, l = attn(q, k, v, None, cu)
        for a, e in [(0, 7), (7, 41), (41, 60)]:
            so, sl = attn(q[:, a:e], k[:, a:e], v[:, a:e], None, None)
            assert torch.allclose(o[:, a:e], so, atol=1e-6) and torch.allclose(l[:, :, a:e], sl, atol=1e-6)

    def large_logits_finite():
        q, k, v = _rand((1, 8, 1, D), 16) * 60.0, _rand((1, 20, 1, D), 17) * 60.0, _rand((1, 20, 1, D), 18)
        o, l = attn(q, k, v, None, None)
        assert torch.isfinite(o).all() and torch.isfinite(l).all()
        ro, rl = attention_fp64(q.numpy(), k.numpy(), v.numpy())
        assert np.abs(o.numpy() - ro).max() < 1e-4

    for name, fn in [
        ("brute", brute),
        ("golden", golden_cases),
        ("single_key", single_key),
        ("equal_keys", equal_keys),
        ("permutation", permutation),
        ("scale_identity", scale_identity),
        ("varlen_concat", varlen_concat),
        ("large_logits_finite", large_logits_finite),
    ]:
        check(name, fn)
    return failed


def _oracle(q, k, v, scale, cu):
    return oa.sdpa_reference(q, k, v, scale, cu_seqlens=cu, chunk=16)


def test_attention_oracle_passes_every_pin():
    assert attention_checks(_oracle) == []


def test_brute_force_rows_are_stochastic():
    q, k = _rand((1, 9, 1, D), 1), _rand((1, 31, 1, D), 2)
    v = torch.ones((1, 31, 1, D))
    o, _ = attention_fp64(q.numpy(), k.numpy(), v.numpy())
    assert np.allclose(o, 1.0, atol=1e-12)


def test_row_sampling_matches_full_result():
    q, k, v = _rand((1, 50, 2, D), 3), _rand((1, 50, 2, D), 4), _rand((1, 50, 2, D), 5)
    cu = torch.tensor([0, 20, 50], dtype=torch.int32)
    rows = torch.tensor([0, 19, 20, 33, 49])
    for c in (None, cu):
        full_o, full_l = oa.sdpa_reference(q, k, v, cu_seqlens=c)
        so, sl = oa.sdpa_rows(q, k, v, rows, cu_seqlens=c)
        assert torch.allclose(so, full_o[:, rows], atol=1e-6)
        assert torch.allclose(sl, full_l[:, :, rows], atol=1e-6)


# Planted mistakes: each replaces the oracle's per-sequence kernel with a
# variant carrying one plausible error; the pins above must reject each one.


def _m_lse_unscaled(q, k, v, scale, chunk):
    o, _ = _ORIG_DENSE(q, k, v, scale, chunk)
    _, l = _ORIG_DENSE(q, k, v, 1.0, chunk)
    return o, l


def _m_lse_log2(q, k, v, scale, chunk):
    o, l = _ORIG_DENSE(q, k, v, scale, chunk)
    return o, l / math.log(2.0)


def _m_scale_sqrt_missing(q, k, v, scale, chunk):
    return _ORIG_DENSE(q, k, v, scale * scale * math.sqrt(q.shape[-1]), chunk)


def _m_values_are_keys(q, k, v, scale, chunk):
    return _ORIG_DENSE(q, k, k, scale, chunk)


def _m_softmax_wrong_axis(q, k, v, scale, chunk):
    qt, kt, vt = (x.transpose(0, 1) for x in (q, k, v))
    s = torch.matmul(qt, kt.transpose(-1, -2)) * scale
    p = torch.softmax(s, dim=-2)  # normalises over queries instead of keys
    return torch.matmul(p, vt).transpose(0, 1), torch.logsumexp(s, dim=-1)


def _m_no_max_subtraction(q, k, v, scale, chunk):
    qt, kt, vt = (x.transpose(0, 1) for x in (q, k, v))
    s = torch.matmul(qt, kt.transpose(-1, -2)) * scale
    e = torch.exp(s)
    z = e.sum(-1, keepdim=True)
    return torch.matmul(e / z, vt).transpose(0, 1), torch.log(z[..., 0])


def _m_drops_last_row(q, k, v, scale, chunk):
    o, l = _ORIG_DENSE(q, k[:-1] if k.shape[0] > 1 else k, v[:-1] if v.shape[0] > 1 else v, scale, chunk)
    return o, l


_ORIG_DENSE = oa._dense


@pytest.mark.parametrize(
    "mutant",
    [
        _m_lse_unscaled,
        _m_lse_log2,
        _m_scale_sqrt_missing,
        _m_values_are_keys,
        _m_softmax_wrong_axis,
        _m_no_max_subtraction,
        _m_drops_last_row,
    ],
    ids=lambda f: f.__name__,
)
def test_planted_attention_mistakes_are_caught(mutant, monkeypatch):
    monkeypatch.setattr(oa, "_dense", mutant)
    assert attention_checks(_oracle) != []


# ---------------------------------------------------------------- q/k norm + RoPE


def rope_checks(fn) -> list[str]:
    failed = []

    def check(name, f):
        try:
            f()
        except Exception:
            failed.append(name)

    def rmsnorm_only():
        x = _rand((2, 5, 3, D), 20, torch.bfloat16)
        w = _rand((D,), 21)
        cos = torch.empty((5, 0))
        y = fn(x, w, cos, cos, 1e-5, None)
        ref = functional.rms_norm(x.float(), (D,), w, 1e-5)
        assert torch.allclose(y, ref, atol=1e-5, rtol=1e-5)

    def complex_form():
        S, H, R = 7, 2, 96
        x = _rand((1, S, H, D), 22, torch.bfloat16)
        w = _rand((D,), 23)
        theta = _rand((S, R // 2), 24) * 3
        full = torch.cat((theta, theta), dim=-1)
        y = fn(x, w, full.cos(), full.sin(), 1e-6, None)
        n = functional.rms_norm(x.float(), (D,), w, 1e-6).double()
        z = torch.complex(n[..., : R // 2], n[..., R // 2 : R]) * torch.polar(
            torch.ones_like(theta, dtype=torch.float64), theta.double()
        ).view(1, S, 1, R // 2)
        expect = torch.cat((z.real, z.imag, n[..., R:]), dim=-1)
        assert torch.allclose(y.double(), expect, atol=2e-5)

    def inversion():
        S, H = 6, 2
        x = _rand((1, S, H, D), 25, torch.bfloat16)
        w = torch.ones(D)
        theta = _rand((S, D // 2), 26)
        full = torch.cat((theta, theta), dim=-1)
        y = fn(x, w, full.cos(), full.sin(), 0.0, None)
        back = fn(y, w, (-full).cos(), (-full).sin(), 0.0, None)
        assert torch.allclose(back, functional.rms_norm(x.float(), (D,), None, 0.0), atol=1e-5)

    def golden_tables():
        g = golden()
        x, w = bf16("rope_x"), bf16("rope_w")
        for R in (96, 128):
            y = fn(x, w, f32(f"rope{R}_cos"), f32(f"rope{R}_sin"), float(g["rope_eps"]), None)
            assert (y - f32(f"rope{R}_out")).abs().max() < 1e-4

    for name, f in [
        ("rmsnorm_only", rmsnorm_only),
        ("complex_form", complex_form),
        ("inversion", inversion),
        ("golden_tables", golden_tables),
    ]:
        check(name, f)
    return failed


def test_qknorm_rope_oracle_passes_every_pin():
    assert rope_checks(oq.qknorm_rope_reference) == []


def test_qknorm_rope_oracle_rejects_bad_rotary_dim():
    x = torch.zeros((1, 2, 1, 8))
    with pytest.raises(ValueError, match="even rotary dimension"):
        oq.qknorm_rope_reference(x, torch.ones(8), torch.zeros((2, 3)), torch.zeros((2, 3)), 1e-5)
    with pytest.raises(ValueError, match="even rotary dimension"):
        oq.qknorm_rope_reference(x, torch.ones(8), torch.zeros((2, 10)), torch.zeros((2, 10)), 1e-5)


def _rope_mutant(kind):
    def fn(x, weight, cos, sin, eps, out_dtype=torch.bfloat16):
        B, S, H, Dh = x.shape
        R = cos.shape[-1]
        value = x.float()
        w = weight.float()
        if kind == "variance_sum":
            variance = (value * value).sum(-1, keepdim=True)
        else:
            variance = (value * value).sum(-1, keepdim=True) / Dh
        if kind == "eps_outside":
            normed = value * (torch.rsqrt(variance) + eps) * w
        elif kind == "no_weight":
            normed = value * torch.rsqrt(variance + eps)
        else:
            normed = value * torch.rsqrt(variance + eps) * w
        out = normed.clone()
        RR = Dh if kind == "full_width" else R
        if RR > 0:
            half = RR // 2
            c = cos.float()
            s = sin.float()
            if kind == "full_width" and R < Dh:
                c = torch.cat((c, torch.ones(S, Dh - R)), dim=-1)
                s = torch.cat((s, torch.zeros(S, Dh - R)), dim=-1)
            c, s = c.view(1, S, 1, RR), s.view(1, S, 1, RR)
            if kind == "sign_flip":
                rotated = torch.cat((normed[..., half:RR], -normed[..., :half]), dim=-1)
            else:
                rotated = torch.cat((-normed[..., half:RR], normed[..., :half]), dim=-1)
            out[..., :RR] = normed[..., :RR] * c + rotated * s
        return out if out_dtype is None else out.to(out_dtype)

    fn.__name__ = kind
    return fn


@pytest.mark.parametrize("kind", ["variance_sum", "eps_outside", "no_weight", "sign_flip", "full_width"])
def test_planted_rope_mistakes_are_caught(kind):
    assert rope_checks(_rope_mutant(kind)) != []
