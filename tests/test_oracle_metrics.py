"""Pins oracle.metrics.error_metrics, the function every parity gate reads.

The metrics restate the reference's ``_error_metrics``
(src/h3_flash/runtime/kernels/transformer.py:16-29) and the numerical block of
benchmarks/benchmark_dense_fa4.py:92-99. Each case below is a hand-built
(actual, reference) pair whose metrics follow from arithmetic done by hand:
a single spike, a constant offset, deltas of both signs, orthogonal,
anti-parallel and scaled vectors, a zero reference and a non-finite value.
Oracles with one planted mistake each (a signed delta, a missing abs, an
unnormalised or wrongly normalised relative L2, a mean over part of the
elements, a cosine of the wrong pair) must fail at least one case.
"""

from __future__ import annotations

import math

import pytest
import torch
from torch.nn import functional

from oracle.metrics import error_metrics


def _t(values) -> torch.Tensor:
    return torch.tensor(values, dtype=torch.float32)


def metric_checks(metrics, tol_floor: float = 0.0) -> list[str]:
    """Run every case on ``metrics(actual, reference)``; return the failed
    ones. ``tol_floor`` raises every relative tolerance to at least that much
    (1e-6 for metrics computed in fp32 rather than float64)."""

    failed = []

    def check(name, fn):
        try:
            fn()
        except Exception:  # an exception is a failed case
            failed.append(name)

    def close(x, y, tol=1e-9):
        tol = max(tol, tol_floor)
        assert math.isclose(x, y, rel_tol=tol, abs_tol=tol), (x, y)

    def spike():
        # 100 ones; one element off by +0.5.
        ref = torch.ones(100)
        act = ref.clone()
        act[17] += 0.5
        m = metrics(act, ref)
        close(m["max_abs"], 0.5)
        close(m["mean_abs"], 0.005)
        close(m["relative_l2"], 0.5 / 10.0)
        close(m["cosine"], 100.5 / (math.sqrt(99 + 1.5**2) * 10.0), 1e-6)
        assert m["finite"]

    def constant_offset():
        # ref = 1..8 (norm sqrt(204)); every element off by -0.25.
        ref = torch.arange(1, 9, dtype=torch.float32)
        m = metrics(ref - 0.25, ref)
        close(m["max_abs"], 0.25)
        close(m["mean_abs"], 0.25)
        close(m["relative_l2"], 0.25 * math.sqrt(8) / math.sqrt(204))

    def both_signs():
        # Deltas +0.3, -0.7, +0.1, -0.1: a signed max gives 0.3, a signed
        # mean -0.1; the absolute ones are 0.7 and 0.3.
        ref = torch.ones(4)
        m = metrics(ref + _t([0.3, -0.7, 0.1, -0.1]), ref)
        close(m["max_abs"], 0.7, 1e-6)
        close(m["mean_abs"], 0.3, 1e-6)
        close(m["relative_l2"], math.sqrt(0.09 + 0.49 + 0.01 + 0.01) / 2.0, 1e-6)

    def orthogonal():
        m = metrics(_t([0.0, 2.0]), _t([1.0, 0.0]))
        close(m["cosine"], 0.0)
        close(m["max_abs"], 2.0)
        close(m["mean_abs"], 1.5)
        close(m["relative_l2"], math.sqrt(5.0))

    def anti_parallel_and_scaled():
        ref = _t([[1.0, -2.0], [3.0, 0.5]])  # 2-D: the metrics flatten
        m = metrics(-ref, ref)
        close(m["cosine"], -1.0, 1e-6)
        close(m["relative_l2"], 2.0, 1e-6)
        m = metrics(3.0 * ref, ref)
        close(m["cosine"], 1.0, 1e-6)
        close(m["relative_l2"], 2.0, 1e-6)
        close(m["max_abs"], 6.0)

    def zero_reference():
        # The reference norm is clamped to 1e-12, so a zero reference gives
        # |delta| / 1e-12 instead of a division by zero.
        m = metrics(_t([3.0, 4.0, 0.0]), torch.zeros(3))
        close(m["relative_l2"], 5.0 / 1e-12, 1e-6)
        close(m["max_abs"], 4.0)
        close(m["mean_abs"], 7.0 / 3.0)

    def exact_match():
        ref = _t([0.5, -1.5, 2.5])
        m = metrics(ref.clone(), ref)
        assert m["max_abs"] == 0.0 and m["mean_abs"] == 0.0 and m["relative_l2"] == 0.0
        close(m["cosine"], 1.0, 1e-9)

    def not_finite():
        act = _t([1.0, float("nan"), 2.0])
        assert not metrics(act, torch.ones(3))["finite"]
        assert not metrics(_t([float("inf"), 0.0]), torch.zeros(2))["finite"]
        assert metrics(torch.ones(3), torch.ones(3))["finite"]

    def bf16_inputs():
        # bf16 actuals are widened before the difference (0.5 is exact in bf16).
        ref = torch.zeros(4)
        m = metrics(_t([0.5, 0.0, 0.0, 0.0]).to(torch.bfloat16), ref)
        close(m["max_abs"], 0.5)
        close(m["mean_abs"], 0.125)

    for name, fn in [
        ("spike", spike),
        ("constant_offset", constant_offset),
        ("both_signs", both_signs),
        ("orthogonal", orthogonal),
        ("anti_parallel_and_scaled", anti_parallel_and_scaled),
        ("zero_reference", zero_reference),
        ("exact_match", exact_match),
        ("not_finite", not_finite),
        ("bf16_inputs", bf16_inputs),
    ]:
        check(name, fn)
    return failed


def test_error_metrics_matches_hand_computed_cases() -> None:
    assert metric_checks(error_metrics) == []


def _mutant(kind: str):
    def metrics(actual, reference):
        a = actual.detach().to(torch.float64)
        r = reference.detach().to(torch.float64)
        signed = a - r
        delta = signed.abs()
        out = {
            "max_abs": float(delta.max()),
            "mean_abs": float(delta.mean()),
            "relative_l2": float(delta.norm() / r.norm().clamp_min(1e-12)),
            "cosine": float(functional.cosine_similarity(a.flatten(), r.flatten(), dim=0)),
            "finite": bool(torch.isfinite(a).all()),
        }
        if kind == "signed_max":
            out["max_abs"] = float(signed.max())
        elif kind == "signed_mean":
            out["mean_abs"] = float(signed.mean())
        elif kind == "l2_unnormalised":
            out["relative_l2"] = float(delta.norm())
        elif kind == "l2_over_actual":
            out["relative_l2"] = float(delta.norm() / a.norm().clamp_min(1e-12))
        elif kind == "mean_over_slice":
            out["mean_abs"] = float(delta.flatten()[:-1].mean())
        elif kind == "cosine_of_delta":
            out["cosine"] = float(functional.cosine_similarity(signed.flatten(), r.flatten(), dim=0))
        elif kind == "finite_of_reference":
            out["finite"] = bool(torch.isfinite(r).all())
        elif kind == "max_over_rows":
            out["max_abs"] = float(delta.reshape(delta.shape[0], -1)[0].max()) if delta.dim() > 1 else float(delta[0])
        return out

    return metrics


@pytest.mark.parametrize(
    "kind",
    [
        "signed_max",
        "signed_mean",
        "l2_unnormalised",
        "l2_over_actual",
        "mean_over_slice",
        "cosine_of_delta",
        "finite_of_reference",
        "max_over_rows",
    ],
)
def test_planted_metric_mistakes_are_caught(kind: str) -> None:
    assert metric_checks(_mutant(kind)) != []


def test_product_audit_metrics_follow_the_pinned_oracle() -> None:
    """h3_flash_amd.audit.error_metrics (the install record's gate) computes
    the same quantities as the pinned oracle, and passes the same cases to
    fp32 precision (it works in fp32, as the reference's gate does)."""

    from h3_flash_amd.audit import error_metrics as audit_metrics

    def as_oracle(actual, reference):
        m = audit_metrics(actual, reference)
        m["finite"] = bool(torch.isfinite(actual.float()).all())
        return m

    assert metric_checks(as_oracle, tol_floor=1e-6) == []
    g = torch.Generator().manual_seed(3)
    a, r = torch.randn(4, 33, generator=g), torch.randn(4, 33, generator=g)
    got, want = audit_metrics(a, r), error_metrics(a, r)
    for key in ("max_abs", "mean_abs", "relative_l2", "cosine"):
        assert math.isclose(got[key], want[key], rel_tol=1e-5, abs_tol=1e-7), key


def test_eager_rope_of_the_gate_matches_the_prologue_oracle() -> None:
    """The gate's eager side (RMSNorm, then rotate-half RoPE over the first R
    columns) equals the oracle's fused closed form in fp32, for R = D and for
    a partial R with pass-through columns."""

    from h3_flash_amd.audit import eager_qknorm_rope
    from oracle.qknorm_rope import qknorm_rope_reference

    g = torch.Generator().manual_seed(9)
    x = torch.randn(1, 6, 2, 128, generator=g)
    w = 1.0 + 0.1 * torch.randn(128, generator=g)
    for R in (128, 96):
        theta = torch.rand(6, R // 2, generator=g) * 6.0
        cos, sin = torch.cos(torch.cat((theta, theta), -1)), torch.sin(torch.cat((theta, theta), -1))
        normed = functional.rms_norm(x, (128,), w, 1e-6)
        got = eager_qknorm_rope(normed, cos, sin)
        want = qknorm_rope_reference(x, w, cos, sin, 1e-6, out_dtype=None)
        assert (got - want).abs().max().item() < 1e-5, R
