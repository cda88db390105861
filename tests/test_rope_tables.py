"""CPU pins of the RoPE tables that define the measured workloads.

The 480p and 768p shards (and the packed video + audio batch) are specified
as q/k through RMSNorm and RoPE: 3D RoPE over the (t, h, w) latent grid with
head-dim bands 44/42/42 and base 10000 for video, 1D RoPE over the token index
for audio, in the rotate-half layout the prologue reads
(src/h3_flash/runtime/kernels/fusions.py:149-170; the table form of
_official_rope, src/h3_flash/runtime/parallel/rank_local_io.py:74-80).

``h3_flash_amd.rope`` builds them; nothing downstream can notice a wrong
table (the HIP path and the oracle are fed the same one), so the tables are
checked here against values computed in float64 from the definition:

* token n of a (T, Hp, Wp) grid sits at (n // (Hp*Wp), (n // Wp) % Hp, n % Wp);
* the 64 angles are t * 10000^(-2i/44) (i < 22), then h * 10000^(-2i/42) and
  w * 10000^(-2i/42) (i < 21), and the table repeats them (rotate-half);
* token 0 has cos = 1, sin = 0; the first frequency of every band is 1;
* the audio table's angle for column c < 64 is n * 10000^(-2c/128).

Planted mistakes (bands swapped, one inverse-frequency vector shared by all
axes as _official_rope does with its module's inv_freq, the grid walked in
the transposed order, the halves interleaved) must each fail the checks.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from h3_flash_amd.rope import grid_positions, inv_freq, rope_1d_tables, rope_3d_tables
from h3_flash_amd.synth import WORKLOADS, rope_tables

BASE = 10000.0


def tol(theta: np.ndarray) -> np.ndarray:
    """fp32 tables: the angle carries the rounding of the product and of
    the inverse frequency (about 1.5e-7 of the angle), plus the cos/sin
    rounding itself."""

    return 1.5e-7 * np.abs(theta) + 2e-6


def expected_angles_3d(grid, dims=(44, 42, 42)) -> np.ndarray:
    """(T*Hp*Wp, sum(dims)/2) float64 angles from the definition."""

    T, Hp, Wp = grid
    n = np.arange(T * Hp * Wp)
    pos = (n // (Hp * Wp), (n // Wp) % Hp, n % Wp)
    cols = []
    for axis, d in enumerate(dims):
        for i in range(d // 2):
            cols.append(pos[axis] * BASE ** (-2.0 * i / d))
    return np.stack(cols, axis=1)


def check_3d(cos: torch.Tensor, sin: torch.Tensor, grid, dims=(44, 42, 42)) -> list[str]:
    """Names of the checks the tables fail (empty: all pass)."""

    bad = []
    half = sum(dims) // 2
    if tuple(cos.shape) != (math.prod(grid), 2 * half) or cos.shape != sin.shape or cos.dtype != torch.float32:
        return ["shape/dtype"]
    c = cos.double().numpy()
    s = sin.double().numpy()
    if not (np.array_equal(c[:, :half], c[:, half:]) and np.array_equal(s[:, :half], s[:, half:])):
        bad.append("rotate-half halves")
    if not (np.all(c[0] == 1.0) and np.all(s[0] == 0.0)):
        bad.append("token 0")
    theta = expected_angles_3d(grid, dims)
    if np.any(np.abs(c[:, :half] - np.cos(theta)) > tol(theta)) or np.any(np.abs(s[:, :half] - np.sin(theta)) > tol(theta)):
        bad.append("angles")
    # each band depends on its own axis only: tokens one step along an axis
    # change exactly that band's columns
    T, Hp, Wp = grid
    edges = np.cumsum((0,) + tuple(d // 2 for d in dims))
    for axis, step in enumerate((Hp * Wp, Wp, 1)):
        if (T, Hp, Wp)[axis] < 2:
            continue
        diff = np.abs(s[step] - s[0]) > 0
        want = np.zeros(half, dtype=bool)
        want[edges[axis] : edges[axis + 1]] = True
        if not np.array_equal(diff[:half], want):
            bad.append(f"band of axis {axis}")
    return bad


def test_inverse_frequencies_closed_form():
    for d in (44, 42, 128, 2):
        f = inv_freq(d).double().numpy()
        assert f.shape == (d // 2,)
        assert f[0] == 1.0
        assert abs(f[-1] - BASE ** (-(d - 2) / d)) <= 2e-7 * f[-1]
        np.testing.assert_allclose(f, BASE ** (-2.0 * np.arange(d // 2) / d), rtol=1e-6)
    with pytest.raises(ValueError):
        inv_freq(43)


def test_grid_positions_row_major():
    pos = grid_positions((3, 4, 5)).numpy()
    n = np.arange(60)
    np.testing.assert_array_equal(pos[:, 0], n // 20)
    np.testing.assert_array_equal(pos[:, 1], (n // 5) % 4)
    np.testing.assert_array_equal(pos[:, 2], n % 5)


@pytest.mark.parametrize("grid", [(3, 4, 5), (2, 7, 3), (32, 30, 52)])
def test_3d_tables_match_the_definition(grid):
    cos, sin = rope_3d_tables(grid)
    assert check_3d(cos, sin, grid) == []


def test_band_edges_and_last_frequencies():
    # columns 0-21 follow t, 22-42 follow h, 43-63 follow w; the last column
    # of each band turns by the band's smallest frequency per step
    grid = (2, 2, 2)
    cos, sin = rope_3d_tables(grid)
    theta_t = np.arccos(np.clip(cos[4].double().numpy(), -1, 1))  # token (1, 0, 0)
    theta_h = np.arccos(np.clip(cos[2].double().numpy(), -1, 1))  # token (0, 1, 0)
    theta_w = np.arccos(np.clip(cos[1].double().numpy(), -1, 1))  # token (0, 0, 1)
    assert np.allclose(theta_t[[0, 21]], [1.0, BASE ** (-42 / 44)], atol=1e-3)
    assert np.all(theta_t[22:64] == 0)
    assert np.allclose(theta_h[[22, 42]], [1.0, BASE ** (-40 / 42)], atol=1e-3)
    assert np.all(theta_h[:22] == 0) and np.all(theta_h[43:64] == 0)
    assert np.allclose(theta_w[[43, 63]], [1.0, BASE ** (-40 / 42)], atol=1e-3)
    assert np.all(theta_w[:43] == 0)


def test_1d_audio_table():
    cos, sin = rope_1d_tables(1296)
    n = np.arange(1296)[:, None]
    theta = n * BASE ** (-2.0 * np.arange(64) / 128)[None, :]
    c, s = cos.double().numpy(), sin.double().numpy()
    assert c.shape == (1296, 128)
    np.testing.assert_array_equal(c[:, :64], c[:, 64:])
    np.testing.assert_array_equal(s[:, :64], s[:, 64:])
    assert np.all(np.abs(c[:, :64] - np.cos(theta)) <= tol(theta))
    assert np.all(np.abs(s[:, :64] - np.sin(theta)) <= tol(theta))
    assert np.all(c[0] == 1) and np.all(s[0] == 0)


def test_workload_tables():
    # the benchmarked shards use exactly these tables: video rows of the
    # packed batch with the 3D grid, the audio rows restarting at token 0
    c2 = WORKLOADS["c2"]
    cos, sin = rope_tables(c2)
    assert check_3d(cos, sin, c2.video_grid) == []
    c5 = WORKLOADS["c5"]
    cos5, sin5 = rope_tables(c5)
    nv = c5.segments[0]
    assert torch.equal(cos5[:nv], cos) and torch.equal(sin5[:nv], sin)
    ca, sa = rope_1d_tables(c5.segments[1])
    assert torch.equal(cos5[nv:], ca) and torch.equal(sin5[nv:], sa)
    c4 = WORKLOADS["c4"]
    assert check_3d(*rope_tables(c4), c4.video_grid) == []


# --- planted mistakes: each must fail check_3d -------------------------------------


def _tables_from_theta(theta: torch.Tensor):
    theta = torch.cat((theta, theta), dim=-1)
    return theta.cos(), theta.sin()


def _swapped_bands(grid):
    pos = grid_positions(grid)
    dims = (42, 44, 42)  # t gets 21 frequencies, h 22
    return _tables_from_theta(torch.cat([pos[:, a : a + 1] * inv_freq(d).view(1, -1) for a, d in enumerate(dims)], -1))


def _axes_h_w_swapped(grid):
    pos = grid_positions(grid)[:, [0, 2, 1]]
    return _tables_from_theta(
        torch.cat([pos[:, a : a + 1] * inv_freq(d).view(1, -1) for a, d in enumerate((44, 42, 42))], -1)
    )


def _shared_inv_freq(grid):
    # one frequency vector for every axis (_official_rope's module.inv_freq),
    # cut to the band widths
    pos = grid_positions(grid)
    f = inv_freq(44)
    return _tables_from_theta(torch.cat([pos[:, a : a + 1] * f[: d // 2].view(1, -1) for a, d in enumerate((44, 42, 42))], -1))


def _transposed_grid(grid):
    # tokens walked w-major instead of t-major
    T, Hp, Wp = grid
    n = torch.arange(T * Hp * Wp)
    pos = torch.stack((n % T, (n // T) % Hp, n // (T * Hp)), dim=-1).float()
    return _tables_from_theta(
        torch.cat([pos[:, a : a + 1] * inv_freq(d).view(1, -1) for a, d in enumerate((44, 42, 42))], -1)
    )


def _interleaved(grid):
    cos, sin = rope_3d_tables(grid)
    idx = torch.arange(128).view(2, 64).t().reshape(-1)  # pairs (c, c + 64) adjacent
    return cos[:, idx].contiguous(), sin[:, idx].contiguous()


def _base_500k(grid):
    pos = grid_positions(grid)
    return _tables_from_theta(
        torch.cat([pos[:, a : a + 1] * inv_freq(d, 5e5).view(1, -1) for a, d in enumerate((44, 42, 42))], -1)
    )


@pytest.mark.parametrize(
    "mutant", [_swapped_bands, _axes_h_w_swapped, _shared_inv_freq, _transposed_grid, _interleaved, _base_500k]
)
def test_planted_mistakes_fail(mutant):
    grid = (3, 4, 5)
    cos, sin = mutant(grid)
    assert check_3d(cos, sin, grid) != []
