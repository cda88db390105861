"""RoPE cos/sin tables in the rotate-half layout the prologue consumes.

The reference never builds tables for the attention path itself; the model
passes ``rotary_emb = (cos, sin)`` of shape (S, R) in fp32, where column c is
paired with column c + R/2 (``cos = cos(cat(theta, theta))``). Its only in-repo
construction is ``_official_rope`` (src/h3_flash/runtime/parallel/rank_local_io.py:74-80):
positions (t, h, w) times per-axis inverse frequencies, concatenated per axis,
then duplicated. These helpers build such tables for the synthetic workloads:

* video tokens: 3D RoPE over a (T, Hp, Wp) latent grid with head-dim bands
  ``dims = (d_t, d_h, d_w)`` (44/42/42 for D = 128), ``inv_a[i] = base^(-2i/d_a)``;
* audio tokens: 1D RoPE over the token index with ``inv[i] = base^(-2i/D)``.

Tables are computed in fp32 like ``_official_rope``.
"""

from __future__ import annotations

import torch

__all__ = ["inv_freq", "rope_3d_tables", "rope_1d_tables", "grid_positions"]


def inv_freq(dim: int, base: float = 10000.0) -> torch.Tensor:
    """Inverse frequencies base^(-2i/dim), i = 0 .. dim/2 - 1 (fp32)."""

    if dim % 2:
        raise ValueError(f"rotary band width must be even, got {dim}")
    exponent = torch.arange(0, dim, 2, dtype=torch.float32) / dim
    return 1.0 / (base**exponent)


def grid_positions(grid: tuple[int, int, int]) -> torch.Tensor:
    """(T*Hp*Wp, 3) float32 positions (t, h, w) of row-major video tokens."""

    t, h, w = grid
    tt = torch.arange(t, dtype=torch.float32).view(t, 1, 1).expand(t, h, w)
    hh = torch.arange(h, dtype=torch.float32).view(1, h, 1).expand(t, h, w)
    ww = torch.arange(w, dtype=torch.float32).view(1, 1, w).expand(t, h, w)
    return torch.stack((tt, hh, ww), dim=-1).reshape(-1, 3)


def rope_3d_tables(
    grid: tuple[int, int, int],
    dims: tuple[int, int, int] = (44, 42, 42),
    base: float = 10000.0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin (T*Hp*Wp, sum(dims)) fp32 for row-major video tokens."""

    pos = grid_positions(grid)
    theta = torch.cat(
        [pos[:, a : a + 1] * inv_freq(d, base).view(1, -1) for a, d in enumerate(dims)], dim=-1
    )
    theta = torch.cat((theta, theta), dim=-1)
    return theta.cos(), theta.sin()


def rope_1d_tables(n: int, dim: int = 128, base: float = 10000.0) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin (n, dim) fp32 for tokens 0 .. n-1 (1D RoPE)."""

    pos = torch.arange(n, dtype=torch.float32).view(-1, 1)
    theta = pos * inv_freq(dim, base).view(1, -1)
    theta = torch.cat((theta, theta), dim=-1)
    return theta.cos(), theta.sin()
