"""Seeded synthetic workloads for the dense H3 attention path.

Shapes are those of one GPU's share of MiniMax H3 DiT self-attention
(B = 1, D = 128, bf16, non-causal, softmax scale 1/sqrt(128)):

=====  =====  ===========================  =====================================
name   heads  sequence                     inputs
=====  =====  ===========================  =====================================
c1     4      4,096                        q, k, v ~ N(0, 1)
c2     5      49,920 = 32 x 30 x 52 video  q, k ~ N(0, 1) -> RMSNorm -> 3D RoPE
c3     40     49,920                       as c2 (all heads on one GPU)
c4     5      129,024 = 32 x 48 x 84       as c2 (768p head shard)
c5     5      49,920 video + 1,296 audio   packed, block-diagonal; audio 1D RoPE
=====  =====  ===========================  =====================================

v is N(0, 1) everywhere. Raw q/k are drawn on the CPU from a seeded
``torch.Generator`` (fp32, then rounded to bf16), so a workload is the same
tensor on every machine.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .rope import rope_1d_tables, rope_3d_tables

__all__ = ["Workload", "WORKLOADS", "make_raw", "attention_flops"]

NORM_EPS = 1e-5
BASE_SEED = 20260902


@dataclass(frozen=True)
class Workload:
    name: str
    heads: int
    segments: tuple[int, ...]
    prologue: bool
    video_grid: tuple[int, int, int] | None
    seed: int
    batch: int = 1
    head_dim: int = 128
    rope_dims: tuple[int, int, int] = (44, 42, 42)

    @property
    def seqlen(self) -> int:
        return sum(self.segments)

    @property
    def varlen(self) -> bool:
        return len(self.segments) > 1

    @property
    def flops(self) -> float:
        return attention_flops(self.batch, self.heads, self.segments, self.head_dim)

    def describe(self) -> str:
        seg = "+".join(str(s) for s in self.segments)
        return f"B={self.batch} H={self.heads} S={seg} D={self.head_dim} non-causal bf16"


def attention_flops(batch: int, heads: int, segments: tuple[int, ...], head_dim: int = 128) -> float:
    """4 * D * H * sum(S_i^2) per batch element (QK^T and PV, 2 flops per MAC)."""

    return float(4 * head_dim * heads * batch * sum(s * s for s in segments))


WORKLOADS: dict[str, Workload] = {
    "c1": Workload("c1", 4, (4096,), False, None, BASE_SEED + 1),
    "c2": Workload("c2", 5, (49920,), True, (32, 30, 52), BASE_SEED + 2),
    "c3": Workload("c3", 40, (49920,), True, (32, 30, 52), BASE_SEED + 3),
    "c4": Workload("c4", 5, (129024,), True, (32, 48, 84), BASE_SEED + 4),
    "c5": Workload("c5", 5, (49920, 1296), True, (32, 30, 52), BASE_SEED + 5),
}


def rope_tables(w: Workload) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 (S, 128) cos/sin for the workload's packed sequence."""

    cos, sin = rope_3d_tables(w.video_grid, w.rope_dims)
    if cos.shape[0] != w.segments[0]:
        raise ValueError(f"grid {w.video_grid} does not cover {w.segments[0]} video tokens")
    if len(w.segments) > 1:
        parts_c, parts_s = [cos], [sin]
        for n in w.segments[1:]:
            c1, s1 = rope_1d_tables(n, w.head_dim)
            parts_c.append(c1)
            parts_s.append(s1)
        cos, sin = torch.cat(parts_c), torch.cat(parts_s)
    return cos.contiguous(), sin.contiguous()


def make_raw(w: Workload, heads: int | None = None) -> dict:
    """CPU tensors of a workload before the prologue.

    Returns ``q_raw, k_raw, v`` (B, S, H, D) bf16, ``w_q, w_k`` (D,) bf16 unit
    gains, ``eps``, ``cos, sin`` (S, 128) fp32 (None when the workload has no
    prologue) and ``cu_seqlens`` (int32, None when dense).
    """

    h = w.heads if heads is None else heads
    gen = torch.Generator(device="cpu").manual_seed(w.seed)
    shape = (w.batch, w.seqlen, h, w.head_dim)
    q = torch.randn(shape, generator=gen, dtype=torch.float32).to(torch.bfloat16)
    k = torch.randn(shape, generator=gen, dtype=torch.float32).to(torch.bfloat16)
    v = torch.randn(shape, generator=gen, dtype=torch.float32).to(torch.bfloat16)
    out = {"q_raw": q, "k_raw": k, "v": v, "eps": NORM_EPS, "cos": None, "sin": None, "cu_seqlens": None}
    out["w_q"] = torch.ones(w.head_dim, dtype=torch.bfloat16)
    out["w_k"] = torch.ones(w.head_dim, dtype=torch.bfloat16)
    if w.prologue:
        out["cos"], out["sin"] = rope_tables(w)
    if w.varlen:
        offsets = [0]
        for s in w.segments:
            offsets.append(offsets[-1] + s)
        out["cu_seqlens"] = torch.tensor(offsets, dtype=torch.int32)
    return out
