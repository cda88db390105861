"""CPU restatement of the packed-Ulysses relayouts — test infrastructure only.

Two independent forms of each movement, so that one pins the other:

* ``pack_qkv_permute`` follows ``pack_qkv_reference``
  (src/h3_flash/runtime/parallel/relayout.py:81-94): reshape each of q, k, v
  to (rows, world, hl, D), move the world axis first, and place the three
  side by side in the last dimension.
* ``pack_qkv_indexed`` follows the index arithmetic of the Triton kernel
  ``_pack_qkv_kernel`` (relayout.py:28-49) element by element:
  dim = o % D, head_slot = o // D, local_head = head_slot % hl,
  row_slot = head_slot // hl, row = row_slot % rows,
  destination = row_slot // rows, global_head = destination * hl + local_head,
  and out[head_slot * 3D + i*D + dim] = X_i[row, global_head, dim].
* ``merge_heads_permute`` follows relayout.py:138-142 (permute(1, 0, 2, 3),
  then reshape), ``merge_heads_indexed`` the kernel ``_merge_heads_kernel``
  (relayout.py:56-67): tail = o % inner, slot = o // inner,
  source = slot % world, row = slot // world,
  out[o] = x[(source * rows + row) * inner + tail].
* ``exchange`` restates what the all-to-all of packed_ulysses.py:85-128 does
  to the buffers of ``world`` ranks (checked by
  benchmarks/check_packed_ulysses.py:20-62): rank r receives slice r of every
  rank's send buffer, concatenated by source rank.

All functions work on numpy arrays of any dtype and move values only.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "exchange_output",
    "exchange_qkv",
    "merge_heads_indexed",
    "merge_heads_permute",
    "pack_qkv_indexed",
    "pack_qkv_permute",
]


def pack_qkv_permute(q: np.ndarray, k: np.ndarray, v: np.ndarray, world: int) -> np.ndarray:
    rows, heads, head_dim = q.shape
    if heads % world:
        raise ValueError(f"heads ({heads}) must divide Ulysses degree ({world})")
    hl = heads // world
    parts = [x.reshape(rows, world, hl, head_dim).transpose(1, 0, 2, 3) for x in (q, k, v)]
    return np.concatenate(parts, axis=-1)


def pack_qkv_indexed(q: np.ndarray, k: np.ndarray, v: np.ndarray, world: int) -> np.ndarray:
    rows, heads, head_dim = q.shape
    if heads % world:
        raise ValueError(f"heads ({heads}) must divide Ulysses degree ({world})")
    hl = heads // world
    out = np.empty(world * rows * hl * 3 * head_dim, dtype=q.dtype)
    sources = (q, k, v)
    for o in range(rows * heads * head_dim):
        dim = o % head_dim
        head_slot = o // head_dim
        local_head = head_slot % hl
        row_slot = head_slot // hl
        row = row_slot % rows
        destination = row_slot // rows
        global_head = destination * hl + local_head
        base = head_slot * 3 * head_dim + dim
        for i, x in enumerate(sources):
            out[base + i * head_dim] = x[row, global_head, dim]
    return out.reshape(world, rows, hl, 3 * head_dim)


def merge_heads_permute(x: np.ndarray) -> np.ndarray:
    world, rows, hl, head_dim = x.shape
    return np.ascontiguousarray(x.transpose(1, 0, 2, 3)).reshape(rows, world * hl, head_dim)


def merge_heads_indexed(x: np.ndarray) -> np.ndarray:
    world, rows, hl, head_dim = x.shape
    inner = hl * head_dim
    flat = x.reshape(-1)
    out = np.empty(rows * world * inner, dtype=x.dtype)
    for o in range(out.size):
        tail = o % inner
        slot = o // inner
        source = slot % world
        row = slot // world
        out[o] = flat[(source * rows + row) * inner + tail]
    return out.reshape(rows, world * hl, head_dim)


def exchange_qkv(send: list[np.ndarray]) -> list[np.ndarray]:
    """All-to-all of destination-major send buffers (world, rows_r, hl, 3D):
    rank r receives (sum rows, hl, 3D), the rows of rank 0 first."""

    world = len(send)
    return [np.concatenate([send[src][dst] for src in range(world)], axis=0) for dst in range(world)]


def exchange_output(outputs: list[np.ndarray], counts: list[int]) -> list[np.ndarray]:
    """Output all-to-all: rank r holds (sum counts, hl, D) attention rows of
    every source rank; source rank s receives (world, counts[s], hl, D), the
    slice of every rank for its own rows."""

    world = len(outputs)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    return [
        np.stack([outputs[r][offsets[s] : offsets[s + 1]] for r in range(world)], axis=0) for s in range(world)
    ]
