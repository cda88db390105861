"""fp32 torch SDPA-math attention oracle (CPU) — test infrastructure only.

Follows the reference's SDPA call form on BSHD tensors
(benchmarks/benchmark_dense_fa4.py:70-77: ``scaled_dot_product_attention(
q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), dropout_p=0.0,
is_causal=False).transpose(1, 2)``) with the math backend in fp32, chunked
over query rows so S = 49,920 never materialises S x S scores per head.
"""

from __future__ import annotations

import math

import torch
from torch.nn import functional
from torch.nn.attention import SDPBackend, sdpa_kernel

__all__ = ["merge_reference", "sdpa_reference", "sdpa_rows"]


def _dense(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, chunk: int):
    """q (S_q, H, D), k/v (S_k, H, D) fp32 -> out (S_q, H, D), lse (H, S_q)."""

    kt = k.transpose(0, 1).unsqueeze(0)  # (1, H, Sk, D)
    vt = v.transpose(0, 1).unsqueeze(0)
    outs, lses = [], []
    for start in range(0, q.shape[0], chunk):
        qc = q[start : start + chunk].transpose(0, 1).unsqueeze(0)  # (1, H, c, D)
        if k.shape[0] == 0:
            outs.append(torch.zeros_like(qc[0].transpose(0, 1)))
            lses.append(torch.full((q.shape[1], qc.shape[2]), -math.inf))
            continue
        with sdpa_kernel(SDPBackend.MATH):
            o = functional.scaled_dot_product_attention(qc, kt, vt, dropout_p=0.0, is_causal=False, scale=scale)
        scores = torch.matmul(qc, kt.transpose(-1, -2)) * scale
        lses.append(torch.logsumexp(scores, dim=-1)[0])
        outs.append(o[0].transpose(0, 1))
    return torch.cat(outs, dim=0), torch.cat(lses, dim=1)


def sdpa_reference(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float | None = None,
    cu_seqlens: torch.Tensor | None = None,
    chunk: int = 2048,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Attention of BSHD inputs in fp32 on the CPU.

    Returns ``out`` (B, Sq, H, D) fp32 and ``lse`` (B, H, Sq) fp32 (natural
    log). With ``cu_seqlens`` (batch 1) each packed segment attends only to
    itself (block-diagonal).
    """

    q32 = q.detach().to("cpu", torch.float32)
    k32 = k.detach().to("cpu", torch.float32)
    v32 = v.detach().to("cpu", torch.float32)
    B, Sq, H, D = q32.shape
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    out = torch.empty((B, Sq, H, D), dtype=torch.float32)
    lse = torch.empty((B, H, Sq), dtype=torch.float32)
    if cu_seqlens is None:
        for b in range(B):
            out[b], lse[b] = _dense(q32[b], k32[b], v32[b], scale, chunk)
        return out, lse
    if B != 1:
        raise ValueError("packed varlen requires batch 1")
    offs = [int(x) for x in cu_seqlens.to("cpu").tolist()]
    for a, e in zip(offs[:-1], offs[1:]):
        if e > a:
            out[0, a:e], lse[0, :, a:e] = _dense(q32[0, a:e], k32[0, a:e], v32[0, a:e], scale, chunk)
    return out, lse


def sdpa_rows(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    rows: torch.Tensor,
    scale: float | None = None,
    cu_seqlens: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Oracle for a sample of query rows (indices into the sequence dim).

    Returns ``out`` (B, len(rows), H, D) and ``lse`` (B, H, len(rows)). With
    ``cu_seqlens``, each row attends to the keys of the segment holding it.
    """

    rows = rows.to("cpu", torch.int64)
    qs = q.detach().to("cpu")[:, rows]
    if cu_seqlens is None:
        return sdpa_reference(qs, k, v, scale)
    offs = torch.tensor([int(x) for x in cu_seqlens.to("cpu").tolist()])
    seg = torch.bucketize(rows, offs[1:], right=True)
    B, _, H, D = q.shape
    out = torch.empty((B, rows.numel(), H, D), dtype=torch.float32)
    lse = torch.empty((B, H, rows.numel()), dtype=torch.float32)
    for s in seg.unique().tolist():
        sel = (seg == s).nonzero().flatten()
        a, e = int(offs[s]), int(offs[s + 1])
        o, l = sdpa_reference(qs[:, sel], k[:, a:e], v[:, a:e], scale)
        out[:, sel], lse[:, :, sel] = o, l
    return out, lse


def merge_reference(outs, lses):
    """fp32 combine of partial attention results over disjoint key ranges:
    lse = logsumexp_i(lse_i), out = sum_i exp(lse_i - lse) * out_i; parts
    with lse = -inf weigh nothing, and a row with no keys gets 0 / -inf.
    outs[i] (B, S, H, D), lses[i] (B, H, S). This is the combine rule of
    ring / context-parallel attention over a forward op's (out, lse) pairs
    (src/h3_flash/runtime/attention/dense_fa4.py:53-81 names the op's
    return_lse argument); it follows from softmax over the union of the key
    ranges, which tests/test_oracle.py checks against the full attention."""

    L = torch.stack([l.float().cpu() for l in lses])  # (n, B, H, S)
    O = torch.stack([o.float().cpu() for o in outs])  # (n, B, S, H, D)
    m = L.max(dim=0).values
    finite = torch.isfinite(m)
    w = torch.where(torch.isfinite(L), torch.exp(L - torch.where(finite, m, torch.zeros_like(m))), torch.zeros_like(L))
    W = w.sum(dim=0)
    wo = w.permute(0, 1, 3, 2).unsqueeze(-1)  # (n, B, S, H, 1)
    out = (wo * O).sum(dim=0) / torch.where(W > 0, W, torch.ones_like(W)).permute(0, 2, 1).unsqueeze(-1)
    lse = torch.where(W > 0, m + torch.log(torch.where(W > 0, W, torch.ones_like(W))), torch.full_like(W, float("-inf")))
    return out, lse
