"""Write the small golden fixtures used by the CPU and GPU parity tests.

    python tests/golden/make_golden.py

Inputs are seeded N(0, 1) values rounded to bf16 (stored as their uint16 bit
patterns); expected outputs are computed here in float64 numpy, independently
of torch's SDPA and of the oracle package:

* attention: softmax(scale * q k^T) v and logsumexp per (batch, head), for a
  dense self-attention case, a cross-attention case (Sq != Sk), and a packed
  varlen case (block-diagonal over cu_seqlens);
* q/k RMSNorm + rotate-half RoPE with per-column cos/sin tables
  (the closed form of src/h3_flash/runtime/kernels/fusions.py:145-170) for
  R = 96 (the reference microbenchmark's rotary width,
  benchmarks/benchmark_transformer_fusions.py:61) and R = 128.

The reference publishes no numeric vectors for this path, so these fixtures
are generated, not copied.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 to bf16 (nearest-even) and return the uint16 bit pattern."""

    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounding = ((u >> 16) & 1) + 0x7FFF
    return ((u + rounding) >> 16).astype(np.uint16)


def bits_to_f64(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def attention64(q, k, v, scale):
    B, Sq, H, D = q.shape
    out = np.zeros((B, Sq, H, D))
    lse = np.zeros((B, H, Sq))
    for b in range(B):
        for h in range(H):
            s = scale * np.einsum("id,jd->ij", q[b, :, h], k[b, :, h])
            m = s.max(axis=1, keepdims=True)
            e = np.exp(s - m)
            z = e.sum(axis=1, keepdims=True)
            out[b, :, h] = np.einsum("ij,jd->id", e / z, v[b, :, h])
            lse[b, h] = (m + np.log(z))[:, 0]
    return out, lse


def qknorm_rope64(x, w, cos, sin, eps):
    B, S, H, D = x.shape
    R = cos.shape[1]
    half = R // 2
    y = np.zeros_like(x)
    for b in range(B):
        for s in range(S):
            for h in range(H):
                row = x[b, s, h]
                n = row / np.sqrt(np.mean(row * row) + eps) * w
                o = n.copy()
                for c in range(R):
                    if c < half:
                        o[c] = n[c] * cos[s, c] - n[c + half] * sin[s, c]
                    else:
                        o[c] = n[c] * cos[s, c] + n[c - half] * sin[s, c]
                y[b, s, h] = o
    return y


def main() -> None:
    rng = np.random.default_rng(20260902)
    D = 128
    scale = 1.0 / np.sqrt(D)
    arrays: dict[str, np.ndarray] = {"scale": np.array(scale)}

    # dense self-attention, ragged length (not a tile multiple)
    B, S, H = 1, 70, 2
    for name in ("q", "k", "v"):
        arrays[f"dense_{name}"] = bf16_bits(rng.standard_normal((B, S, H, D)))
    q, k, v = (bits_to_f64(arrays[f"dense_{n}"]) for n in ("q", "k", "v"))
    out, lse = attention64(q, k, v, scale)
    arrays["dense_out"], arrays["dense_lse"] = out.astype(np.float32), lse.astype(np.float32)

    # packed varlen on the same tensors: segments [0, 23), [23, 70)
    cu = np.array([0, 23, 70], dtype=np.int32)
    vo = np.zeros_like(out)
    vl = np.zeros_like(lse)
    for a, e in zip(cu[:-1], cu[1:]):
        o, l = attention64(q[:, a:e], k[:, a:e], v[:, a:e], scale)
        vo[:, a:e], vl[:, :, a:e] = o, l
    arrays["varlen_cu"], arrays["varlen_out"], arrays["varlen_lse"] = cu, vo.astype(np.float32), vl.astype(np.float32)

    # cross attention, Sq != Sk, batch 2
    B, Sq, Sk, H = 2, 17, 81, 1
    arrays["cross_q"] = bf16_bits(rng.standard_normal((B, Sq, H, D)))
    arrays["cross_k"] = bf16_bits(rng.standard_normal((B, Sk, H, D)))
    arrays["cross_v"] = bf16_bits(rng.standard_normal((B, Sk, H, D)))
    out, lse = attention64(*(bits_to_f64(arrays[f"cross_{n}"]) for n in ("q", "k", "v")), scale)
    arrays["cross_out"], arrays["cross_lse"] = out.astype(np.float32), lse.astype(np.float32)

    # q/k RMSNorm + partial RoPE
    B, S, H = 1, 9, 3
    eps = 1e-5
    arrays["rope_eps"] = np.array(eps)
    arrays["rope_x"] = bf16_bits(rng.standard_normal((B, S, H, D)) * 3.0)
    arrays["rope_w"] = bf16_bits(rng.standard_normal(D))
    x = bits_to_f64(arrays["rope_x"])
    w = bits_to_f64(arrays["rope_w"])
    for R in (96, 128):
        angles = rng.standard_normal((S, R)).astype(np.float32)
        c, s = np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)
        arrays[f"rope{R}_cos"], arrays[f"rope{R}_sin"] = c, s
        y = qknorm_rope64(x, w, c.astype(np.float64), s.astype(np.float64), eps)
        arrays[f"rope{R}_out"] = y.astype(np.float32)

    np.savez_compressed(HERE / "golden_small.npz", **arrays)
    print(HERE / "golden_small.npz", sum(a.nbytes for a in arrays.values()), "bytes")


if __name__ == "__main__":
    main()
