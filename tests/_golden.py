"""Loader for tests/golden/golden_small.npz (inputs as bf16 bit patterns)."""

from __future__ import annotations

from functools import lru_cache
from pathlib import Path

import numpy as np
import torch

PATH = Path(__file__).resolve().parent / "golden" / "golden_small.npz"


@lru_cache(maxsize=1)
def golden() -> dict[str, np.ndarray]:
    with np.load(PATH, allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


def bf16(name: str) -> torch.Tensor:
    bits = golden()[name].astype(np.int16)
    return torch.from_numpy(bits.copy()).view(torch.bfloat16)


def f32(name: str) -> torch.Tensor:
    return torch.from_numpy(golden()[name].astype(np.float32).copy())
