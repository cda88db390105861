"""CPU tests of the host side of the fused projection: the rotate-half table
check that decides whether ``qkv_projection`` may read only the first half of
the RoPE tables.

The check is remembered per pair of table objects and their versions. A
freed table's memory is handed out again by the allocator and a new tensor
starts at version 0, so an answer keyed on addresses could be returned for
a different table of the same shape; these tests build exactly that case.
"""

from __future__ import annotations

import gc

import numpy as np
import torch

from h3_flash_amd.projection import rotate_half_tables


def _tables(seqlen: int, R: int, rotate_half: bool, seed: int):
    g = torch.Generator().manual_seed(seed)
    theta = torch.rand((seqlen, R // 2), generator=g) * 6.0
    if rotate_half:
        theta = torch.cat((theta, theta), dim=-1)
    else:
        theta = torch.cat((theta, theta + 0.25), dim=-1)
    return theta.cos(), theta.sin()


def test_rotate_half_detected():
    cos, sin = _tables(9, 64, True, 0)
    assert rotate_half_tables(cos, sin)
    assert rotate_half_tables(cos, sin)  # the remembered answer
    c2, s2 = _tables(9, 64, False, 1)
    assert not rotate_half_tables(c2, s2)


def test_reused_memory_is_checked_again():
    # Two tensor objects over the same memory, each new at version 0: a
    # rotate-half pair is checked and dropped, the memory is rewritten with a
    # pair that is not in that form, and new tensors wrap it at the same
    # addresses. This is what the caching allocator does with the fp32
    # temporaries of a caller's tables.
    mem = np.empty((2, 16, 128), dtype=np.float32)
    c, s = _tables(16, 128, True, 2)
    mem[0], mem[1] = c.numpy(), s.numpy()
    cos, sin = torch.from_numpy(mem[0]), torch.from_numpy(mem[1])
    assert rotate_half_tables(cos, sin)
    addrs = (cos.data_ptr(), sin.data_ptr())
    del cos, sin
    gc.collect()
    c, s = _tables(16, 128, False, 3)
    mem[0], mem[1] = c.numpy(), s.numpy()
    cos2, sin2 = torch.from_numpy(mem[0]), torch.from_numpy(mem[1])
    assert (cos2.data_ptr(), sin2.data_ptr()) == addrs and cos2._version == 0 and sin2._version == 0
    assert not rotate_half_tables(cos2, sin2)


def test_in_place_change_is_seen():
    cos, sin = _tables(8, 32, True, 3)
    assert rotate_half_tables(cos, sin)
    sin[:, 20] += 0.5  # breaks the equality of columns 4 and 20
    assert not rotate_half_tables(cos, sin)
    sin[:, 20] -= 0.5
    assert rotate_half_tables(cos, sin) == bool(torch.equal(sin[:, :16], sin[:, 16:]))


def test_other_sin_object_is_checked_again():
    cos, sin = _tables(8, 32, True, 4)
    assert rotate_half_tables(cos, sin)
    bad = sin.clone()
    bad[:, 3] += 1.0
    assert not rotate_half_tables(cos, bad)
    assert rotate_half_tables(cos, sin)


def test_odd_or_mismatched_tables_are_rejected():
    cos, sin = _tables(4, 32, True, 5)
    assert not rotate_half_tables(cos[:, :31], sin[:, :31])
    assert not rotate_half_tables(cos, sin[:, :30])
