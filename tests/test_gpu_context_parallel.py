"""GPU parity of the LSE merge (through the C ABI) and of the ring schedule
of context parallelism run on one device.

Merge bar: against the fp32 oracle merge of the same partials, every bf16
output within one bf16 ulp (or 1e-6 absolute) and LSE within 1e-5; fp32
outputs within 1e-5 relative. Ring schedule bar: the attention tolerance of
the path (max abs 2e-2, mean abs 2e-3, |dLSE| 1e-3) against the fp32 SDPA
oracle on all keys.
"""

from __future__ import annotations

import pytest
import torch

from h3_flash_amd import flash_attn_func, hip_forward_op
from h3_flash_amd.context_parallel import chunked_attention, merge_attention
from oracle.attention import merge_reference, sdpa_reference
from oracle.metrics import ATTN_MAX_ABS, ATTN_MEAN_ABS, LSE_MAX_ABS, error_metrics
from tests.test_gpu_fusions import assert_parity

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _partials(n, B=1, S=300, H=5, D=128, dtype=torch.bfloat16, seed=0, empty=()):
    g = torch.Generator().manual_seed(seed)
    outs = [torch.randn((B, S, H, D), generator=g).to(dtype) for _ in range(n)]
    lses = [torch.randn((B, H, S), generator=g) * 4 for _ in range(n)]
    for i in empty:
        lses[i][:] = float("-inf")
    lses[0][0, 0, :7] = float("-inf")  # some rows have no keys in part 0
    if n > 1:
        for l in lses:
            l[0, 1, 3] = float("-inf")  # one row has no keys anywhere
    return outs, lses


@pytest.mark.parametrize("n", [1, 2, 3, 5, 8, 13, 16])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_merge_matches_oracle(n, dtype):
    outs, lses = _partials(n, dtype=dtype, seed=n, empty=(1,) if n > 2 else ())
    o, l = merge_attention([x.to(DEV) for x in outs], [x.to(DEV) for x in lses])
    ro, rl = merge_reference(outs, lses)
    assert o.dtype == dtype
    if dtype == torch.bfloat16:
        assert_parity(o, ro.to(torch.bfloat16), f"merge{n}")
    else:
        torch.testing.assert_close(o.cpu(), ro, rtol=1e-5, atol=1e-6)
    finite = torch.isfinite(rl)
    assert torch.equal(torch.isfinite(l.cpu()), finite)
    assert (l.cpu()[finite] - rl[finite]).abs().max().item() <= 1e-5
    if n > 1:
        assert torch.count_nonzero(o[0, 3, 1]) == 0 and l[0, 1, 3].item() == float("-inf")


@pytest.mark.parametrize("D", [8, 64, 200, 512])
@pytest.mark.parametrize("n", [3, 13])
def test_merge_head_dims(D, n):
    # lane groups of 1, 8, 32 and 64 lanes (200: the last group is partly idle)
    outs, lses = _partials(n, S=40, H=3, D=D, dtype=torch.float32, seed=D + n, empty=(1,))
    o, l = merge_attention([x.to(DEV) for x in outs], [x.to(DEV) for x in lses])
    ro, rl = merge_reference(outs, lses)
    torch.testing.assert_close(o.cpu(), ro, rtol=1e-5, atol=1e-6)
    fin = torch.isfinite(rl)
    assert torch.equal(torch.isfinite(l.cpu()), fin)
    assert (l.cpu()[fin] - rl[fin]).abs().max().item() <= 1e-5


@pytest.mark.parametrize("D", [8, 128])
def test_merge_batched(D):
    # workgroups take 16 tokens of one head (D = 8: four heads' groups); the
    # sequence is not a multiple of 16, so each batch's last chunk is partial
    g = torch.Generator().manual_seed(D)
    B, S, H, n = 3, 37, 2, 4
    outs = [torch.randn((B, S, H, D), generator=g).to(torch.bfloat16) for _ in range(n)]
    lses = [torch.randn((B, H, S), generator=g) * 4 for _ in range(n)]
    lses[2][1, 0, 5:20] = float("-inf")
    o, l = merge_attention([x.to(DEV) for x in outs], [x.to(DEV) for x in lses])
    ro, rl = merge_reference(outs, lses)
    assert_parity(o, ro.to(torch.bfloat16), f"batched D={D}")
    assert (l.cpu() - rl).abs().max().item() <= 1e-5


def test_merge_more_than_sixteen_parts_and_in_place():
    outs, lses = _partials(21, S=64, seed=3)
    ro, rl = merge_reference(outs, lses)
    o, l = merge_attention([x.to(DEV) for x in outs], [x.to(DEV) for x in lses])
    assert_parity(o, ro.to(torch.bfloat16), "merge21")
    # a caller's fp32 output takes the dtype from it, as with 16 parts or fewer
    o32 = torch.empty(outs[0].shape, dtype=torch.float32, device=DEV)
    got, _ = merge_attention([x.to(DEV) for x in outs], [x.to(DEV) for x in lses], out=o32)
    assert got.data_ptr() == o32.data_ptr() and got.dtype == torch.float32
    assert (got.cpu() - ro).abs().max().item() <= 2e-3
    # in place: out and lse alias part 0
    d_outs = [x.to(DEV) for x in outs[:4]]
    d_lses = [x.to(DEV) for x in lses[:4]]
    ro4, rl4 = merge_reference(outs[:4], lses[:4])
    o4, l4 = merge_attention(d_outs, d_lses, out=d_outs[0], lse=d_lses[0])
    assert o4.data_ptr() == d_outs[0].data_ptr()
    assert_parity(o4, ro4.to(torch.bfloat16), "in-place")
    fin = torch.isfinite(rl4)
    assert (l4.cpu()[fin] - rl4[fin]).abs().max().item() <= 1e-5


@pytest.mark.parametrize("chunks", [1, 2, 3, 8])
def test_ring_schedule_on_one_device(chunks):
    g = torch.Generator().manual_seed(chunks)
    q, k, v = (torch.randn((1, 4096, 4, 128), generator=g).to(torch.bfloat16) for _ in range(3))
    o, l = chunked_attention(q.to(DEV), k.to(DEV), v.to(DEV), chunks)
    ro, rl = sdpa_reference(q, k, v)
    m = error_metrics(o.float().cpu(), ro)
    assert m["finite"] and m["max_abs"] <= ATTN_MAX_ABS and m["mean_abs"] <= ATTN_MEAN_ABS, m
    assert (l.cpu() - rl).abs().max().item() <= LSE_MAX_ABS


def test_forward_op_with_lse_feeds_the_merge():
    """The context-parallel template's per-chunk calls: hip_forward_op with
    return_lse on BSHD chunks of one sequence gives (B, S, H) LSEs, which
    broadcast against the output as the template's ring merge uses them, and
    which merge_attention takes with lse_layout='bsh'."""

    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn((2, 777, 3, 128), generator=g).to(torch.bfloat16).to(DEV) for _ in range(3))
    parts = [
        hip_forward_op(None, q, k[:, a:b], v[:, a:b], return_lse=True, scale=0.1)
        for a, b in ((0, 300), (300, 301), (301, 777))
    ]
    for o_i, l_i in parts:
        assert l_i.shape == (2, 777, 3) and o_i.shape == (2, 777, 3, 128)
    o, l = merge_attention([p[0] for p in parts], [p[1] for p in parts], lse_layout="bsh")
    assert l.shape == (2, 777, 3)
    full_o, full_l = flash_attn_func(q, k, v, softmax_scale=0.1)
    ro, rl = sdpa_reference(q.cpu(), k.cpu(), v.cpu(), scale=0.1)
    m = error_metrics(o.float().cpu(), ro)
    assert m["max_abs"] <= ATTN_MAX_ABS and m["mean_abs"] <= ATTN_MEAN_ABS, m
    assert (l.transpose(1, 2).cpu() - rl).abs().max().item() <= LSE_MAX_ABS
    assert (l.transpose(1, 2) - full_l).abs().max().item() <= LSE_MAX_ABS

    # The template's own two-part ring update on (B, S, H, 1) LSEs
    # (out = prev - sigmoid(lse - prev_lse) * (prev - out)) over the same
    # chunks equals the merge.
    prev_o, prev_l = None, None
    for o_i, l_i in parts:
        o_i, l_i = o_i.float(), l_i.unsqueeze(-1)
        if prev_o is not None:
            o_i = prev_o - torch.sigmoid(l_i - prev_l) * (prev_o - o_i)
            l_i = prev_l - torch.nn.functional.logsigmoid(prev_l - l_i)
        prev_o, prev_l = o_i, l_i
    assert (prev_o - o.float()).abs().max().item() <= 2e-2
    assert (prev_l.squeeze(-1) - l).abs().max().item() <= 1e-5

    # A caller's contiguous (B, S, H) LSE buffer is filled in place.
    buf = torch.empty((2, 777, 3), device=DEV)
    _, l2 = merge_attention([p[0] for p in parts], [p[1] for p in parts], lse=buf, lse_layout="bsh")
    assert l2 is buf and torch.equal(buf, l)


def test_merge_errors():
    o = torch.zeros((1, 4, 2, 128), dtype=torch.bfloat16, device=DEV)
    l = torch.zeros((1, 2, 4), device=DEV)
    with pytest.raises(ValueError):
        merge_attention([o, o], [l])
    with pytest.raises(ValueError):
        merge_attention([o], [torch.zeros((1, 2, 5), device=DEV)])
    with pytest.raises(TypeError):
        merge_attention([o.half()], [l])
    with pytest.raises(ValueError, match="out must be"):
        merge_attention([o, o], [l, l], out=torch.empty((1, 4, 2, 128), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="lse must be"):
        merge_attention([o, o], [l, l], lse=torch.empty((1, 2, 4)))
    with pytest.raises(ValueError, match="'bsh' LSEs"):
        merge_attention([o, o], [l, l], lse_layout="bsh")  # (B, H, S) given as (B, S, H)
    with pytest.raises(ValueError, match="lse_layout"):
        merge_attention([o], [l], lse_layout="hbs")
