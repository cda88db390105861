"""GPU parity of the HIP attention kernel against the CPU oracle.

Tolerance (bf16 output against an fp32-accumulated SDPA-math reference on
identical bf16 inputs): max abs <= 2e-2, mean abs <= 2e-3, |dLSE| <= 1e-3.
Full-size workloads are checked on seeded samples of query rows (each row
against the full key range) and through size-independent properties.
"""

from __future__ import annotations

import pytest
import torch

from h3_flash_amd import flash_attn_func, flash_attn_varlen_func
from h3_flash_amd.prologue import fused_qk_norm_rope
from h3_flash_amd.synth import WORKLOADS, make_raw
from oracle.attention import sdpa_reference, sdpa_rows
from oracle.metrics import ATTN_MAX_ABS, ATTN_MEAN_ABS, LSE_MAX_ABS, error_metrics
from tests._golden import bf16, f32, golden

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _rand(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16)


def assert_parity(out, lse, ref_out, ref_lse, tag=""):
    m = error_metrics(out.float(), ref_out)
    lse_err = (lse.detach().cpu().double() - ref_lse.double()).abs().max().item() if lse.numel() else 0.0
    assert m["finite"], tag
    assert m["max_abs"] <= ATTN_MAX_ABS, (tag, m)
    assert m["mean_abs"] <= ATTN_MEAN_ABS, (tag, m)
    assert lse_err <= LSE_MAX_ABS, (tag, lse_err)
    return m, lse_err


def run(q, k, v, **kw):
    out, lse = flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), **kw)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu()


def test_golden_dense_cross_varlen():
    g = golden()
    scale = float(g["scale"])
    for case in ("dense", "cross"):
        out, lse = run(bf16(f"{case}_q"), bf16(f"{case}_k"), bf16(f"{case}_v"), softmax_scale=scale)
        assert_parity(out, lse, f32(f"{case}_out"), f32(f"{case}_lse"), case)
    cu = torch.from_numpy(g["varlen_cu"]).to(DEV)
    out, lse = run(bf16("dense_q"), bf16("dense_k"), bf16("dense_v"), softmax_scale=scale, cu_seqlens_q=cu,
                   cu_seqlens_k=cu, max_seqlen_q=47)
    assert_parity(out, lse, f32("varlen_out"), f32("varlen_lse"), "varlen")


@pytest.mark.parametrize(
    "B,Sq,Sk,H",
    [
        (1, 1, 1, 1),
        (1, 7, 7, 2),
        (2, 63, 65, 3),
        (1, 64, 64, 1),
        (1, 65, 129, 2),
        (1, 129, 1000, 1),
        (1, 300, 300, 5),
        (2, 1000, 513, 2),
        (1, 2048, 77, 1),
    ],
)
def test_ragged_shapes(B, Sq, Sk, H):
    q, k, v = _rand((B, Sq, H, 128), 1), _rand((B, Sk, H, 128), 2), _rand((B, Sk, H, 128), 3)
    out, lse = run(q, k, v)
    ref_o, ref_l = sdpa_reference(q, k, v)
    assert_parity(out, lse, ref_o, ref_l, (B, Sq, Sk, H))


def test_c1_full():
    w = WORKLOADS["c1"]
    raw = make_raw(w)
    out, lse = run(raw["q_raw"], raw["k_raw"], raw["v"])
    ref_o, ref_l = sdpa_reference(raw["q_raw"], raw["k_raw"], raw["v"])
    assert_parity(out, lse, ref_o, ref_l, "c1")


def test_strided_views_of_packed_qkv():
    # q/k/v as views of one (B, S, H, 3D) projection, like to_qkv(...).chunk(3)
    qkv = _rand((2, 333, 3, 3 * 128), 4).to(DEV)
    q, k, v = qkv.chunk(3, dim=-1)
    assert not q.is_contiguous()
    out, lse = flash_attn_func(q, k, v)
    ref_o, ref_l = sdpa_reference(q.cpu(), k.cpu(), v.cpu())
    assert_parity(out.cpu(), lse.cpu(), ref_o, ref_l, "strided")


def test_softmax_scale_argument():
    q, k, v = _rand((1, 200, 2, 128), 5), _rand((1, 300, 2, 128), 6), _rand((1, 300, 2, 128), 7)
    for scale in (0.02, 0.25):
        out, lse = run(q, k, v, softmax_scale=scale)
        ref_o, ref_l = sdpa_reference(q, k, v, scale)
        assert_parity(out, lse, ref_o, ref_l, scale)


@pytest.mark.parametrize("scale", [1e-4, 2.0, 12.0, 60.0])
def test_extreme_softmax_scales_on_random_data(scale):
    # Large scales make random scores span hundreds of log2 units: the row-sum
    # rescale and the overflow recompute run on ordinary data, in whole tiles
    # and in the pieces of a split tail (64 tiles at S=4096 H=4). The softmax
    # is then peaked and |O| reaches the scale of v (~4) instead of ~6e-3, so
    # the bf16 rounding of the output and of P (as in the reference's bf16
    # FA kernel) sets the error: the bound is relative to the largest |O|
    # (4 bf16 ulps of it), with relative-L2 and cosine gates and the LSE
    # within 1e-3 plus 1e-6 of its magnitude.
    for shape in ((1, 700, 3), (1, 4096, 4)):
        B, S, H = shape
        q, k, v = (_rand((B, S, H, 128), 90 + i) for i in range(3))
        out, lse = run(q, k, v, softmax_scale=scale)
        ref_o, ref_l = sdpa_reference(q, k, v, scale)
        m = error_metrics(out.float(), ref_o)
        peak = max(ref_o.abs().max().item(), 1.0)
        lse_err = ((lse.double() - ref_l.double()).abs() - 1e-6 * ref_l.double().abs()).max().item()
        assert m["finite"], (scale, shape)
        assert m["max_abs"] <= max(ATTN_MAX_ABS, 2 ** -6 * peak), (scale, shape, m)
        assert m["relative_l2"] <= 4e-3 and m["cosine"] >= 0.99999, (scale, shape, m)
        assert lse_err <= LSE_MAX_ABS, (scale, shape, lse_err)


def test_preallocated_outputs_and_current_stream():
    q, k, v = (_rand((1, 130, 1, 128), s).to(DEV) for s in (8, 9, 10))
    out = torch.empty_like(q)
    lse = torch.empty((1, 1, 130), dtype=torch.float32, device=DEV)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        o2, l2 = flash_attn_func(q, k, v, out=out, lse=lse)
    stream.synchronize()
    assert o2.data_ptr() == out.data_ptr() and l2.data_ptr() == lse.data_ptr()
    ref_o, ref_l = sdpa_reference(q.cpu(), k.cpu(), v.cpu())
    assert_parity(out.cpu(), lse.cpu(), ref_o, ref_l, "stream")


def test_varlen_many_segments_including_empty():
    offs = [0, 1, 17, 17, 145, 146, 400, 657]
    cu = torch.tensor(offs, dtype=torch.int32)
    S = offs[-1]
    q, k, v = _rand((1, S, 3, 128), 11), _rand((1, S, 3, 128), 12), _rand((1, S, 3, 128), 13)
    out, lse = run(q, k, v, cu_seqlens_q=cu.to(DEV), cu_seqlens_k=cu.to(DEV))
    ref_o, ref_l = sdpa_reference(q, k, v, cu_seqlens=cu)
    assert_parity(out, lse, ref_o, ref_l, "varlen")
    # FA varlen call form on (total, H, D)
    o3, l3 = flash_attn_varlen_func(q[0].to(DEV), k[0].to(DEV), v[0].to(DEV), cu.to(DEV), cu.to(DEV), 256, 256)
    assert torch.equal(o3.cpu(), out[0]) and torch.equal(l3.cpu(), lse[0])


def test_cross_varlen_with_segments_that_have_no_keys():
    # separate q and k offsets; segments 0 and 2 have queries but no keys
    cu_q = torch.tensor([0, 5, 70, 300], dtype=torch.int32)
    cu_k = torch.tensor([0, 0, 100, 100], dtype=torch.int32)
    q = _rand((1, 300, 2, 128), 41)
    k, v = _rand((1, 100, 2, 128), 42), _rand((1, 100, 2, 128), 43)
    out, lse = run(q, k, v, cu_seqlens_q=cu_q.to(DEV), cu_seqlens_k=cu_k.to(DEV))
    assert torch.all(out[:, :5] == 0) and torch.all(out[:, 70:] == 0)
    assert torch.all(torch.isneginf(lse[:, :, :5])) and torch.all(torch.isneginf(lse[:, :, 70:]))
    ref_o, ref_l = sdpa_reference(q[:, 5:70], k, v)
    assert_parity(out[:, 5:70], lse[:, :, 5:70], ref_o, ref_l, "cross varlen")


def test_empty_key_range_gives_zero_and_minus_inf():
    q = _rand((1, 5, 1, 128), 14).to(DEV)
    k = torch.empty((1, 0, 1, 128), dtype=torch.bfloat16, device=DEV)
    out, lse = flash_attn_func(q, k, k)
    torch.cuda.synchronize()
    assert torch.all(out == 0) and torch.all(torch.isneginf(lse))


def _aligned_scores(beta, alpha=30.0, Sq=300, H=2, seed=22):
    """q rows ~ alpha*u, k rows ~ beta_j*u (plus noise): logits*log2(e)*scale
    grow like 0.1275*alpha*beta_j along the keys."""
    g = torch.Generator().manual_seed(seed)
    S, D = beta.numel(), 128
    u = torch.randn(D, generator=g)
    u = u / u.norm()
    q = (alpha * u + 0.05 * torch.randn((1, Sq, H, D), generator=g)).to(torch.bfloat16)
    k = (beta[None, :, None, None] * u + 0.05 * torch.randn((1, S, H, D), generator=g)).to(torch.bfloat16)
    v = torch.randn((1, S, H, D), generator=g).to(torch.bfloat16)
    return q, k, v


def test_scores_rising_along_the_keys():
    # ~120 log2 units of growth after the first tile: several whole-exponent
    # raises of the softmax offset, each rescaling P, O and l
    q, k, v = _aligned_scores(torch.linspace(0.0, 31.0, 1000))
    out, lse = run(q, k, v)
    ref_o, ref_l = sdpa_reference(q, k, v)
    assert_parity(out, lse, ref_o, ref_l, "rising")


def test_score_jump_past_exponent_range():
    # ~300 log2 units above every earlier key: exp2 overflows and the tile is
    # recomputed against its exact max; once in a middle tile, once in the last
    for pos in (400, 990):
        beta = torch.zeros(1000)
        beta[pos:pos + 10] = 80.0
        q, k, v = _aligned_scores(beta, seed=23 + pos)
        out, lse = run(q, k, v)
        ref_o, ref_l = sdpa_reference(q, k, v)
        assert_parity(out, lse, ref_o, ref_l, ("jump", pos))


@pytest.mark.parametrize("excess", [20.0, 63.5, 100.0, 127.9986, 140.0])
def test_one_key_far_above_the_first_tile(excess):
    # Every query is e0 and every key is zero except key pos = 88.5 * e0, so
    # the first tile of a key range has max 0 and key pos scores
    # fl32(88.5 * c) = `excess` log2 units above it, c = fl32(scale * log2 e)
    # as the library computes it. 20 and 63.5 take the power-of-two rescale;
    # 100 and up are recomputed against the exact max. 127.9986 gives a p that
    # is finite in fp32 but rounds to inf in bf16 (log2 p in [127.9972, 128)),
    # and 140 overflows fp32 itself. The key sits in the second tile of the
    # whole range (100) and of the second of four key-range pieces (1100).
    import numpy as np

    S, H = 4096, 4
    scale = excess / (88.5 * 1.4426950408889634)
    c = np.float32(np.float32(scale) * np.float32(1.4426950408889634))
    e = float(np.float32(np.float32(88.5) * c))
    assert abs(e - excess) < 1e-3
    if excess == 127.9986:
        assert 127.9972 < e < 128.0
    q = torch.zeros((1, S, H, 128), dtype=torch.bfloat16)
    q[..., 0] = 1.0
    v = _rand((1, S, H, 128), 31)
    for pos in (100, 1100):
        k = torch.zeros((1, S, H, 128), dtype=torch.bfloat16)
        k[0, pos, :, 0] = 88.5
        ref_o, ref_l = sdpa_reference(q[:, :1], k, v, scale)
        ref_o, ref_l = ref_o.expand(1, S, H, 128), ref_l.expand(1, H, S)
        peak = max(ref_o.abs().max().item(), 1.0)
        for split in (False, True):
            out, lse = run(q, k, v, softmax_scale=scale, split_tail=split)
            m = error_metrics(out.float(), ref_o)
            lse_err = (lse.double() - ref_l.double()).abs().max().item()
            tag = (excess, pos, split)
            assert m["finite"], tag
            assert m["max_abs"] <= max(ATTN_MAX_ABS, 2 ** -7 * peak), (tag, m)
            assert lse_err <= LSE_MAX_ABS, (tag, lse_err)


def test_split_tail_matches_whole_tiles():
    # on a 256-CU part: c1 (64 tiles) runs every tile as 4 key-range pieces,
    # the 3-batch shape (84 tiles, ragged key range) as 3 pieces
    for shape in ((1, 4096, 4096, 4), (3, 1000, 3000, 7)):
        B, Sq, Sk, H = shape
        q, k, v = (_rand(s_, 40 + i).to(DEV) for i, s_ in enumerate(((B, Sq, H, 128), (B, Sk, H, 128), (B, Sk, H, 128))))
        o1, l1 = flash_attn_func(q, k, v)
        o0, l0 = flash_attn_func(q, k, v, split_tail=False)
        torch.cuda.synchronize()
        assert (o1.float() - o0.float()).abs().max().item() <= 8e-3, shape
        assert (l1 - l0).abs().max().item() <= 1e-5, shape
        ref_o, ref_l = sdpa_reference(q.cpu(), k.cpu(), v.cpu())
        assert_parity(o1.cpu(), l1.cpu(), ref_o, ref_l, ("split", shape))


def test_dynamic_tail_matches_whole_tiles():
    # on a 256-CU part: 320 tiles (256 whole, the last 64 as 4 key-range
    # pieces each, taken from the tail counter), then 336 tiles over two
    # batches with a ragged key range (256 whole, 80 in pieces)
    for B, S, H in ((1, 16384, 5), (2, 6000, 7)):
        q, k, v = (_rand((B, S, H, 128), 60 + i).to(DEV) for i in range(3))
        o1, l1 = flash_attn_func(q, k, v)
        o0, l0 = flash_attn_func(q, k, v, split_tail=False)
        torch.cuda.synchronize()
        assert (o1.float() - o0.float()).abs().max().item() <= 8e-3, (B, S, H)
        assert (l1 - l0).abs().max().item() <= 1e-5, (B, S, H)
        # and against the oracle on seeded rows of the last tiles (the pieces)
        rows = torch.randint(S - 2048, S, (64,), generator=torch.Generator().manual_seed(S))
        ref_o, ref_l = sdpa_rows(q.cpu(), k.cpu(), v.cpu(), rows)
        got_o, got_l = o1.cpu()[:, rows], l1.cpu()[:, :, rows]
        assert_parity(got_o, got_l, ref_o, ref_l, ("dynamic tail", B, S, H))
        # repeated launches reuse the counter: same result every time
        o2, l2 = flash_attn_func(q, k, v)
        assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_dynamic_tail_on_concurrent_streams():
    # two dynamic-tail launches in flight at once on two streams: each call
    # has its own workspace and counter, so both equal their serial results
    ins = [[_rand((1, 16384, 5, 128), 80 + 3 * j + i).to(DEV) for i in range(3)] for j in range(2)]
    serial = [flash_attn_func(*x) for x in ins]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(2)]
    for s_ in streams:
        s_.wait_stream(torch.cuda.current_stream())
    results = []
    for x, s_ in zip(ins, streams):
        with torch.cuda.stream(s_):
            results.append(flash_attn_func(*x))
    for s_ in streams:
        torch.cuda.current_stream().wait_stream(s_)
    torch.cuda.synchronize()
    for (o, l), (so, sl) in zip(results, serial):
        assert torch.equal(o, so) and torch.equal(l, sl)


def test_small_or_misaligned_workspace_runs_whole_tiles():
    # through the C ABI: no workspace, one byte short, or not 256-byte
    # aligned -> every tile runs whole (bit-identical to split_tail=False);
    # exactly the size asked for -> the split result
    import ctypes
    import math

    from h3_flash_amd import _ext

    lib = _ext.load_library()
    for B, S, H in ((1, 4096, 4), (1, 16384, 5)):
        q, k, v = (_rand((B, S, H, 128), 70 + i).to(DEV) for i in range(3))
        whole = flash_attn_func(q, k, v, split_tail=False)
        split = flash_attn_func(q, k, v)

        def call(offset, short):
            out = torch.empty_like(q)
            lse = torch.empty((B, H, S), device=DEV)
            a = _ext.AttnArgs()
            a.abi_version = _ext.ABI_VERSION
            a.q, a.k, a.v, a.o, a.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr()
            a.batch, a.heads, a.seqlen_q, a.seqlen_k, a.head_dim = B, H, S, S, 128
            for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
                getattr(a, name)[:] = (S * H * 128, H * 128, 128)
            a.lse_stride[:] = (H * S, S)
            a.softmax_scale = 1.0 / math.sqrt(128)
            need = lib.h3a_attn_fwd_workspace_size(ctypes.byref(a))
            assert need > 0
            ws = torch.empty(need + 512, dtype=torch.uint8, device=DEV)
            assert ws.data_ptr() % 256 == 0
            if offset is not None:
                a.workspace, a.workspace_bytes = ws.data_ptr() + offset, need - short
            rc = lib.h3a_attn_fwd(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream))
            assert rc == _ext.H3A_OK, _ext.last_error(lib)
            torch.cuda.synchronize()
            return out, lse

        for offset, short, expect in ((None, 0, whole), (0, 1, whole), (16, 0, whole), (0, 0, split)):
            out, lse = call(offset, short)
            assert torch.equal(out, expect[0]) and torch.equal(lse, expect[1]), (B, S, H, offset, short)


@pytest.mark.parametrize(
    "B, S, H, segments",
    [
        (1, 4096, 4, None),
        (1, 16384, 5, None),
        (1, 3000, 2, None),
        (1, 0, 4, (20_000, 5_000)),
        (1, 0, 2, (1500, 1400, 1207)),
        (1, 0, 5, (3000,) + (40,) * 30),
    ],
    ids=["static-split", "dynamic-tail-d-major", "whole", "planned-varlen", "persistent-varlen", "planned-short-varlen"],
)
def test_null_lse_gives_the_same_output(B, S, H, segments):
    # lse = NULL through the C ABI (the caller wants no LSE): every launch
    # kind writes the same output as with an LSE, the tail's partial LSEs
    # still going to the workspace for the merge
    import ctypes
    import math

    from h3_flash_amd import _ext

    lib = _ext.load_library()
    cu = None
    if segments is not None:
        S = sum(segments)
        cu = torch.tensor([0, *torch.cumsum(torch.tensor(segments), 0).tolist()], dtype=torch.int32, device=DEV)
    q, k, v = (_rand((B, S, H, 128), 80 + i).to(DEV) for i in range(3))
    kw = {} if cu is None else dict(cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=max(segments))
    ref_out, _ = flash_attn_func(q, k, v, **kw)
    out = torch.full_like(q, 7.0)
    a = _ext.AttnArgs()
    a.abi_version = _ext.ABI_VERSION
    a.q, a.k, a.v, a.o, a.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), None
    a.batch, a.heads, a.seqlen_q, a.seqlen_k, a.head_dim = B, H, S, S, 128
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        getattr(a, name)[:] = (S * H * 128, H * 128, 128)
    a.softmax_scale = 1.0 / math.sqrt(128)
    if cu is not None:
        a.cu_seqlens_q = a.cu_seqlens_k = cu.data_ptr()
        a.num_segments, a.max_seqlen_q = len(segments), max(segments)
    need = lib.h3a_attn_fwd_workspace_size(ctypes.byref(a))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=DEV)
    a.workspace, a.workspace_bytes = ws.data_ptr(), need
    rc = lib.h3a_attn_fwd(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream))
    assert rc == _ext.H3A_OK, _ext.last_error(lib)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out)


def test_workspace_plan_on_this_device():
    import ctypes

    from h3_flash_amd import _ext

    lib = _ext.load_library()
    cus = torch.cuda.get_device_properties(0).multi_processor_count

    def need(B, S, H):
        a = _ext.AttnArgs()
        a.abi_version = _ext.ABI_VERSION
        a.q = a.k = a.v = a.o = 1 << 20
        a.batch, a.heads, a.seqlen_q, a.seqlen_k, a.head_dim = B, H, S, S, 128
        for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
            getattr(a, name)[:] = (S * H * 128, H * 128, 128)
        a.lse_stride[:] = (H * S, S)
        a.softmax_scale = 0.088
        return lib.h3a_attn_fwd_workspace_size(ctypes.byref(a))

    per_piece = 256 * (128 * 2 + 4)  # bf16 O and an fp32 LSE per row; a multiple of 256

    def vt(B, S, H):  # d-major V: 128 rows of keys per (batch, head), padded to 64 keys,
        # for sequences of 16,384 keys or more (shorter ones read V as given)
        return B * H * 128 * ((S + 63) // 64 * 64) * 2 if S >= 16384 else 0

    def total(split, B, S, H):  # split data, 256-byte aligned, then the d-major V
        return (split + 255) // 256 * 256 + vt(B, S, H)

    if cus == 256:
        # more tiles than CUs: the last round's tiles become 4 pieces each in
        # the dynamic tail, plus 256 bytes for its counter
        assert need(1, 49920, 5) == total(4 * 207 * per_piece + 256, 1, 49920, 5)  # 975 tiles: 768 whole
        # 1440 tiles of 160 key tiles: 3 pieces each (at least 48 key tiles per piece)
        assert need(1, 256 * 40, 36) == total(3 * 160 * per_piece + 256, 1, 256 * 40, 36)
        assert need(1, 256 * 128, 8) == total(4 * 256 * per_piece + 256, 1, 256 * 128, 8)  # 1024 tiles
        # one partial round: static pieces when it keeps under 70% of the CUs busy
        assert need(1, 4096, 4) == total(4 * 64 * per_piece, 1, 4096, 4)  # 64 tiles, 4 pieces each
        assert need(1, 256 * 200, 1) == vt(1, 256 * 200, 1)  # 200 tiles (78%): whole
        # two key tiles: 2 pieces (70 keys: no d-major V)
        assert need(1, 70, 1) == total(2 * per_piece, 1, 70, 1) == 2 * per_piece
        # 201 tiles (78%): whole; the d-major V pads 51,201 keys to 51,264
        assert need(1, 51201, 1) == need(1, 51264, 1) == vt(1, 51264, 1) == 128 * 51264 * 2
    assert need(1, 64, 1) == 0  # one key tile: nothing to split, no d-major V


def _varlen_workspace(lens, H):
    import ctypes

    from h3_flash_amd import _ext

    S = int(sum(lens))
    a = _ext.AttnArgs()
    a.abi_version = _ext.ABI_VERSION
    a.q = a.k = a.v = a.o = 1 << 20
    a.batch, a.heads, a.seqlen_q, a.seqlen_k, a.head_dim = 1, H, S, S, 128
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        getattr(a, name)[:] = (S * H * 128, H * 128, 128)
    a.lse_stride[:] = (H * S, S)
    a.softmax_scale = 0.088
    a.cu_seqlens_q = a.cu_seqlens_k = 1 << 20
    a.num_segments, a.max_seqlen_q = len(lens), int(max(lens))
    return _ext.load_library().h3a_attn_fwd_workspace_size(ctypes.byref(a))


def test_short_segments_route_by_length_spread():
    """Packed calls whose longest segment has fewer than 4,096 rows run on
    the persistent launch (its 256-byte tile counter) unless their lengths
    vary (the longest at least 1.6 times the mean) and there are few tiles
    per CU (at most 3.2 rounds, or 9 with segments of 2,900 rows or more):
    then the planned list (no tiles past a segment's rows, longest segments
    first, the last round as key-range pieces) balances the CUs. The
    workspace each asks for tells the two apart. The planned route then
    matches the oracle on sampled rows of its segments."""

    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the rule's rounds are stated for a 256-CU part")
    g = torch.Generator().manual_seed(23)
    ragged_long = torch.randint(1, 4096, (40,), generator=g).tolist()  # mean ~2,000: 6.6 rounds at H5
    ragged_short = torch.randint(1, 2049, (60,), generator=g).tolist()  # mean ~1,000: 5.3 rounds at H5
    assert _varlen_workspace([1024] * 48, 5) == 256  # equal lengths: persistent
    assert _varlen_workspace([2048] * 8, 5) == 256  # equal lengths, 1.3 rounds: persistent
    assert _varlen_workspace(ragged_short, 5) == 256  # varied, 5.3 rounds of short tiles: persistent
    assert _varlen_workspace(ragged_long, 5) > 256  # varied, 6.6 rounds, tiles up to 64 key tiles: planned
    tiny = [3000] + [40] * 30
    assert _varlen_workspace(tiny, 5) > 256  # varied, 0.6 rounds: planned

    for lens, H, seed in ((tiny, 5, 31), ([3900, 40, 2500, 7, 1200, 3100, 64, 900], 2, 32)):
        assert _varlen_workspace(lens, H) > 256
        cu = torch.tensor([0, *torch.cumsum(torch.tensor(lens), 0).tolist()], dtype=torch.int32)
        S = int(cu[-1])
        q, k, v = (_rand((1, S, H, 128), seed * 3 + i) for i in range(3))
        out, lse = flash_attn_func(
            q.to(DEV), k.to(DEV), v.to(DEV), cu_seqlens_q=cu.to(DEV), cu_seqlens_k=cu.to(DEV), max_seqlen_q=max(lens)
        )
        torch.cuda.synchronize()
        rows = _sample_rows(S, 200, seed, extra=[int(c) for c in cu[1:-1]])
        ref_o, ref_l = sdpa_rows(q, k, v, rows, cu_seqlens=cu)
        idx = rows.to(DEV)
        assert_parity(out[:, idx].cpu(), lse[:, :, idx].cpu(), ref_o, ref_l, ("planned short", len(lens), H))


def test_planned_short_cross_segments_with_empty_ranges():
    """Packed cross attention whose short query segments vary in length with
    few tiles per CU takes the planned list: query and key segments of
    different lengths, some key ranges empty (O = 0, LSE = -inf) and some
    query ranges empty. Against one workgroup per tile within the path's
    tolerance, and sampled rows of every non-empty segment against the
    oracle."""
    g = torch.Generator().manual_seed(37)
    n_seg, H = 24, 2
    lq = torch.randint(0, 3500, (n_seg,), generator=g)
    lk = torch.randint(0, 5000, (n_seg,), generator=g)
    lq[0], lk[0] = 3500, 0  # the longest query segment sees no keys
    lq[3], lq[7] = 0, 1
    lk[5] = 0
    cq = torch.zeros(n_seg + 1, dtype=torch.int32)
    ck = torch.zeros(n_seg + 1, dtype=torch.int32)
    cq[1:], ck[1:] = torch.cumsum(lq, 0), torch.cumsum(lk, 0)
    Sq, Sk = int(cq[-1]), int(ck[-1])
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert _varlen_workspace(lq.tolist(), H) > 256  # the planned list, not the persistent counter
    q = _rand((1, Sq, H, 128), 41).to(DEV)
    k = _rand((1, Sk, H, 128), 42).to(DEV)
    v = _rand((1, Sk, H, 128), 43).to(DEV)
    kw = dict(cu_seqlens_q=cq.to(DEV), cu_seqlens_k=ck.to(DEV), max_seqlen_q=int(lq.max()))
    out, lse = flash_attn_func(q, k, v, **kw)
    o_d, l_d = flash_attn_func(q, k, v, split_tail=False, **kw)
    torch.cuda.synchronize()
    a, b = int(cq[0]), int(cq[1])
    assert torch.count_nonzero(out[:, a:b]).item() == 0
    assert bool(torch.isneginf(lse[..., a:b]).all())
    live = torch.isfinite(l_d)
    assert torch.equal(live, torch.isfinite(lse))
    assert_parity(out.cpu(), torch.where(live, lse, 0).cpu(), o_d.float().cpu(), torch.where(live, l_d, 0).cpu(),
                  "planned vs one workgroup per tile")
    for s_ in range(n_seg):
        qa, qb, ka, kb = int(cq[s_]), int(cq[s_ + 1]), int(ck[s_]), int(ck[s_ + 1])
        if qb == qa or kb == ka:
            continue
        rows = torch.unique(torch.tensor([qa, qb - 1, (qa + qb) // 2]))
        ref_o, ref_l = sdpa_reference(q[:, qa:qb].cpu(), k[:, ka:kb].cpu(), v[:, ka:kb].cpu())
        loc = rows - qa
        assert_parity(out[:, rows.to(DEV)].cpu(), lse[..., rows.to(DEV)].cpu(), ref_o[:, loc], ref_l[..., loc],
                      ("segment", s_))


def test_unsupported_requests_raise():
    q = _rand((1, 8, 2, 128), 15).to(DEV)
    with pytest.raises(RuntimeError, match="non-causal"):
        flash_attn_func(q, q, q, causal=True)
    with pytest.raises(RuntimeError, match="grouped-query"):
        flash_attn_func(q, q[:, :, :1].contiguous(), q[:, :, :1].contiguous())
    with pytest.raises(ValueError, match="head_dim"):
        x = _rand((1, 8, 2, 64), 16).to(DEV)
        flash_attn_func(x, x, x)
    # preallocated outputs on another device are refused before any launch
    with pytest.raises(ValueError, match="out must be"):
        flash_attn_func(q, q, q, out=torch.empty((1, 8, 2, 128), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="lse must be"):
        flash_attn_func(q, q, q, lse=torch.empty((1, 2, 8)))


def _prologue_inputs(name):
    w = WORKLOADS[name]
    raw = make_raw(w)
    q, k = fused_qk_norm_rope(
        raw["q_raw"].to(DEV), raw["k_raw"].to(DEV), raw["w_q"], raw["w_k"], raw["cos"], raw["sin"], raw["eps"], raw["eps"]
    )
    cu = raw["cu_seqlens"]
    return q, k, raw["v"].to(DEV), cu


def _sample_rows(S, n, seed, extra=()):
    g = torch.Generator().manual_seed(seed)
    rows = torch.randint(0, S, (n,), generator=g)
    fixed = torch.tensor([0, 1, S - 1, S - 2, *extra], dtype=torch.int64)
    return torch.unique(torch.cat((rows, fixed)))


@pytest.mark.parametrize("name", ["c2", "c4"])
def test_full_size_sampled_rows(name):
    q, k, v, _ = _prologue_inputs(name)
    out, lse = flash_attn_func(q, k, v)
    torch.cuda.synchronize()
    rows = _sample_rows(q.shape[1], 96, 17)
    ref_o, ref_l = sdpa_rows(q.cpu(), k.cpu(), v.cpu(), rows)
    assert_parity(out[:, rows.to(DEV)].cpu(), lse[:, :, rows.to(DEV)].cpu(), ref_o, ref_l, name)


def test_c3_all_heads_sampled_rows():
    q, k, v, _ = _prologue_inputs("c3")
    out, lse = flash_attn_func(q, k, v)
    torch.cuda.synchronize()
    rows = _sample_rows(q.shape[1], 64, 18)
    ref_o, ref_l = sdpa_rows(q.cpu(), k.cpu(), v.cpu(), rows)
    assert_parity(out[:, rows.to(DEV)].cpu(), lse[:, :, rows.to(DEV)].cpu(), ref_o, ref_l, "c3")


def test_c5_packed_varlen_sampled_rows():
    q, k, v, cu = _prologue_inputs("c5")
    out, lse = flash_attn_func(q, k, v, cu_seqlens_q=cu.to(DEV), cu_seqlens_k=cu.to(DEV), max_seqlen_q=49920)
    torch.cuda.synchronize()
    # rows from both segments, including the ragged audio tail 51,200 .. 51,215
    rows = _sample_rows(q.shape[1], 96, 19, extra=(49919, 49920, 49921, 51199, 51200, 51207, 51215))
    ref_o, ref_l = sdpa_rows(q.cpu(), k.cpu(), v.cpu(), rows, cu_seqlens=cu)
    assert_parity(out[:, rows.to(DEV)].cpu(), lse[:, :, rows.to(DEV)].cpu(), ref_o, ref_l, "c5")
    # the audio segment must not see video keys: compare with a standalone
    # run, bit for bit on the same kernel form (split_tail=False: dispatch
    # order, V as given) and within the tolerance for the default planned
    # launch (d-major V, work list)
    a0 = 49920
    oa_, la_ = flash_attn_func(
        q[:, a0:].contiguous(), k[:, a0:].contiguous(), v[:, a0:].contiguous(), split_tail=False
    )
    ou, lu = flash_attn_func(q, k, v, cu_seqlens_q=cu.to(DEV), cu_seqlens_k=cu.to(DEV), max_seqlen_q=49920,
                             split_tail=False)
    torch.cuda.synchronize()
    assert torch.equal(oa_, ou[:, a0:]) and torch.equal(la_, lu[:, :, a0:])
    assert_parity(out[:, a0:].cpu(), lse[:, :, a0:].cpu(), oa_.float().cpu(), la_.cpu(), "c5 audio")


@pytest.mark.parametrize(
    "segments",
    [
        (49_920, 1_296),
        (1_024,) * 48,
        (40_000, 40_000),
        (49_920, 30_000, 20_000, 1_296),
        (0, 700, 0, 3_000, 5),
        (300,),
    ],
)
def test_planned_varlen_segmentations(segments):
    """Packed varlen launches with a workspace run a work list planned on the
    device (longest segments first, the last round's tiles cut into pieces
    from a counter) and a d-major V with each segment padded to 64 keys. The
    result must match the unplanned launch (dispatch order, V as given)
    within the path's tolerance, sampled rows the oracle, and be the same
    bits on every run."""

    print(f"case: planned varlen {segments}", flush=True)
    H = 5
    S = sum(segments)
    g = torch.Generator().manual_seed(len(segments) * 7 + S)
    q, k, v = (torch.randn((1, S, H, 128), generator=g).to(torch.bfloat16) for _ in range(3))
    bounds = [0]
    for n in segments:
        bounds.append(bounds[-1] + n)
    cu = torch.tensor(bounds, dtype=torch.int32, device=DEV)
    kw = {"cu_seqlens_q": cu, "cu_seqlens_k": cu, "max_seqlen_q": max(max(segments), 1)}
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    out, lse = flash_attn_func(qd, kd, vd, **kw)
    out2, lse2 = flash_attn_func(qd, kd, vd, **kw)
    ou, lu = flash_attn_func(qd, kd, vd, split_tail=False, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out, out2) and torch.equal(lse, lse2)
    assert_parity(out.cpu(), lse.cpu(), ou.float().cpu(), lu.cpu(), f"planned vs unplanned {segments}")
    rows = torch.unique(torch.tensor([b for b in bounds[:-1]] + [b - 1 for b in bounds[1:] if b > 0] + [S // 2]))
    rows = rows[(rows >= 0) & (rows < S)]
    ref_o, ref_l = sdpa_rows(q, k, v, rows, cu_seqlens=cu.cpu())
    assert_parity(out[:, rows.to(DEV)].cpu(), lse[:, :, rows.to(DEV)].cpu(), ref_o, ref_l, f"oracle {segments}")


@pytest.mark.parametrize("name", ["c2", "c3", "c4"])
def test_full_size_properties(name):
    """Size-independent properties over every row of the full workloads:
    C2 (the bench shape), C3 (40 heads) and C4 (129,024 keys: the longest
    key stream, the most offset raises per row)."""

    print(f"case: full-size properties {name}", flush=True)
    q, k, v, _ = _prologue_inputs(name)
    out, lse = flash_attn_func(q, k, v)
    # (1) rows are convex combinations of v rows: bounded by the column extrema
    vmin, vmax = v.float().amin(dim=1, keepdim=True), v.float().amax(dim=1, keepdim=True)
    assert torch.all(out.float() >= vmin - 1e-2) and torch.all(out.float() <= vmax + 1e-2)
    # (2) constant values are reproduced whatever the weights
    ones = torch.ones_like(v)
    o1, l1 = flash_attn_func(q, k, ones)
    assert (o1.float() - 1.0).abs().max().item() <= 8e-3
    assert torch.equal(l1, lse)  # LSE does not depend on v
    # (3) a joint permutation of keys and values leaves the output unchanged
    perm = torch.randperm(k.shape[1], generator=torch.Generator().manual_seed(3)).to(DEV)
    o2, l2 = flash_attn_func(q, k[:, perm].contiguous(), v[:, perm].contiguous())
    assert (o2.float() - out.float()).abs().max().item() <= 2e-2
    assert (l2 - lse).abs().max().item() <= 1e-3
    # (4) deterministic: same inputs, same bits
    o3, l3 = flash_attn_func(q, k, v)
    assert torch.equal(o3, out) and torch.equal(l3, lse)
    torch.cuda.synchronize()


@pytest.mark.gpu
@pytest.mark.parametrize("seed,n_seg,max_len", [(0, 300, 2048), (1, 700, 512), (2, 400, 300), (3, 200, 4000)])
def test_persistent_short_segments_match_dispatch_order(seed, n_seg, max_len):
    """Packed short segments (fewer than 4,096 rows) with a workspace run on
    persistent workgroups that claim tiles from a counter and prefetch each
    next tile's Q and first K / V during the current tile's last iterations.
    Many tiles per workgroup, ragged lengths, empty segments and one-row
    segments: outputs and LSE match the one-workgroup-per-tile launch
    (split_tail=False, no workspace) bit for bit, and sampled segments match
    the oracle."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(0, max_len + 1, (n_seg,), generator=g)
    lens[0], lens[-1] = max_len, 1
    lens[n_seg // 2] = 0
    H = 2
    cu = torch.zeros(n_seg + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0)
    S = int(cu[-1])
    q, k, v = (_rand((1, S, H, 128), seed * 3 + i).to(DEV) for i in range(3))
    cu_d = cu.to(DEV)
    kw = dict(cu_seqlens_q=cu_d, cu_seqlens_k=cu_d, max_seqlen_q=int(lens.max()))
    o_p, l_p = flash_attn_func(q, k, v, **kw)
    o_d, l_d = flash_attn_func(q, k, v, split_tail=False, **kw)
    torch.cuda.synchronize()
    assert torch.equal(o_p, o_d)
    assert torch.equal(l_p, l_d)
    for s in (0, 1, n_seg // 3, n_seg - 1):
        a, b = int(cu[s]), int(cu[s + 1])
        if b == a:
            continue
        ref_o, ref_l = sdpa_reference(q[:, a:b].cpu(), k[:, a:b].cpu(), v[:, a:b].cpu())
        assert_parity(o_p[:, a:b].cpu(), l_p[..., a:b].cpu(), ref_o, ref_l, ("segment", s, b - a))


@pytest.mark.gpu
@pytest.mark.parametrize("scale", [12.0, 60.0])
def test_persistent_short_segments_on_extreme_scores(scale):
    """The persistent launch's softmax offset raise and overflow recompute
    (random scores at large scales, in tiles that carry a prefetched next
    tile): bit for bit equal to one workgroup per tile, and sampled segments
    within the extreme-scale bounds of the oracle."""
    g = torch.Generator().manual_seed(int(scale))
    n_seg, H = 200, 2
    lens = torch.randint(1, 1500, (n_seg,), generator=g)
    cu = torch.zeros(n_seg + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0)
    S = int(cu[-1])
    q, k, v = (_rand((1, S, H, 128), 70 + i).to(DEV) for i in range(3))
    kw = dict(cu_seqlens_q=cu.to(DEV), cu_seqlens_k=cu.to(DEV), max_seqlen_q=int(lens.max()), softmax_scale=scale)
    o_p, l_p = flash_attn_func(q, k, v, **kw)
    o_d, l_d = flash_attn_func(q, k, v, split_tail=False, **kw)
    torch.cuda.synchronize()
    assert torch.equal(o_p, o_d) and torch.equal(l_p, l_d)
    for s in (0, n_seg // 2, n_seg - 1):
        a, b = int(cu[s]), int(cu[s + 1])
        ref_o, ref_l = sdpa_reference(q[:, a:b].cpu(), k[:, a:b].cpu(), v[:, a:b].cpu(), scale)
        m = error_metrics(o_p[:, a:b].float().cpu(), ref_o)
        peak = max(ref_o.abs().max().item(), 1.0)
        lse_err = ((l_p[..., a:b].double().cpu() - ref_l.double()).abs() - 1e-6 * ref_l.double().abs()).max().item()
        assert m["finite"], (scale, s)
        assert m["max_abs"] <= max(ATTN_MAX_ABS, 2**-6 * peak), (scale, s, m)
        assert m["relative_l2"] <= 4e-3 and m["cosine"] >= 0.99999, (scale, s, m)
        assert lse_err <= LSE_MAX_ABS, (scale, s, lse_err)


@pytest.mark.gpu
def test_persistent_stores_stay_inside_their_rows_and_heads():
    """The persistent launch writes O as 16-byte stores, 32 contiguous bytes
    of each row per store (the two half-waves exchange head dims first).
    Into views of larger buffers filled with a sentinel: O a head slice of a
    (1, S, H + 2, 128) tensor, the LSE a column slice; packed rows past the
    last segment (no segment covers them) and every element outside the
    views keep the sentinel, and the rows inside the segments equal one
    workgroup per tile written into fresh tensors (8-byte stores)."""
    g = torch.Generator().manual_seed(19)
    n_seg, H, S = 60, 3, 40_000
    lens = torch.randint(0, 600, (n_seg,), generator=g)
    lens[0], lens[1], lens[2] = 257, 1, 0
    cu = torch.zeros(n_seg + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0)
    used = int(cu[-1])
    assert used < S - 1000
    q, k, v = (_rand((1, S, H, 128), 90 + i).to(DEV) for i in range(3))
    kw = dict(cu_seqlens_q=cu.to(DEV), cu_seqlens_k=cu.to(DEV), max_seqlen_q=int(lens.max()))
    sentinel = -7.25
    big_o = torch.full((1, S, H + 2, 128), sentinel, dtype=torch.bfloat16, device=DEV)
    big_l = torch.full((1, H, S + 64), sentinel, dtype=torch.float32, device=DEV)
    out, lse = big_o[:, :, 1 : H + 1], big_l[:, :, 32 : S + 32]
    flash_attn_func(q, k, v, out=out, lse=lse, **kw)
    o_d, l_d = flash_attn_func(q, k, v, split_tail=False, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out[:, :used], o_d[:, :used])
    assert torch.equal(lse[..., :used], l_d[..., :used])
    assert bool((out[:, used:].float() == sentinel).all())
    assert bool((lse[..., used:] == sentinel).all())
    assert bool((big_o[:, :, 0].float() == sentinel).all()) and bool((big_o[:, :, H + 1].float() == sentinel).all())
    assert bool((big_l[..., :32] == sentinel).all()) and bool((big_l[..., S + 32 :] == sentinel).all())


@pytest.mark.gpu
def test_persistent_cross_segments_with_empty_key_ranges():
    """Packed cross attention on the persistent launch: query and key
    segments of different lengths, some key ranges empty (those rows give
    O = 0 and LSE = -inf) and some query ranges empty, many tiles per
    workgroup. The next-tile prefetch skips tiles without keys. Bit for bit
    equal to one workgroup per tile, and sampled segments match the oracle."""
    g = torch.Generator().manual_seed(11)
    n_seg, H = 400, 2
    lq = torch.randint(0, 1500, (n_seg,), generator=g)
    lk = torch.randint(0, 3000, (n_seg,), generator=g)
    lk[::7] = 0
    lq[::11] = 0
    lq[1], lk[1] = 1400, 0
    cq = torch.zeros(n_seg + 1, dtype=torch.int32)
    ck = torch.zeros(n_seg + 1, dtype=torch.int32)
    cq[1:], ck[1:] = torch.cumsum(lq, 0), torch.cumsum(lk, 0)
    q = _rand((1, int(cq[-1]), H, 128), 21).to(DEV)
    k = _rand((1, int(ck[-1]), H, 128), 22).to(DEV)
    v = _rand((1, int(ck[-1]), H, 128), 23).to(DEV)
    kw = dict(cu_seqlens_q=cq.to(DEV), cu_seqlens_k=ck.to(DEV), max_seqlen_q=int(lq.max()))
    o_p, l_p = flash_attn_func(q, k, v, **kw)
    o_d, l_d = flash_attn_func(q, k, v, split_tail=False, **kw)
    torch.cuda.synchronize()
    assert torch.equal(o_p, o_d)
    assert torch.equal(l_p, l_d)
    a, b = int(cq[1]), int(cq[2])
    assert torch.count_nonzero(o_p[:, a:b]).item() == 0
    assert bool(torch.isneginf(l_p[..., a:b]).all())
    for s in (0, 2, n_seg // 2, n_seg - 2):
        qa, qb, ka, kb = int(cq[s]), int(cq[s + 1]), int(ck[s]), int(ck[s + 1])
        if qb == qa or kb == ka:
            continue
        ref_o, ref_l = sdpa_reference(q[:, qa:qb].cpu(), k[:, ka:kb].cpu(), v[:, ka:kb].cpu())
        assert_parity(o_p[:, qa:qb].cpu(), l_p[..., qa:qb].cpu(), ref_o, ref_l, ("segment", s))
