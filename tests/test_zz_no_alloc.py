"""GPU test of h3a_attn_fwd_noalloc, the attention entry point that allocates
nothing (its tail workspace is a file-scope device array).

Two calls in a row through the C ABI, the second on a smaller input, each
checked against h3a_attn_fwd with a caller-allocated workspace on the same
inputs (the path's tolerance: max abs 2e-2, mean abs 2e-3, |dLSE| 1e-3) and
on sampled rows against the CPU oracle. The large call uses the dynamic
tail, whose plan is fitted to the 64 MiB array; the small one a static
split. The second call must not see the first call's partial results.
Packed short segments run the persistent launch with its tile counter in
the same array, likewise twice.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from h3_flash_amd import _ext
from oracle.attention import sdpa_rows
from oracle.metrics import ATTN_MAX_ABS, ATTN_MEAN_ABS, LSE_MAX_ABS, error_metrics

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _args(q, k, v, out, lse, workspace=None, cu=None):
    a = _ext.AttnArgs()
    a.abi_version = _ext.ABI_VERSION
    a.q, a.k, a.v, a.o, a.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr()
    B, S, H, D = q.shape
    a.batch, a.heads, a.seqlen_q, a.seqlen_k, a.head_dim = B, H, S, k.shape[1], D
    for name, t in (("q_stride", q), ("k_stride", k), ("v_stride", v), ("o_stride", out)):
        getattr(a, name)[:] = t.stride()[:3]
    a.lse_stride[:] = (lse.stride(0), lse.stride(1))
    a.softmax_scale = D**-0.5
    if workspace is not None:
        a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel()
    if cu is not None:
        lens = (cu[1:] - cu[:-1]).tolist()
        a.cu_seqlens_q = a.cu_seqlens_k = cu.data_ptr()
        a.num_segments, a.max_seqlen_q = len(lens), max(lens)
    return a


def _inputs(B, S, H, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return [torch.randn((B, S, H, 128), device=DEV, generator=g).to(torch.bfloat16) for _ in range(3)]


def _run_both(lib, q, k, v, cu=None):
    B, S, H, _ = q.shape
    stream = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    out_a, out_b = torch.empty_like(q), torch.empty_like(q)
    lse_a = torch.empty((B, H, S), dtype=torch.float32, device=DEV)
    lse_b = torch.empty_like(lse_a)
    args = _args(q, k, v, out_a, lse_a, cu=cu)
    need = lib.h3a_attn_fwd_workspace_size(ctypes.byref(args))
    assert need > 0  # every shape below uses a workspace: a split tail, a tile counter or a work list
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    args = _args(q, k, v, out_a, lse_a, ws, cu=cu)
    assert lib.h3a_attn_fwd(ctypes.byref(args), stream) == _ext.H3A_OK, _ext.last_error(lib)
    rc = lib.h3a_attn_fwd_noalloc(ctypes.byref(_args(q, k, v, out_b, lse_b, cu=cu)), stream)
    assert rc == _ext.H3A_OK, _ext.last_error(lib)
    torch.cuda.synchronize()
    return (out_a, lse_a), (out_b, lse_b)


def _assert_close(out, lse, ref_out, ref_lse, tag):
    m = error_metrics(out.float().cpu(), ref_out.float().cpu())
    lse_err = (lse.cpu().double() - ref_lse.cpu().double()).abs().max().item()
    assert m["finite"] and m["max_abs"] <= ATTN_MAX_ABS and m["mean_abs"] <= ATTN_MEAN_ABS, (tag, m)
    assert lse_err <= LSE_MAX_ABS, (tag, lse_err)


def test_noalloc_matches_the_workspace_entry_point_twice():
    lib = _ext.load_library()
    for B, S, H, seed in ((1, 49_920, 5, 61), (1, 4_096, 4, 62)):
        print(f"case: h3a_attn_fwd_noalloc B={B} S={S} H={H}", flush=True)
        q, k, v = _inputs(B, S, H, seed)
        (out_a, lse_a), (out_b, lse_b) = _run_both(lib, q, k, v)
        _assert_close(out_b, lse_b, out_a, lse_a, f"S={S} vs h3a_attn_fwd")
        rows = torch.tensor([0, 1, S // 3, S - 257, S - 1])
        ref_o, ref_l = sdpa_rows(q.cpu(), k.cpu(), v.cpu(), rows)
        _assert_close(out_b[:, rows.to(DEV)], lse_b[:, :, rows.to(DEV)], ref_o, ref_l, f"S={S} vs oracle")


def test_noalloc_packed_short_segments_twice():
    # Packed short segments run the persistent launch from the scratch (its
    # tile counter there, zeroed by the launch): equal lengths take the same
    # launch with a workspace (bit-identical); varied ones, which take the
    # planned list there, within the path's tolerance. The second call is
    # smaller and follows the first on the same scratch.
    lib = _ext.load_library()
    for lens, H, seed, same in (([1024] * 48, 5, 64, True), ([3000] + [40] * 30 + [900, 7, 2500], 2, 65, False)):
        print(f"case: h3a_attn_fwd_noalloc packed {len(lens)} segments H={H}", flush=True)
        cu = torch.tensor([0, *torch.cumsum(torch.tensor(lens), 0).tolist()], dtype=torch.int32, device=DEV)
        S = int(cu[-1])
        q, k, v = _inputs(1, S, H, seed)
        (out_a, lse_a), (out_b, lse_b) = _run_both(lib, q, k, v, cu)
        if same:
            assert torch.equal(out_a, out_b) and torch.equal(lse_a, lse_b)
        _assert_close(out_b, lse_b, out_a, lse_a, f"packed {len(lens)} vs h3a_attn_fwd")
        rows = torch.unique(torch.tensor([0, 1, S // 3, S - 2, S - 1, *cu[1:-1].tolist()]))
        ref_o, ref_l = sdpa_rows(q.cpu(), k.cpu(), v.cpu(), rows, cu_seqlens=cu.cpu())
        _assert_close(out_b[:, rows.to(DEV)], lse_b[:, :, rows.to(DEV)], ref_o, ref_l, f"packed {len(lens)} vs oracle")


def test_noalloc_rejects_what_the_launch_rejects():
    lib = _ext.load_library()
    q, k, v = _inputs(1, 256, 1, 63)
    out, lse = torch.empty_like(q), torch.empty((1, 1, 256), device=DEV)
    a = _args(q, k, v, out, lse)
    a.head_dim = 64
    assert lib.h3a_attn_fwd_noalloc(ctypes.byref(a), None) == _ext.H3A_EUNSUPPORTED
    assert "head_dim" in _ext.last_error(lib)
