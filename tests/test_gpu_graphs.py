"""The hot path captured in a HIP graph (torch.cuda.CUDAGraph), the way a
serving loop would replay it: the prologue, the attention with its
split-tail workspace and merge kernel, the attention's dynamic tail (its
counter is reset by a kernel recorded in the graph), a packed varlen launch
whose work list is planned on the device (the segmentation changes between
replays: the recorded planning kernel reads the new offsets), a packed
launch of short segments on the persistent kernel (its tile counter reset by
a recorded kernel; the segmentation changes between replays), and a row
fusion. Each replay runs on new inputs written into the captured buffers by
eager work, and must equal the eager launches on the same inputs bit for bit
(same kernels, same launch shapes, deterministic)."""

from __future__ import annotations

import pytest
import torch

from h3_flash_amd import flash_attn_func
from h3_flash_amd.context_parallel import merge_attention
from h3_flash_amd.fusions import fused_rmsnorm_modulate
from h3_flash_amd.prologue import fused_qk_norm_rope
from h3_flash_amd.rope import rope_3d_tables

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _fill(tensors, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    for t in tensors:
        t.copy_(torch.randn(t.shape, device=DEV, generator=g).to(t.dtype))


def test_prologue_attention_and_fusion_replay_in_a_graph():
    S, H, D, C = 4096, 4, 128, 1024  # 64 query tiles: the split-tail path with its workspace
    q_raw, k_raw, v = (torch.empty((1, S, H, D), dtype=torch.bfloat16, device=DEV) for _ in range(3))
    # 320 tiles: the dynamic-tail path (counter reset, queued pieces, merge)
    q2, k2, v2 = (torch.empty((1, 16384, 5, D), dtype=torch.bfloat16, device=DEV) for _ in range(3))
    # packed varlen over 6,000 rows; segment offsets rewritten before every replay
    q3, k3, v3 = (torch.empty((1, 6000, 5, D), dtype=torch.bfloat16, device=DEV) for _ in range(3))
    cu = torch.tensor([0, 4000, 6000], dtype=torch.int32, device=DEV)
    segmentations = ([0, 4000, 6000], [0, 1000, 6000], [0, 5999, 6000], [0, 0, 6000], [0, 3000, 6000])
    x = torch.empty((1, 512, C), dtype=torch.bfloat16, device=DEV)
    w = torch.ones(D, dtype=torch.bfloat16, device=DEV)
    wm = torch.empty(C, dtype=torch.bfloat16, device=DEV)
    table = torch.empty((9, 2 * C), dtype=torch.bfloat16, device=DEV)
    index = torch.arange(512, device=DEV) % 9
    cos, sin = (t.to(DEV) for t in rope_3d_tables((4, 32, 32)))

    def step():
        q, k = fused_qk_norm_rope(q_raw, k_raw, w, w, cos, sin, 1e-5, 1e-5)
        o1, l1 = flash_attn_func(q, k[:, : S // 2], v[:, : S // 2])
        o2, l2 = flash_attn_func(q, k[:, S // 2 :], v[:, S // 2 :])
        o, l = merge_attention([o1, o2], [l1, l2])
        full, full_lse = flash_attn_func(q, k, v)
        y = fused_rmsnorm_modulate(x, wm, table[:, :C], table[:, C:], index, 1e-5)
        tail_o, tail_l = flash_attn_func(q2, k2, v2)
        var_o, var_l = flash_attn_func(q3, k3, v3, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=6000)
        return o, l, full, full_lse, y, tail_o, tail_l, var_o, var_l

    _fill([q_raw, k_raw, v, x, wm, table, q2, k2, v2, q3, k3, v3], 0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    torch.cuda.synchronize()

    for replay in range(4):
        _fill([q_raw, k_raw, v, x, wm, table, q2, k2, v2, q3, k3, v3], 100 + replay)
        cu.copy_(torch.tensor(segmentations[replay + 1], dtype=torch.int32))
        eager = [t.clone() for t in step()]
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        names = ("merged", "merged_lse", "attn", "lse", "modulate", "tail_attn", "tail_lse", "varlen", "varlen_lse")
        for name, got, want in zip(names, captured, eager):
            assert torch.equal(got, want), f"replay {replay}: {name} differs from the eager launch"
    # the merge of the two key halves is the full attention within the path's tolerance
    o, l, full, full_lse = captured[:4]
    assert (o.float() - full.float()).abs().max().item() <= 2e-2
    assert (l - full_lse).abs().max().item() <= 1e-3


@pytest.mark.parametrize("heads", [5, 40])
def test_persistent_short_segment_launch_replays_in_a_graph(heads):
    # a packed launch whose longest segment is under 4,096 rows, the longest
    # at most 1.6 times the mean (12,000 rows in 5 segments of at most 3,000),
    # runs one workgroup per CU that claims tiles from a counter (reset by a
    # kernel recorded in the graph); the segmentation changes between
    # replays, the number of segments (and max_seqlen_q) staying what was
    # captured
    rows, D, max_q = 12000, 128, 3000
    q, k, v = (torch.empty((1, rows, heads, D), dtype=torch.bfloat16, device=DEV) for _ in range(3))
    segmentations = (  # every row in a segment, as the eager comparison needs
        [0, 3000, 6000, 9000, 12000, 12000],
        [0, 1024, 3500, 6000, 9000, 12000],
        [0, 1, 3000, 6000, 9000, 12000],
        [0, 0, 3000, 6000, 9000, 12000],
        [0, 700, 3700, 6500, 9500, 12000],
    )
    cu = torch.tensor(segmentations[0], dtype=torch.int32, device=DEV)

    def step():
        return flash_attn_func(q, k, v, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=max_q)

    _fill([q, k, v], heads)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    torch.cuda.synchronize()

    for replay in range(4):
        _fill([q, k, v], 200 + replay)
        cu.copy_(torch.tensor(segmentations[replay + 1], dtype=torch.int32))
        eager = [t.clone() for t in step()]
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, got, want in zip(("out", "lse"), captured, eager):
            assert torch.equal(got, want), f"replay {replay}: {name} differs from the eager launch"
        # and the segments really are independent: the last segment's rows
        # equal a standalone launch over them (whole tiles, as the packed
        # launch runs them)
        a, e = segmentations[replay + 1][-2], segmentations[replay + 1][-1]
        if e > a:
            alone = flash_attn_func(
                q[:, a:e].contiguous(), k[:, a:e].contiguous(), v[:, a:e].contiguous(), split_tail=False
            )
            torch.cuda.synchronize()
            assert torch.equal(captured[0][:, a:e], alone[0]), replay
