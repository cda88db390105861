"""The projection GEMM (h3a_proj_gemm) on the GPU against the CPU oracle in
the reference's rounding order (the projection rounded to bf16, then the q/k
RMSNorm + RoPE): plain sections and sections with the norm + RoPE epilogue,
ragged token counts, half-width last tiles, rotary widths that are multiples
of 32 (partners in the same lane, the tables' first half read) and any other
even width or table form (partners from the token's other lanes, every
rotated column read), more tiles than CUs (one workgroup per tile), the 480p
rank and 40-head projection shapes (sampled rows), hipBLASLt's own linear,
and the attention processor with fused projections and its fallback record."""

from __future__ import annotations

import math

import pytest
import torch

from h3_flash_amd import DenseMiniMaxH3Processor, install_dense_hip
from h3_flash_amd.projection import Section, out_projection, proj_gemm, qkv_projection, rotate_half_tables
from h3_flash_amd.rope import rope_3d_tables
from oracle.metrics import error_metrics
from oracle.projection import projection_reference

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def tables(seqlen: int, R: int, seed: int = 0):
    """Rotate-half tables (cos(cat(theta, theta)))."""

    pos = torch.arange(seqlen, dtype=torch.float32)[:, None]
    inv = 10000.0 ** (-torch.arange(0, R, 2, dtype=torch.float32) / max(R, 1))
    theta = pos * inv + seed
    theta = torch.cat((theta, theta), dim=1)
    return theta.cos().contiguous(), theta.sin().contiguous()


def assert_matches(got: torch.Tensor, ref: torch.Tensor, what: str = "", rounded_projection: bool = False):
    """Within one bf16 step of the oracle's value plus 2^-9 of the row's RMS
    (the two sides sum the K products in different orders, and a value that
    nearly cancels keeps that absolute error), and mostly bit-identical.

    ``rounded_projection`` (q and k: the projection is rounded to bf16 before
    the norm): where the two summation orders put a projection value on two
    sides of a bf16 rounding boundary, the normalised value moves by up to
    2^-7 of itself, and both outputs its rotation feeds move with it. Those
    elements (rare) may differ by up to 2^-4 of the row's RMS."""

    got, ref = got.float().cpu(), ref.float()
    d = (got - ref).abs()
    ulp = 2.0 ** (torch.floor(torch.log2(ref.abs().clamp_min(1e-30))) - 7)
    rms = ref.pow(2).mean(dim=1, keepdim=True).sqrt()
    tight = ulp + rms * 2.0**-9
    bad = d > tight
    if rounded_projection:
        loose = ulp + rms * 2.0**-4
        assert not (d > loose).any(), (what, int((d > loose).sum()), float((d / loose).max()))
        assert bad.float().mean() <= 5e-3, (what, int(bad.sum()))
    else:
        assert not bad.any(), (what, int(bad.sum()), float((d / tight).max()))
    assert (d == 0).float().mean() > 0.99, (what, float((d == 0).float().mean()))


def make(M, K, heads, R, bias, seed=0):
    g = torch.Generator().manual_seed(seed)
    n = heads * 128
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    w = (torch.randn((3 * n, K), generator=g) / math.sqrt(K)).to(torch.bfloat16)
    b = (0.1 * torch.randn(3 * n, generator=g)).to(torch.bfloat16) if bias else None
    nwq = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16)
    nwk = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16)
    return x, w, b, nwq, nwk


def run_qkv(x, w, b, nwq, nwk, cos, sin, seqlen, eps=1e-6, rotate_half=True):
    n = w.shape[0] // 3
    xd, wd = x.to(DEV), w.to(DEV)
    bd = b.to(DEV) if b is not None else None
    y = torch.empty((x.shape[0], 3 * n), dtype=torch.bfloat16, device=DEV)
    secs = [
        Section(wd[:n], y[:, :n], None if bd is None else bd[:n], nwq.to(DEV), eps),
        Section(wd[n : 2 * n], y[:, n : 2 * n], None if bd is None else bd[n : 2 * n], nwk.to(DEV), eps),
        Section(wd[2 * n :], y[:, 2 * n :], None if bd is None else bd[2 * n :]),
    ]
    c, s = (None, None) if cos is None else (cos.to(DEV), sin.to(DEV))
    proj_gemm(xd, secs, c, s, seqlen, rotate_half=rotate_half)
    torch.cuda.synchronize()
    return y.cpu()


def check_qkv(x, w, b, nwq, nwk, cos, sin, seqlen, y, rows=None, eps=1e-6):
    n = w.shape[0] // 3
    xs = x if rows is None else x[rows]
    ys = y if rows is None else y[rows]
    if rows is not None and cos is not None:
        # sampled rows keep their own table rows
        idx = torch.as_tensor(rows) % seqlen
        cos, sin, seqlen = cos[idx], sin[idx], len(rows)
    bb = (lambda i: None) if b is None else (lambda i: b[i * n : (i + 1) * n])
    assert_matches(ys[:, :n], projection_reference(xs, w[:n], bb(0), nwq, eps, cos, sin, seqlen), "q", True)
    assert_matches(ys[:, n : 2 * n], projection_reference(xs, w[n : 2 * n], bb(1), nwk, eps, cos, sin, seqlen), "k", True)
    assert_matches(ys[:, 2 * n :], projection_reference(xs, w[2 * n :], bb(2)), "v")


@pytest.mark.parametrize(
    "M, K, heads, R, bias, seqlen",
    [
        (608, 256, 2, 128, True, 608),   # ragged last token tile
        (300, 128, 1, 96, False, 100),   # half-width feature tiles, 3 sequences
        (296, 384, 2, 64, True, 296),
        (256, 512, 3, 32, True, 128),    # a half-width tile per section
        (1000, 256, 2, 0, True, 1000),   # the norm alone
    ],
)
def test_qkv_sections_match_the_oracle(M, K, heads, R, bias, seqlen):
    x, w, b, nwq, nwk = make(M, K, heads, R, bias, seed=M + K)
    cos, sin = tables(seqlen, R) if R else (None, None)
    y = run_qkv(x, w, b, nwq, nwk, cos, sin, seqlen)
    check_qkv(x, w, b, nwq, nwk, cos, sin, seqlen, y)


def test_3d_rope_tables_of_the_480p_grid():
    grid = (2, 10, 16)
    S = grid[0] * grid[1] * grid[2]
    cos, sin = rope_3d_tables(grid)
    x, w, b, nwq, nwk = make(2 * S, 512, 3, 128, True, seed=5)
    y = run_qkv(x, w, b, nwq, nwk, cos, sin, S)
    check_qkv(x, w, b, nwq, nwk, cos, sin, S, y)


@pytest.mark.parametrize(
    "R, form",
    [(126, "rotate-half"), (42, "rotate-half"), (2, "rotate-half"), (34, "rotate-half"), (96, "any"),
     (128, "rotate-half, read whole"), (64, "rotate-half, padded rows")],
)
def test_any_even_rotary_width(R, form):
    # widths that are not a multiple of 32 (R = 6 * 21 from a 21-frequency
    # 3D table, as _official_rope builds it: rank_local_io.py:74-80) and
    # tables in another form: partners from the token's other lanes, tables
    # read at every rotated column
    M, K, heads = 520, 256, 2
    x, w, b, nwq, nwk = make(M, K, heads, R, True, seed=R)
    if form == "any":
        g = torch.Generator().manual_seed(R)
        ang = torch.rand((M, R), generator=g) * 6.0
        cos, sin = ang.cos(), ang.sin()
        assert not rotate_half_tables(cos, sin)
    else:
        cos, sin = tables(M, R, seed=3)
    if form == "rotate-half, padded rows":
        # rows of 66 floats (264 bytes: not 16-byte rows) holding 64 columns,
        # read in place: the epilogue reads every rotated column
        n = w.shape[0] // 3
        y = torch.empty((M, 3 * n), dtype=torch.bfloat16, device=DEV)
        wd = w.to(DEV)
        bd = b.to(DEV)
        secs = [
            Section(wd[:n], y[:, :n], bd[:n], nwq.to(DEV), 1e-6),
            Section(wd[n : 2 * n], y[:, n : 2 * n], bd[n : 2 * n], nwk.to(DEV), 1e-6),
            Section(wd[2 * n :], y[:, 2 * n :], bd[2 * n :]),
        ]
        full_c = torch.zeros((M, 66), device=DEV)
        full_s = torch.zeros((M, 66), device=DEV)
        full_c[:, :R], full_s[:, :R] = cos.to(DEV), sin.to(DEV)
        assert full_c[:, :R].stride(0) == 66
        proj_gemm(x.to(DEV), secs, full_c[:, :R], full_s[:, :R], M, rotate_half=True)
        torch.cuda.synchronize()
        check_qkv(x, w, b, nwq, nwk, cos, sin, M, y.cpu())
        return
    y = run_qkv(x, w, b, nwq, nwk, cos, sin, M, rotate_half=form == "rotate-half")
    check_qkv(x, w, b, nwq, nwk, cos, sin, M, y)
    # table rows wrapping per sequence, with sampled rows
    y = run_qkv(x, w, b, nwq, nwk, cos[:130], sin[:130], 130, rotate_half=form == "rotate-half")
    check_qkv(x, w, b, nwq, nwk, cos[:130], sin[:130], 130, y)


def test_more_tiles_than_cus():
    # 17 token tiles x 60 feature tiles: 1,020 workgroups (one per tile),
    # about four per CU, each XCD a contiguous range; the last token tile
    # ragged
    x, w, b, nwq, nwk = make(4096 + 96, 256, 40, 128, True, seed=7)
    cos, sin = tables(4192, 128, seed=1)
    y = run_qkv(x, w, b, nwq, nwk, cos, sin, 4192)
    check_qkv(x, w, b, nwq, nwk, cos, sin, 4192, y)


@pytest.mark.parametrize("M, heads", [(6240, 40), (49920, 40)])
def test_block_projection_shapes_on_sampled_rows(M, heads):
    # one 8-way Ulysses rank's 6,240 tokens and the full 49,920 at 40 heads
    # (hidden 5,120), table rows m mod S; rows sampled across the token tiles
    x, w, b, nwq, nwk = make(M, heads * 128, heads, 128, True, seed=M)
    cos, sin = tables(M, 128, seed=2)
    y = run_qkv(x, w, b, nwq, nwk, cos, sin, M)
    g = torch.Generator().manual_seed(M)
    rows = sorted(set(torch.randint(0, M, (40,), generator=g).tolist()) | {0, 255, 256, M - 1})
    check_qkv(x, w, b, nwq, nwk, cos, sin, M, y, rows=rows)


def test_plain_projection_matches_hipblaslt_linear():
    g = torch.Generator(device=DEV).manual_seed(3)
    x = torch.randn((4096 + 40, 5120), device=DEV, generator=g).to(torch.bfloat16)
    w = (torch.randn((5120, 5120), device=DEV, generator=g) / 72).to(torch.bfloat16)
    b = (0.1 * torch.randn(5120, device=DEV, generator=g)).to(torch.bfloat16)
    lin = torch.nn.Linear(5120, 5120, device=DEV, dtype=torch.bfloat16)
    lin.weight.data, lin.bias.data = w, b
    ours = out_projection(lin, x.view(1, -1, 5120))
    ref = torch.nn.functional.linear(x, w, b)
    torch.cuda.synchronize()
    assert ours is not None and ours.shape == (1, 4136, 5120)
    d = (ours.view_as(ref).float() - ref.float()).abs()
    ulp = 2.0 ** (torch.floor(torch.log2(ref.float().abs().clamp_min(1e-30))) - 7)
    assert (d <= ulp).all(), float((d / ulp).max())
    assert (d == 0).float().mean() > 0.99


def test_wide_plain_rows_take_the_staged_stores():
    # three plain sections writing 3 x 2,816 bf16 = 16.5 KiB rows: the rows
    # go out through LDS like the RoPE sections' (narrower launches store
    # from registers); every section within one ulp of hipBLASLt
    g = torch.Generator(device=DEV).manual_seed(11)
    m, k, n = 1000 + 40, 512, 2816
    x = torch.randn((m, k), device=DEV, generator=g).to(torch.bfloat16)
    w = (torch.randn((3 * n, k), device=DEV, generator=g) / k**0.5).to(torch.bfloat16)
    b = (0.1 * torch.randn(3 * n, device=DEV, generator=g)).to(torch.bfloat16)
    y = torch.empty((m, 3 * n), device=DEV, dtype=torch.bfloat16)
    proj_gemm(x, [Section(w[i * n : (i + 1) * n], y[:, i * n : (i + 1) * n], b[i * n : (i + 1) * n]) for i in range(3)])
    ref = torch.nn.functional.linear(x, w, b)
    torch.cuda.synchronize()
    d = (y.float() - ref.float()).abs()
    ulp = 2.0 ** (torch.floor(torch.log2(ref.float().abs().clamp_min(1e-30))) - 7)
    assert (d <= ulp).all(), float((d / ulp).max())
    assert (d == 0).float().mean() > 0.99


def test_repeated_launches_are_bitwise_identical():
    x, w, b, nwq, nwk = make(2000, 512, 4, 128, True, seed=9)
    cos, sin = tables(2000, 128)
    y1 = run_qkv(x, w, b, nwq, nwk, cos, sin, 2000)
    y2 = run_qkv(x, w, b, nwq, nwk, cos, sin, 2000)
    assert torch.equal(y1, y2)


class H3Attention(torch.nn.Module):
    """Stand-in with the attributes the processor protocol reads."""

    def __init__(self, heads: int, fused: bool) -> None:
        super().__init__()
        hidden = heads * 128
        self.heads = heads
        self.fused_projections = fused
        g = torch.Generator().manual_seed(heads + fused)
        init = lambda *shape: torch.randn(shape, generator=g) / shape[-1] ** 0.5  # noqa: E731
        if fused:
            self.to_qkv = torch.nn.Linear(hidden, 3 * hidden, bias=True)
            self.to_qkv.weight.data = init(3 * hidden, hidden)
        else:
            self.to_q, self.to_k, self.to_v = (torch.nn.Linear(hidden, hidden, bias=True) for _ in range(3))
            for lin in (self.to_q, self.to_k, self.to_v):
                lin.weight.data = init(hidden, hidden)
        self.norm_q = torch.nn.RMSNorm(128, eps=1e-6)
        self.norm_k = torch.nn.RMSNorm(128, eps=1e-6)
        self.norm_q.weight.data = 1.0 + 0.1 * torch.randn(128, generator=g)
        self.norm_k.weight.data = 1.0 + 0.1 * torch.randn(128, generator=g)
        self.to_out = torch.nn.ModuleList([torch.nn.Linear(hidden, hidden, bias=True), torch.nn.Dropout(0.0)])
        self.processor = None

    def set_processor(self, processor):
        self.processor = processor

    def forward(self, hidden_states, rotary_emb=None, attention_mask=None):
        return self.processor(self, hidden_states, rotary_emb, attention_mask)


@pytest.mark.parametrize("fused", [False, True])
def test_processor_with_fused_projections(fused):
    heads, grid = 2, (2, 10, 13)
    S = grid[0] * grid[1] * grid[2]
    attn = H3Attention(heads, fused).to(torch.bfloat16).to(DEV)
    x = torch.randn((1, S, heads * 128), generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(DEV)
    cos, sin = (t.to(DEV) for t in rope_3d_tables(grid))
    assert rotate_half_tables(cos, sin)
    assert qkv_projection(attn, x, (cos, sin)) is not None
    outs = {}
    for fuse, fuse_out in ((False, False), (True, False), (True, True)):
        processor = DenseMiniMaxH3Processor(fuse_projections=fuse, fuse_out_projection=fuse_out)
        attn.set_processor(processor)
        with torch.no_grad():
            outs[fuse, fuse_out] = attn(x, rotary_emb=(cos, sin)).float()
        assert processor.calls == 1
    torch.cuda.synchronize()
    # the paths differ only by where q/k are rounded (once in the fused
    # epilogue, twice in the separate steps) and the GEMMs' summation order
    for key in ((True, False), (True, True)):
        m = error_metrics(outs[key], outs[False, False])
        assert m["finite"] and m["relative_l2"] < 1e-2 and m["cosine"] > 0.9999, (key, m)


def test_tables_of_any_form_take_the_fused_launch():
    # tables that are not in the rotate-half form are read at every rotated
    # column: the fused launch runs and matches the separate steps
    attn = H3Attention(1, False).to(torch.bfloat16).to(DEV)
    x = torch.randn((1, 64, 128), device=DEV).to(torch.bfloat16)
    cos, sin = torch.rand((64, 128), device=DEV), torch.rand((64, 128), device=DEV)  # not rotate-half
    assert not rotate_half_tables(cos, sin)
    why = []
    fused = qkv_projection(attn, x, (cos, sin), why)
    assert fused is not None and why == []
    processor = DenseMiniMaxH3Processor(fuse_projections=False)
    attn.set_processor(processor)
    with torch.no_grad():
        q, k, v = processor._projections(attn, x, (cos, sin))
    torch.cuda.synchronize()
    for got, want in zip(fused, (q, k, v)):
        d = (got.float() - want.float()).abs()
        assert d.max() <= 2.0**-4 and d.mean() <= 2.0**-10, float(d.max())


def test_fallbacks_are_recorded_in_the_install_audit():
    class Transformer(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.blocks = torch.nn.ModuleList([H3Attention(1, False) for _ in range(2)])

    t = Transformer().to(torch.bfloat16).to(DEV)
    record = install_dense_hip(t, H3Attention, fuse_projections=True)
    assert record["fuse_projections"] is True and record["projection_fallbacks"] == {}
    x = torch.randn((1, 64, 128), device=DEV).to(torch.bfloat16)
    cos, sin = (z.to(DEV) for z in rope_3d_tables((1, 8, 8)))
    with torch.no_grad():
        for blk in t.blocks:
            blk(x, rotary_emb=(cos, sin))  # fused: nothing recorded
        assert record["projection_fallbacks"] == {}
        for blk in t.blocks:
            blk(x)  # no RoPE: the module's own norms, recorded per call
        odd = torch.rand((64, 7), device=DEV)
        with pytest.raises(ValueError):
            t.blocks[0](x, rotary_emb=(odd, odd))  # an odd width: recorded, then the prologue refuses it
    torch.cuda.synchronize()
    fb = record["projection_fallbacks"]
    assert fb["no rotary_emb: the module's own norms apply"] == 2
    assert sum(v for k, v in fb.items() if k.startswith("rotary tables of shape (64, 7)")) == 1
    assert qkv_projection(t.blocks[0], x, None) is None  # the module's own norms apply without RoPE
    # norms without an eps (torch's RMSNorm(eps=None)): the fused launch
    # declines with the reason, and the separate steps then refuse the module
    # with their own message, as for any norm they cannot fuse
    blk = t.blocks[1]
    blk.norm_k.eps = None
    why: list[str] = []
    assert qkv_projection(blk, x, (cos, sin), why) is None
    assert why == ["norm_q / norm_k carry no eps"]
    with torch.no_grad(), pytest.raises(RuntimeError, match="needs norm_q/norm_k"):
        blk(x, rotary_emb=(cos, sin))
    assert record["projection_fallbacks"]["norm_q / norm_k carry no eps"] == 1
