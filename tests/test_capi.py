"""The C-ABI library: it loads, exports every entry point include/h3attn.h
declares, and rejects bad arguments before any device work (runs without a
GPU: every call here returns from validation)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from h3_flash_amd import _ext

# These calls carry fake device pointers and must return from validation; on a
# host with a visible GPU a case that slipped through would launch on them, so
# they only run where no GPU is visible (the GPU tests cover real tensors).
host_only = pytest.mark.skipif(torch.cuda.is_available(), reason="fake device pointers: GPU-less hosts only")

HEADER = Path(__file__).resolve().parents[1] / "include" / "h3attn.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(h3a_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    return _ext.load_library()


def test_header_declares_the_expected_entry_points():
    assert declared_functions() == [
        "h3a_abi_version",
        "h3a_attn_fwd",
        "h3a_attn_fwd_noalloc",
        "h3a_attn_fwd_workspace_size",
        "h3a_attn_merge",
        "h3a_clock_sample",
        "h3a_last_error",
        "h3a_merge_heads",
        "h3a_pack_qkv",
        "h3a_proj_gemm",
        "h3a_qknorm_rope",
        "h3a_qknorm_rope_pack",
        "h3a_residual_gate_rmsnorm_modulate",
        "h3a_rmsnorm_modulate",
        "h3a_swiglu",
    ]


def test_library_exports_every_declared_function(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert name in _ext.SIGNATURES, name


def test_abi_version(lib):
    assert lib.h3a_abi_version() == _ext.ABI_VERSION == 4


def test_clock_sample_rejects_bad_pointers(lib):
    assert lib.h3a_clock_sample(None, None) == _ext.H3A_EINVAL
    assert b"NULL" in lib.h3a_last_error()
    assert lib.h3a_clock_sample(ctypes.c_void_p((1 << 20) + 4), None) == _ext.H3A_EINVAL
    assert b"aligned" in lib.h3a_last_error()


def _attn_args(**overrides):
    a = _ext.AttnArgs()
    a.abi_version = _ext.ABI_VERSION
    a.q = a.k = a.v = a.o = 1 << 20
    a.batch, a.heads, a.seqlen_q, a.seqlen_k, a.head_dim = 1, 1, 16, 16, 128
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        getattr(a, name)[:] = (16 * 128, 128, 128)
    a.lse_stride[:] = (16, 16)
    a.softmax_scale = 0.088
    for k, v in overrides.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "overrides, code, message",
    [
        ({"abi_version": 7}, _ext.H3A_EINVAL, "abi_version"),
        ({"causal": 1}, _ext.H3A_EUNSUPPORTED, "causal"),
        ({"head_dim": 64}, _ext.H3A_EUNSUPPORTED, "head_dim must be 128"),
        ({"heads": 0}, _ext.H3A_EINVAL, "extent"),
        ({"softmax_scale": 0.0}, _ext.H3A_EINVAL, "softmax_scale"),
        ({"softmax_scale": float("nan")}, _ext.H3A_EINVAL, "softmax_scale"),
        ({"q": None}, _ext.H3A_EINVAL, "NULL"),
        ({"k": (1 << 20) + 4}, _ext.H3A_EINVAL, "aligned"),
        ({"batch": 2, "cu_seqlens_q": 1 << 20, "cu_seqlens_k": 1 << 20, "num_segments": 1, "max_seqlen_q": 8},
         _ext.H3A_EINVAL, "batch == 1"),
        ({"cu_seqlens_q": 1 << 20, "num_segments": 1, "max_seqlen_q": 8}, _ext.H3A_EINVAL, "cu_seqlens_k"),
        ({"cu_seqlens_q": 1 << 20, "cu_seqlens_k": 1 << 20, "num_segments": 1, "max_seqlen_q": 99},
         _ext.H3A_EINVAL, "max_seqlen_q"),
        ({"q_stride": (ctypes.c_int64 * 3)(1 << 25, 1 << 21, 128)}, _ext.H3A_EUNSUPPORTED, "row stride"),
        # a row stride whose window span would overflow a 64-bit product
        ({"k_stride": (ctypes.c_int64 * 3)(1 << 62, 1 << 61, 128)}, _ext.H3A_EUNSUPPORTED, "row stride"),
        ({"lse": (1 << 20) + 2}, _ext.H3A_EINVAL, "lse must be 4-byte aligned"),
        ({"lse": 1 << 20, "lse_stride": (ctypes.c_int64 * 2)(-16, 16)}, _ext.H3A_EINVAL, "non-negative strides"),
        # extents that 32-bit launch fields would truncate
        ({"heads": (1 << 32) + 1}, _ext.H3A_EUNSUPPORTED, "below 2^31"),
        ({"batch": 1 << 31}, _ext.H3A_EUNSUPPORTED, "below 2^31"),
    ],
)
@host_only
def test_attn_validation(lib, overrides, code, message):
    a = _attn_args(**overrides)
    rc = lib.h3a_attn_fwd(ctypes.byref(a), None)
    assert rc == code
    assert message in _ext.last_error(lib)


@host_only
def test_attn_bad_strides(lib):
    a = _attn_args()
    a.k_stride[:] = (16 * 128, 100, 128)
    assert lib.h3a_attn_fwd(ctypes.byref(a), None) == _ext.H3A_EINVAL
    a = _attn_args()
    a.v_stride[:] = (16 * 128, 132, 4)
    assert lib.h3a_attn_fwd(ctypes.byref(a), None) == _ext.H3A_EINVAL


@host_only
def test_attn_null_args_and_empty_problem(lib):
    assert lib.h3a_attn_fwd(None, None) == _ext.H3A_EINVAL
    # empty problems return before any device work
    assert lib.h3a_attn_fwd(ctypes.byref(_attn_args(seqlen_q=0)), None) == _ext.H3A_OK
    assert lib.h3a_attn_fwd(ctypes.byref(_attn_args(batch=0)), None) == _ext.H3A_OK
    assert _ext.last_error(lib) == ""


def test_row_stride_limit_is_one_window_of_rows(lib):
    # 576 rows of a view must span under 2^31 bytes: 1,864,135 elements is
    # the largest sequence stride (1,864,128 the largest multiple of 8)
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        ok = _attn_args()
        getattr(ok, name)[:] = (0, 1_864_128, 128)
        assert lib.h3a_attn_fwd_workspace_size(ctypes.byref(ok)) >= 0, name
        bad = _attn_args()
        getattr(bad, name)[:] = (0, 1_864_136, 128)
        assert lib.h3a_attn_fwd_workspace_size(ctypes.byref(bad)) == _ext.H3A_EUNSUPPORTED, name
        assert "2^31" in _ext.last_error(lib)


def test_workspace_size_validates_like_the_launch(lib):
    # host-only call: no device work whether or not a GPU is visible
    assert lib.h3a_attn_fwd_workspace_size(None) == _ext.H3A_EINVAL
    assert lib.h3a_attn_fwd_workspace_size(ctypes.byref(_attn_args(head_dim=64))) == _ext.H3A_EUNSUPPORTED
    assert lib.h3a_attn_fwd_workspace_size(ctypes.byref(_attn_args(seqlen_q=0))) == 0
    assert lib.h3a_attn_fwd_workspace_size(ctypes.byref(_attn_args())) >= 0


def _rope_args(**overrides):
    a = _ext.QkNormRopeArgs()
    a.abi_version = _ext.ABI_VERSION
    a.xq = a.yq = a.wq = 1 << 20
    a.cos = a.sin = 1 << 21
    a.table_stride = 128
    a.batch, a.seqlen, a.heads, a.head_dim, a.rotary_dim = 1, 4, 2, 128, 128
    a.xq_stride[:] = a.yq_stride[:] = (4 * 2 * 128, 2 * 128, 128)
    a.eps_q = a.eps_k = 1e-5
    for k, v in overrides.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "overrides, code, message",
    [
        ({"rotary_dim": 3}, _ext.H3A_EINVAL, "even rotary dimension no wider than the head"),
        ({"rotary_dim": 130}, _ext.H3A_EINVAL, "even rotary dimension no wider than the head"),
        ({"head_dim": 100, "rotary_dim": 96}, _ext.H3A_EUNSUPPORTED, "multiple of 8"),
        ({"w_dtype": 5}, _ext.H3A_EINVAL, "weight dtype"),
        ({"xk": 1 << 20}, _ext.H3A_EINVAL, "xk given without"),
        ({"cos": None}, _ext.H3A_EINVAL, "cos/sin"),
        ({"table_stride": 64}, _ext.H3A_EINVAL, "table_stride"),
        ({"sin": (1 << 21) + 2}, _ext.H3A_EINVAL, "cos/sin must be 4-byte aligned"),
        ({"abi_version": 0}, _ext.H3A_EINVAL, "abi_version"),
        ({"seqlen": 1 << 40, "heads": 1 << 40}, _ext.H3A_EUNSUPPORTED, "limits 2^31"),  # no 64-bit wrap
    ],
)
@host_only
def test_rope_validation(lib, overrides, code, message):
    a = _rope_args(**overrides)
    assert lib.h3a_qknorm_rope(ctypes.byref(a), None) == code
    assert message in _ext.last_error(lib)


def _pack_args(**overrides):
    a = _ext.PackQkvArgs()
    a.abi_version = _ext.ABI_VERSION
    a.q = a.k = a.v = 1 << 20
    a.out = 1 << 22
    a.elem_bytes = 2
    a.rows, a.heads, a.head_dim, a.world = 4, 8, 128, 2
    for name in ("q_stride", "k_stride", "v_stride"):
        getattr(a, name)[:] = (8 * 128, 128)
    for k, v in overrides.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "overrides, code, message",
    [
        ({"abi_version": 1}, _ext.H3A_EINVAL, "abi_version"),
        ({"heads": 6, "world": 4}, _ext.H3A_EINVAL, "heads (6) must divide Ulysses degree (4)"),
        ({"elem_bytes": 3}, _ext.H3A_EINVAL, "elem_bytes"),
        ({"world": 0}, _ext.H3A_EINVAL, "extents"),
        ({"head_dim": 0}, _ext.H3A_EINVAL, "extents"),
        ({"v": None}, _ext.H3A_EINVAL, "NULL"),
        ({"rows": 1 << 28}, _ext.H3A_EUNSUPPORTED, "2^31"),
        ({"rows": 1 << 40, "heads": 1 << 40, "world": 1}, _ext.H3A_EUNSUPPORTED, "2^31"),  # no 64-bit wrap
        ({"head_dim": 1 << 62}, _ext.H3A_EUNSUPPORTED, "2^30"),
    ],
)
@host_only
def test_pack_validation(lib, overrides, code, message):
    a = _pack_args(**overrides)
    assert lib.h3a_pack_qkv(ctypes.byref(a), None) == code
    assert message in _ext.last_error(lib)


@host_only
def test_pack_negative_stride_and_empty(lib):
    a = _pack_args()
    a.k_stride[:] = (-1024, 128)
    assert lib.h3a_pack_qkv(ctypes.byref(a), None) == _ext.H3A_EINVAL
    assert lib.h3a_pack_qkv(ctypes.byref(_pack_args(rows=0)), None) == _ext.H3A_OK
    assert lib.h3a_pack_qkv(None, None) == _ext.H3A_EINVAL


def _merge_args(**overrides):
    a = _ext.MergeHeadsArgs()
    a.abi_version = _ext.ABI_VERSION
    a.x, a.out = 1 << 20, 1 << 22
    a.elem_bytes, a.world, a.rows, a.inner = 2, 4, 8, 640
    a.x_stride[:] = (8 * 640, 640)
    for k, v in overrides.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "overrides, code, message",
    [
        ({"abi_version": 9}, _ext.H3A_EINVAL, "abi_version"),
        ({"elem_bytes": 0}, _ext.H3A_EINVAL, "elem_bytes"),
        ({"world": 0}, _ext.H3A_EINVAL, "extents"),
        ({"rows": -1}, _ext.H3A_EINVAL, "extents"),
        ({"x": None}, _ext.H3A_EINVAL, "NULL"),
    ],
)
@host_only
def test_merge_validation(lib, overrides, code, message):
    a = _merge_args(**overrides)
    assert lib.h3a_merge_heads(ctypes.byref(a), None) == code
    assert message in _ext.last_error(lib)


@host_only
def test_merge_empty(lib):
    assert lib.h3a_merge_heads(ctypes.byref(_merge_args(rows=0)), None) == _ext.H3A_OK
    assert lib.h3a_merge_heads(ctypes.byref(_merge_args(inner=0)), None) == _ext.H3A_OK


def _rope_pack_args(**overrides):
    a = _ext.QkNormRopePackArgs()
    a.abi_version = _ext.ABI_VERSION
    a.q = a.k = a.v = a.wq = a.wk = 1 << 20
    a.out = 1 << 22
    a.cos = a.sin = 1 << 21
    a.table_stride = 128
    a.rows, a.heads, a.head_dim, a.rotary_dim, a.world = 4, 8, 128, 128, 2
    for name in ("q_stride", "k_stride", "v_stride"):
        getattr(a, name)[:] = (8 * 128, 128)
    a.eps_q = a.eps_k = 1e-5
    for k, v in overrides.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "overrides, code, message",
    [
        ({"abi_version": 2}, _ext.H3A_EINVAL, "abi_version"),
        ({"rotary_dim": 7}, _ext.H3A_EINVAL, "even rotary dimension no wider than the head"),
        ({"heads": 8, "world": 3}, _ext.H3A_EINVAL, "heads (8) must divide Ulysses degree (3)"),
        ({"cos": (1 << 21) + 2}, _ext.H3A_EINVAL, "cos/sin must be 4-byte aligned"),
        ({"head_dim": 100, "rotary_dim": 96}, _ext.H3A_EUNSUPPORTED, "multiple of 8"),
        ({"out": None}, _ext.H3A_EINVAL, "NULL"),
        ({"k": (1 << 20) + 2}, _ext.H3A_EINVAL, "aligned"),
        ({"w_dtype": 3}, _ext.H3A_EINVAL, "weight dtype"),
    ],
)
@host_only
def test_rope_pack_validation(lib, overrides, code, message):
    a = _rope_pack_args(**overrides)
    assert lib.h3a_qknorm_rope_pack(ctypes.byref(a), None) == code
    assert message in _ext.last_error(lib)


@pytest.mark.parametrize("overrides", [{"rotary_dim": 42}, {"rotary_dim": 126}, {"rotary_dim": 2}, {"cos": (1 << 21) + 4}])
@host_only
def test_rope_pack_takes_every_even_width_and_4_byte_tables(lib, overrides):
    # validation passes; on a host without a GPU the launch itself fails
    a = _rope_pack_args(**overrides)
    assert lib.h3a_qknorm_rope_pack(ctypes.byref(a), None) == _ext.H3A_ELAUNCH
    assert "launch failed" in _ext.last_error(lib)


def _modulate_args(**overrides):
    a = _ext.RmsnormModulateArgs()
    a.abi_version = _ext.ABI_VERSION
    a.x, a.out, a.weight, a.scale, a.shift, a.index = 1 << 20, 1 << 22, 1 << 23, 1 << 24, 1 << 25, 1 << 26
    a.w_dtype = a.table_dtype = _ext.H3A_DTYPE_BF16
    a.index_dtype = _ext.H3A_DTYPE_I64
    a.scale_stride = a.shift_stride = 6 * 512
    a.table_rows, a.n_index, a.rows, a.cols = 9, 16, 16, 512
    a.x_stride = a.out_stride = 512
    a.eps = 1e-5
    for k, v in overrides.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "overrides, code, message",
    [
        ({"abi_version": 0}, _ext.H3A_EINVAL, "abi_version"),
        ({"cols": 0}, _ext.H3A_EINVAL, "extents"),
        ({"rows": -3}, _ext.H3A_EINVAL, "extents"),
        ({"w_dtype": 2}, _ext.H3A_EINVAL, "weight dtype"),
        ({"table_dtype": 3}, _ext.H3A_EINVAL, "table dtype"),
        ({"index_dtype": _ext.H3A_DTYPE_F32}, _ext.H3A_EINVAL, "int32 or int64"),
        ({"n_index": 0}, _ext.H3A_EINVAL, "n_index"),
        ({"table_rows": 0}, _ext.H3A_EINVAL, "table_rows"),
        ({"eps": -1.0}, _ext.H3A_EINVAL, "eps"),
        ({"scale_stride": 100}, _ext.H3A_EINVAL, "table row stride"),
        ({"x_stride": 100}, _ext.H3A_EINVAL, "x row stride"),
        ({"shift": None}, _ext.H3A_EINVAL, "NULL"),
        ({"out": None}, _ext.H3A_EINVAL, "NULL out"),
    ],
)
@host_only
def test_modulate_validation(lib, overrides, code, message):
    a = _modulate_args(**overrides)
    assert lib.h3a_rmsnorm_modulate(ctypes.byref(a), None) == code
    assert message in _ext.last_error(lib)


@host_only
def test_residual_modulate_validation(lib):
    a = _ext.ResidualGateRmsnormModulateArgs()
    a.abi_version = _ext.ABI_VERSION
    a.residual = a.branch = a.hidden_out = a.normed_out = 1 << 20
    a.weight = a.gate = a.scale = a.shift = a.index = 1 << 22
    a.index_dtype = _ext.H3A_DTYPE_I32
    a.gate_stride = a.scale_stride = a.shift_stride = 64
    a.table_rows, a.n_index, a.rows, a.cols = 4, 4, 8, 64
    a.residual_stride = a.branch_stride = a.hidden_stride = a.normed_stride = 64
    a.gate_stride = 32
    assert lib.h3a_residual_gate_rmsnorm_modulate(ctypes.byref(a), None) == _ext.H3A_EINVAL
    assert "table row stride" in _ext.last_error(lib)
    a.gate_stride, a.hidden_out = 64, None
    assert lib.h3a_residual_gate_rmsnorm_modulate(ctypes.byref(a), None) == _ext.H3A_EINVAL
    assert "hidden_out" in _ext.last_error(lib)
    a.rows = 0
    a.hidden_out = 1 << 20
    assert lib.h3a_residual_gate_rmsnorm_modulate(ctypes.byref(a), None) == _ext.H3A_OK


@host_only
def test_swiglu_validation(lib):
    a = _ext.SwigluArgs()
    a.abi_version = _ext.ABI_VERSION
    a.x, a.out = 1 << 20, 1 << 22
    a.rows, a.cols, a.x_stride, a.out_stride = 4, 64, 100, 64
    assert lib.h3a_swiglu(ctypes.byref(a), None) == _ext.H3A_EINVAL
    assert "2*cols" in _ext.last_error(lib)
    a.x_stride, a.x = 128, None
    assert lib.h3a_swiglu(ctypes.byref(a), None) == _ext.H3A_EINVAL
    a.rows = 0
    assert lib.h3a_swiglu(ctypes.byref(a), None) == _ext.H3A_OK
    assert lib.h3a_swiglu(None, None) == _ext.H3A_EINVAL


def _attn_merge_args(**overrides):
    a = _ext.AttnMergeArgs()
    a.abi_version = _ext.ABI_VERSION
    a.n_parts = 2
    a.o_parts[0], a.o_parts[1] = 1 << 20, 1 << 21
    a.lse_parts[0], a.lse_parts[1] = 1 << 22, 1 << 23
    a.part_dtype = a.out_dtype = _ext.H3A_DTYPE_BF16
    a.o, a.lse = 1 << 24, 1 << 25
    a.batch, a.heads, a.seqlen, a.head_dim = 1, 2, 8, 128
    a.part_o_stride[:] = a.o_stride[:] = (8 * 2 * 128, 2 * 128, 128)
    a.part_lse_stride[:] = a.lse_stride[:] = (2 * 8, 8)
    for k, v in overrides.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "overrides, code, message",
    [
        ({"abi_version": 2}, _ext.H3A_EINVAL, "abi_version"),
        ({"n_parts": 0}, _ext.H3A_EINVAL, "n_parts"),
        ({"n_parts": 17}, _ext.H3A_EINVAL, "n_parts"),
        ({"head_dim": 100}, _ext.H3A_EUNSUPPORTED, "multiple of 8"),
        ({"heads": 0}, _ext.H3A_EINVAL, "extents"),
        ({"part_dtype": _ext.H3A_DTYPE_I32}, _ext.H3A_EINVAL, "bf16 or fp32"),
        ({"o": None}, _ext.H3A_EINVAL, "NULL output"),
        ({"o": (1 << 24) + 8}, _ext.H3A_EINVAL, "aligned"),
        ({"batch": 1 << 30, "seqlen": 1 << 30, "heads": 1 << 30}, _ext.H3A_EUNSUPPORTED, "too many rows"),
        # under 2^40 rows, but one extent past the 32-bit launch fields
        ({"seqlen": 1 << 33, "heads": 1}, _ext.H3A_EUNSUPPORTED, "too many rows"),
        ({"heads": 1 << 32, "seqlen": 2}, _ext.H3A_EUNSUPPORTED, "too many rows"),
    ],
)
@host_only
def test_attn_merge_validation(lib, overrides, code, message):
    a = _attn_merge_args(**overrides)
    assert lib.h3a_attn_merge(ctypes.byref(a), None) == code
    assert message in _ext.last_error(lib)


@host_only
def test_attn_merge_null_part_and_empty(lib):
    a = _attn_merge_args()
    a.lse_parts[1] = None
    assert lib.h3a_attn_merge(ctypes.byref(a), None) == _ext.H3A_EINVAL
    assert "NULL part 1" in _ext.last_error(lib)
    a = _attn_merge_args()
    a.o_stride[:] = (8 * 2 * 128, 2 * 128, 100)
    assert lib.h3a_attn_merge(ctypes.byref(a), None) == _ext.H3A_EINVAL
    assert lib.h3a_attn_merge(ctypes.byref(_attn_merge_args(seqlen=0)), None) == _ext.H3A_OK
    a = _attn_merge_args()
    a.lse_parts[0] = (1 << 22) + 2
    assert lib.h3a_attn_merge(ctypes.byref(a), None) == _ext.H3A_EINVAL
    assert "LSE of part 0 must be 4-byte aligned" in _ext.last_error(lib)
    a = _attn_merge_args()
    a.part_lse_stride[:] = (-8, 8)
    assert lib.h3a_attn_merge(ctypes.byref(a), None) == _ext.H3A_EINVAL
    assert "LSE strides must be non-negative" in _ext.last_error(lib)


def _proj_args(n_sections=3, **overrides):
    a = _ext.ProjArgs()
    a.abi_version = _ext.ABI_VERSION
    a.x = 1 << 20
    a.x_stride, a.m, a.k, a.head_dim = 256, 300, 256, 128
    a.num_sections = n_sections
    for i in range(n_sections):
        d = a.sections[i]
        d.weight, d.weight_stride, d.n = (1 << 24) + i * (1 << 20), 256, 256
        d.y, d.y_stride = (1 << 28) + i * 512, 768
        d.mode = _ext.H3A_PROJ_QKNORM_ROPE if i < 2 else _ext.H3A_PROJ_PLAIN
        d.norm_weight, d.eps = 1 << 22, 1e-6
    a.cos, a.sin, a.table_stride, a.rotary_dim, a.seqlen = 1 << 21, (1 << 21) + (1 << 19), 128, 128, 300
    a.rotate_half_tables = 1
    for k, v in overrides.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "overrides, code, message",
    [
        ({"abi_version": 3}, _ext.H3A_EINVAL, "abi_version"),
        ({"head_dim": 64}, _ext.H3A_EUNSUPPORTED, "head_dim must be 128"),
        ({"num_sections": 0}, _ext.H3A_EINVAL, "num_sections"),
        ({"num_sections": 4}, _ext.H3A_EINVAL, "num_sections"),
        ({"k": 200, "x_stride": 256}, _ext.H3A_EUNSUPPORTED, "multiple of 128"),
        ({"rotary_dim": 45}, _ext.H3A_EINVAL, "even rotary dimension no wider than the head"),
        ({"rotary_dim": 130}, _ext.H3A_EINVAL, "even rotary dimension no wider than the head"),
        ({"x": (1 << 20) + 8}, _ext.H3A_EINVAL, "x must be a 16-byte aligned"),
        ({"x_stride": 252}, _ext.H3A_EINVAL, "x_stride"),
        ({"cos": None}, _ext.H3A_EINVAL, "NULL cos/sin"),
        ({"table_stride": 64}, _ext.H3A_EINVAL, "table_stride"),
        ({"sin": (1 << 21) + 2}, _ext.H3A_EINVAL, "4-byte aligned"),
        ({"seqlen": 0}, _ext.H3A_EINVAL, "seqlen"),
        ({"seqlen": 1 << 23}, _ext.H3A_EUNSUPPORTED, "less than 2^32 bytes"),  # 8M rows x 512 bytes
        ({"table_stride": 1 << 62}, _ext.H3A_EUNSUPPORTED, "less than 2^32 bytes"),  # no 64-bit overflow
        ({"x_stride": 1 << 61}, _ext.H3A_EUNSUPPORTED, "x_stride too large"),
        ({"m": -1}, _ext.H3A_EINVAL, "extents"),
    ],
)
@host_only
def test_proj_gemm_validation(lib, overrides, code, message):
    a = _proj_args(**overrides)
    assert lib.h3a_proj_gemm(ctypes.byref(a), None) == code
    assert message in _ext.last_error(lib)


@pytest.mark.parametrize(
    "overrides",
    [
        {"rotary_dim": 126, "table_stride": 126},  # any even width, rows of any length
        {"rotary_dim": 2},
        {"rotary_dim": 48},
        {"rotate_half_tables": 0},  # tables of any form
        {"sin": (1 << 21) + 8},  # 4-byte aligned tables
    ],
)
@host_only
def test_proj_gemm_takes_any_even_width_and_table_form(lib, overrides):
    # validation passes; on a host without a GPU the launch itself fails
    a = _proj_args(**overrides)
    assert lib.h3a_proj_gemm(ctypes.byref(a), None) == _ext.H3A_ELAUNCH
    assert "launch failed" in _ext.last_error(lib)


@host_only
def test_proj_gemm_section_validation(lib):
    for field, value, message in [
        ("n", 200, "multiple of 128"),
        ("weight", (1 << 24) + 4, "16-byte aligned"),
        ("weight_stride", 100, "strides"),
        ("y_stride", 100, "strides"),
        ("mode", 7, "unknown mode"),
        ("bias", (1 << 23) + 4, "bias must be 8-byte aligned"),
        ("norm_weight", None, "norm_weight"),
        ("y_stride", 1 << 25, "y_stride too large"),  # 127 rows of 64 MiB pass 2^32 bytes
        ("y_stride", 1 << 61, "y_stride too large"),  # would overflow a 64-bit product
        ("weight_stride", 1 << 61, "weight_stride too large"),
    ]:
        a = _proj_args()
        setattr(a.sections[0], field, value)
        assert lib.h3a_proj_gemm(ctypes.byref(a), None) != _ext.H3A_OK, field
        assert message in _ext.last_error(lib), (field, _ext.last_error(lib))
    # plain sections only: no tables needed, rotary_dim and the table flag ignored
    a = _proj_args(n_sections=1, rotary_dim=48, rotate_half_tables=0, cos=None, sin=None, m=0)
    a.sections[0].mode = _ext.H3A_PROJ_PLAIN
    assert lib.h3a_proj_gemm(ctypes.byref(a), None) == _ext.H3A_OK
    assert lib.h3a_proj_gemm(None, None) == _ext.H3A_EINVAL
