"""ctypes binding of the C ABI in ``include/h3attn.h``.

The structures below mirror the header's argument structs field for field. Loading fails loudly (``RuntimeError``) when the library has
not been built: there is no other implementation behind these entry points.
"""

from __future__ import annotations

import ctypes
import hashlib
import threading
from pathlib import Path

from ._build import LIB_PATH

ABI_VERSION = 4

H3A_OK = 0
H3A_EINVAL = -1
H3A_EUNSUPPORTED = -2
H3A_ELAUNCH = -3

H3A_DTYPE_BF16 = 0
H3A_DTYPE_F32 = 1
H3A_DTYPE_I32 = 2
H3A_DTYPE_I64 = 3

# Bytes of the device array behind h3a_attn_fwd_noalloc (H3A_NOALLOC_SCRATCH_BYTES).
H3A_NOALLOC_SCRATCH_BYTES = 64 << 20

_I64x3 = ctypes.c_int64 * 3
_I64x2 = ctypes.c_int64 * 2


class AttnArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("batch", ctypes.c_int64),
        ("heads", ctypes.c_int64),
        ("seqlen_q", ctypes.c_int64),
        ("seqlen_k", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("q_stride", _I64x3),
        ("k_stride", _I64x3),
        ("v_stride", _I64x3),
        ("o_stride", _I64x3),
        ("lse_stride", _I64x2),
        ("softmax_scale", ctypes.c_float),
        ("causal", ctypes.c_int32),
        ("cu_seqlens_q", ctypes.c_void_p),
        ("cu_seqlens_k", ctypes.c_void_p),
        ("num_segments", ctypes.c_int32),
        ("max_seqlen_q", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_int64),
    ]


class QkNormRopeArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("xq", ctypes.c_void_p),
        ("xk", ctypes.c_void_p),
        ("yq", ctypes.c_void_p),
        ("yk", ctypes.c_void_p),
        ("wq", ctypes.c_void_p),
        ("wk", ctypes.c_void_p),
        ("w_dtype", ctypes.c_int32),
        ("cos", ctypes.c_void_p),
        ("sin", ctypes.c_void_p),
        ("table_stride", ctypes.c_int64),
        ("batch", ctypes.c_int64),
        ("seqlen", ctypes.c_int64),
        ("heads", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("rotary_dim", ctypes.c_int64),
        ("xq_stride", _I64x3),
        ("xk_stride", _I64x3),
        ("yq_stride", _I64x3),
        ("yk_stride", _I64x3),
        ("eps_q", ctypes.c_float),
        ("eps_k", ctypes.c_float),
    ]


class PackQkvArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("elem_bytes", ctypes.c_int64),
        ("rows", ctypes.c_int64),
        ("heads", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("world", ctypes.c_int64),
        ("q_stride", _I64x2),
        ("k_stride", _I64x2),
        ("v_stride", _I64x2),
    ]


class MergeHeadsArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("x", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("elem_bytes", ctypes.c_int64),
        ("world", ctypes.c_int64),
        ("rows", ctypes.c_int64),
        ("inner", ctypes.c_int64),
        ("x_stride", _I64x2),
    ]


class QkNormRopePackArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("wq", ctypes.c_void_p),
        ("wk", ctypes.c_void_p),
        ("w_dtype", ctypes.c_int32),
        ("cos", ctypes.c_void_p),
        ("sin", ctypes.c_void_p),
        ("table_stride", ctypes.c_int64),
        ("rows", ctypes.c_int64),
        ("heads", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("rotary_dim", ctypes.c_int64),
        ("world", ctypes.c_int64),
        ("q_stride", _I64x2),
        ("k_stride", _I64x2),
        ("v_stride", _I64x2),
        ("eps_q", ctypes.c_float),
        ("eps_k", ctypes.c_float),
    ]


class RmsnormModulateArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("x", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("weight", ctypes.c_void_p),
        ("w_dtype", ctypes.c_int32),
        ("scale", ctypes.c_void_p),
        ("shift", ctypes.c_void_p),
        ("table_dtype", ctypes.c_int32),
        ("scale_stride", ctypes.c_int64),
        ("shift_stride", ctypes.c_int64),
        ("table_rows", ctypes.c_int64),
        ("index", ctypes.c_void_p),
        ("index_dtype", ctypes.c_int32),
        ("n_index", ctypes.c_int64),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("x_stride", ctypes.c_int64),
        ("out_stride", ctypes.c_int64),
        ("eps", ctypes.c_float),
    ]


class ResidualGateRmsnormModulateArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("residual", ctypes.c_void_p),
        ("branch", ctypes.c_void_p),
        ("hidden_out", ctypes.c_void_p),
        ("normed_out", ctypes.c_void_p),
        ("weight", ctypes.c_void_p),
        ("w_dtype", ctypes.c_int32),
        ("gate", ctypes.c_void_p),
        ("scale", ctypes.c_void_p),
        ("shift", ctypes.c_void_p),
        ("table_dtype", ctypes.c_int32),
        ("gate_stride", ctypes.c_int64),
        ("scale_stride", ctypes.c_int64),
        ("shift_stride", ctypes.c_int64),
        ("table_rows", ctypes.c_int64),
        ("index", ctypes.c_void_p),
        ("index_dtype", ctypes.c_int32),
        ("n_index", ctypes.c_int64),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("residual_stride", ctypes.c_int64),
        ("branch_stride", ctypes.c_int64),
        ("hidden_stride", ctypes.c_int64),
        ("normed_stride", ctypes.c_int64),
        ("eps", ctypes.c_float),
    ]


class SwigluArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("x", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("x_stride", ctypes.c_int64),
        ("out_stride", ctypes.c_int64),
    ]


H3A_MERGE_MAX_PARTS = 16
_PtrParts = ctypes.c_void_p * H3A_MERGE_MAX_PARTS


class AttnMergeArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("n_parts", ctypes.c_int32),
        ("o_parts", _PtrParts),
        ("lse_parts", _PtrParts),
        ("part_dtype", ctypes.c_int32),
        ("o", ctypes.c_void_p),
        ("out_dtype", ctypes.c_int32),
        ("lse", ctypes.c_void_p),
        ("batch", ctypes.c_int64),
        ("heads", ctypes.c_int64),
        ("seqlen", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("part_o_stride", _I64x3),
        ("part_lse_stride", _I64x2),
        ("o_stride", _I64x3),
        ("lse_stride", _I64x2),
    ]


H3A_PROJ_PLAIN = 0
H3A_PROJ_QKNORM_ROPE = 1
H3A_PROJ_MAX_SECTIONS = 3
H3A_CLOCK_RECORDS = 2048  # records of one h3a_clock_sample launch


class ProjSection(ctypes.Structure):
    _fields_ = [
        ("weight", ctypes.c_void_p),
        ("weight_stride", ctypes.c_int64),
        ("n", ctypes.c_int64),
        ("bias", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("y_stride", ctypes.c_int64),
        ("mode", ctypes.c_int32),
        ("norm_weight", ctypes.c_void_p),
        ("eps", ctypes.c_float),
    ]


class ProjArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("x", ctypes.c_void_p),
        ("x_stride", ctypes.c_int64),
        ("m", ctypes.c_int64),
        ("k", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("num_sections", ctypes.c_int32),
        ("sections", ProjSection * H3A_PROJ_MAX_SECTIONS),
        ("cos", ctypes.c_void_p),
        ("sin", ctypes.c_void_p),
        ("table_stride", ctypes.c_int64),
        ("rotary_dim", ctypes.c_int64),
        ("seqlen", ctypes.c_int64),
        ("rotate_half_tables", ctypes.c_int32),
    ]


# Every function the header declares, with its ctypes signature.
SIGNATURES = {
    "h3a_attn_fwd": (ctypes.c_int, [ctypes.POINTER(AttnArgs), ctypes.c_void_p]),
    "h3a_attn_fwd_workspace_size": (ctypes.c_int64, [ctypes.POINTER(AttnArgs)]),
    "h3a_attn_fwd_noalloc": (ctypes.c_int, [ctypes.POINTER(AttnArgs), ctypes.c_void_p]),
    "h3a_qknorm_rope": (ctypes.c_int, [ctypes.POINTER(QkNormRopeArgs), ctypes.c_void_p]),
    "h3a_pack_qkv": (ctypes.c_int, [ctypes.POINTER(PackQkvArgs), ctypes.c_void_p]),
    "h3a_merge_heads": (ctypes.c_int, [ctypes.POINTER(MergeHeadsArgs), ctypes.c_void_p]),
    "h3a_qknorm_rope_pack": (ctypes.c_int, [ctypes.POINTER(QkNormRopePackArgs), ctypes.c_void_p]),
    "h3a_rmsnorm_modulate": (ctypes.c_int, [ctypes.POINTER(RmsnormModulateArgs), ctypes.c_void_p]),
    "h3a_residual_gate_rmsnorm_modulate": (
        ctypes.c_int,
        [ctypes.POINTER(ResidualGateRmsnormModulateArgs), ctypes.c_void_p],
    ),
    "h3a_swiglu": (ctypes.c_int, [ctypes.POINTER(SwigluArgs), ctypes.c_void_p]),
    "h3a_attn_merge": (ctypes.c_int, [ctypes.POINTER(AttnMergeArgs), ctypes.c_void_p]),
    "h3a_proj_gemm": (ctypes.c_int, [ctypes.POINTER(ProjArgs), ctypes.c_void_p]),
    "h3a_clock_sample": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "h3a_last_error": (ctypes.c_char_p, []),
    "h3a_abi_version": (ctypes.c_int, []),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library_path() -> Path:
    return LIB_PATH


def load_library(path: Path | None = None) -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise RuntimeError if absent."""

    global _lib
    target = Path(path) if path is not None else LIB_PATH
    with _lock:
        if _lib is not None and path is None:
            return _lib
        if not target.is_file():
            raise RuntimeError(
                f"HIP attention library not found at {target}; build it with "
                "`python -m h3_flash_amd._build` (hipcc, gfx950)"
            )
        lib = ctypes.CDLL(str(target))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.h3a_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(
                f"HIP attention library ABI {version} does not match binding ABI {ABI_VERSION}"
            )
        if path is None:
            _lib = lib
        return lib


def last_error(lib: ctypes.CDLL) -> str:
    message = lib.h3a_last_error()
    return message.decode("utf-8", "replace") if message else ""


def provenance() -> dict:
    """Identity of the loaded library, for install-time audit records."""

    lib = load_library()
    digest = hashlib.sha256(LIB_PATH.read_bytes()).hexdigest()
    return {
        "library": str(LIB_PATH),
        "abi_version": int(lib.h3a_abi_version()),
        "arch": "gfx950",
        "sha256": digest,
    }
