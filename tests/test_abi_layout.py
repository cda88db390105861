"""The ctypes structures in h3_flash_amd/_ext.py against the C header: a C
program compiled from include/h3attn.h prints sizeof and offsetof of every
field that the binding declares, and both must agree (a field missing from
the header fails to compile)."""

from __future__ import annotations

import ctypes
import json
import shutil
import subprocess
from pathlib import Path

import pytest

from h3_flash_amd import _ext

ROOT = Path(__file__).resolve().parents[1]
STRUCTS = {
    "h3a_attn_args": _ext.AttnArgs,
    "h3a_qknorm_rope_args": _ext.QkNormRopeArgs,
    "h3a_pack_qkv_args": _ext.PackQkvArgs,
    "h3a_merge_heads_args": _ext.MergeHeadsArgs,
    "h3a_qknorm_rope_pack_args": _ext.QkNormRopePackArgs,
    "h3a_rmsnorm_modulate_args": _ext.RmsnormModulateArgs,
    "h3a_residual_gate_rmsnorm_modulate_args": _ext.ResidualGateRmsnormModulateArgs,
    "h3a_swiglu_args": _ext.SwigluArgs,
    "h3a_attn_merge_args": _ext.AttnMergeArgs,
    "h3a_proj_section": _ext.ProjSection,
    "h3a_proj_args": _ext.ProjArgs,
}


@pytest.fixture(scope="module")
def c_layout(tmp_path_factory):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    lines = ["#include <stddef.h>", "#include <stdio.h>", '#include "h3attn.h"', "int main(void) {", 'printf("{");']
    first = True
    for cname, cls in STRUCTS.items():
        sep = "" if first else ","
        first = False
        lines.append(f'printf("{sep}\\"{cname}\\": {{\\"size\\": %zu", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'printf(", \\"{field}\\": %zu", offsetof({cname}, {field}));')
        lines.append('printf("}");')
    lines += ['printf("}\\n");', "return 0;", "}"]
    d = tmp_path_factory.mktemp("abi")
    src, exe = d / "layout.c", d / "layout"
    src.write_text("\n".join(lines) + "\n")
    subprocess.run([cc, "-std=c11", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    return json.loads(subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout)


@pytest.mark.parametrize("cname", sorted(STRUCTS))
def test_ctypes_structure_matches_the_header(c_layout, cname):
    cls = STRUCTS[cname]
    want = c_layout[cname]
    assert ctypes.sizeof(cls) == want["size"], (cname, ctypes.sizeof(cls), want["size"])
    for field, _ in cls._fields_:
        assert getattr(cls, field).offset == want[field], (cname, field)
