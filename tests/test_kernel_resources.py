"""Register and scratch use of every kernel in the built library.

The library's gfx950 code objects carry the compiler's per-kernel metadata
(the AMDGPU note of each code object, a msgpack map): the private segment
size (scratch bytes per lane), the VGPR / AGPR counts and the spill counts.
Scratch traffic in the attention kernel's key loop would cost bandwidth and
issue slots on every key tile, and the wide forms (views whose span reaches
2^31 bytes) sit at the 256-register limit of two waves per SIMD, where a
change elsewhere in the kernel easily tips them into spilling. So:

* no kernel uses scratch (private segment 0, no VGPR spills);
* the attention forms run one 512-thread workgroup per CU: two waves per
  SIMD (at most 256 VGPRs + AGPRs per wave) and at most the CU's 160 KiB of
  LDS.

Reads the built library only (skipped where it has not been built); the
parse needs no GPU.
"""

from __future__ import annotations

import struct

import pytest

from h3_flash_amd._build import LIB_PATH

msgpack = pytest.importorskip("msgpack")

BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
SHT_NOTE = 7
NT_AMDGPU_METADATA = 32


def elf_sections(elf: bytes) -> dict[str, tuple[int, int, int]]:
    """name -> (file offset, size, type) of an ELF64 little-endian file."""

    shoff = struct.unpack_from("<Q", elf, 0x28)[0]
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", elf, 0x3A)
    headers = [struct.unpack_from("<IIQQQQIIQQ", elf, shoff + i * shentsize) for i in range(shnum)]
    names_at = headers[shstrndx][4]

    def name(off: int) -> str:
        end = elf.index(b"\0", names_at + off)
        return elf[names_at + off : end].decode()

    return {name(h[0]): (h[4], h[5], h[1]) for h in headers}


def gfx950_code_objects(lib: bytes):
    """The gfx950 code objects of every offload bundle in .hip_fatbin (one
    bundle per linked source file)."""

    off, size, _ = elf_sections(lib)[".hip_fatbin"]
    fat = lib[off : off + size]
    pos = fat.find(BUNDLE_MAGIC)
    while pos >= 0:
        (entries,) = struct.unpack_from("<Q", fat, pos + len(BUNDLE_MAGIC))
        p = pos + len(BUNDLE_MAGIC) + 8
        for _ in range(entries):
            e_off, e_size, t_size = struct.unpack_from("<QQQ", fat, p)
            triple = fat[p + 24 : p + 24 + t_size].decode()
            p += 24 + t_size
            if triple.endswith("gfx950") and e_size:
                yield fat[pos + e_off : pos + e_off + e_size]
        pos = fat.find(BUNDLE_MAGIC, pos + len(BUNDLE_MAGIC))


def kernel_metadata(code_object: bytes):
    """The amdhsa.kernels entries of a code object's AMDGPU metadata note."""

    for off, size, typ in elf_sections(code_object).values():
        if typ != SHT_NOTE:
            continue
        p = off
        while p < off + size:
            n_size, d_size, n_type = struct.unpack_from("<III", code_object, p)
            name = code_object[p + 12 : p + 12 + n_size].rstrip(b"\0")
            desc = p + 12 + ((n_size + 3) & ~3)
            if name == b"AMDGPU" and n_type == NT_AMDGPU_METADATA:
                yield from msgpack.unpackb(code_object[desc : desc + d_size], raw=False)["amdhsa.kernels"]
            p = desc + ((d_size + 3) & ~3)


@pytest.fixture(scope="module")
def kernels() -> dict[str, dict]:
    if not LIB_PATH.is_file():
        pytest.skip("library not built")
    lib = LIB_PATH.read_bytes()
    found = {}
    for co in gfx950_code_objects(lib):
        for k in kernel_metadata(co):
            found[k[".name"]] = k
    return found


def test_every_source_contributes_kernels(kernels):
    names = " ".join(kernels)
    for part in ("attn_fwd_kernel", "attn_merge_kernel", "attn_vt_kernel", "qknorm_rope_kernel", "pack_qkv_kernel",
                 "modulate_kernel", "attn_merge_parts_kernel", "proj_gemm_kernel", "clock_sample_kernel"):
        assert part in names, part


def test_no_kernel_uses_scratch(kernels):
    spilled = {
        name: (k[".private_segment_fixed_size"], k.get(".vgpr_spill_count", 0))
        for name, k in kernels.items()
        if k[".private_segment_fixed_size"] != 0 or k.get(".vgpr_spill_count", 0) != 0
    }
    assert spilled == {}


def test_attention_forms_fit_one_workgroup_per_cu(kernels):
    forms = {name: k for name, k in kernels.items() if "attn_fwd_kernel" in name or "attn_fwd_persist_kernel" in name}
    # narrow / wide x token-major / d-major V, and the persistent launch
    assert len(forms) == 5
    for name, k in forms.items():
        assert k[".vgpr_count"] + k.get(".agpr_count", 0) <= 256, (name, k[".vgpr_count"], k.get(".agpr_count"))
        assert k[".group_segment_fixed_size"] <= 160 * 1024, name
        assert k[".max_flat_workgroup_size"] == 512, name
