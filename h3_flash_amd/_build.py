"""Compile the gfx950 HIP library ``_lib/libh3attn.so`` in-tree.

Run as ``python -m h3_flash_amd._build``. The library is the only native
artefact of the package; the Python side binds it through ctypes.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
CSRC_DIR = PACKAGE_DIR / "csrc"
LIB_DIR = PACKAGE_DIR / "_lib"
LIB_PATH = LIB_DIR / "libh3attn.so"
INCLUDE_DIR = REPO_DIR / "include"

SOURCES = ("capi.hip", "attn_fwd.hip", "qknorm_rope.hip", "relayout.hip", "fusions.hip", "attn_merge.hip", "proj_gemm.hip", "clock.hip")

HIPCC_FLAGS = (
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-fvisibility=hidden",
    # Packed fp32 VALU forms stay disabled: only scalar fp32 VALU is emitted.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
)


def hipcc() -> str:
    """Path of hipcc (ROCM_PATH/bin first, then PATH)."""
    root = os.environ.get("ROCM_PATH", "/opt/rocm")
    candidate = Path(root) / "bin" / "hipcc"
    if candidate.is_file():
        return str(candidate)
    found = shutil.which("hipcc")
    if found is None:
        raise RuntimeError("hipcc not found: set ROCM_PATH or put hipcc on PATH")
    return found


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed ({result.returncode}):\n{result.stdout}\n{result.stderr}")


def build_library(verbose: bool = False, extra_flags: tuple[str, ...] = ()) -> Path:
    """Compile every HIP source into ``_lib/libh3attn.so`` and return its path.

    The sources compile in parallel to objects in a temporary directory (no
    device code crosses translation units), then link into the library. The
    output is written to a temporary name and renamed, so a concurrent reader
    never sees a half-written library.
    """

    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    compiler = hipcc()
    flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory(prefix="h3a_build_") as objdir:
        objects = [str(Path(objdir) / (Path(name).stem + ".o")) for name in SOURCES]
        # A fixed compilation-unit id per source: by default it hashes the
        # invocation, whose object path is a fresh temporary directory, and
        # the library's bytes (its sha256, which the bench matches against
        # profiled counters) would change with every build.
        compiles = [
            [compiler, *flags, *extra_flags, f"-cuid=h3a_{Path(name).stem}", f"-I{INCLUDE_DIR}", "-c", str(CSRC_DIR / name),
             "-o", obj]
            for name, obj in zip(SOURCES, objects)
        ]
        workers = max(1, min(len(compiles), os.cpu_count() or 1, 8))
        with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
            for future in [pool.submit(_run, cmd, verbose) for cmd in compiles]:
                future.result()
        _run([compiler, *HIPCC_FLAGS, *extra_flags, *objects, "-o", str(tmp)], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build_library(verbose="-v" in sys.argv)
    print(path)
