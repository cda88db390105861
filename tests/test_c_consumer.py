"""The C ABI from C: tests/c/consumer.c is compiled as C11 against
include/h3attn.h and linked with the built library (no Python, no ctypes),
then calls the entry points that need no GPU: the version, argument
validation with its error codes and messages, and the workspace query.
Skipped where no C compiler or no built library is present."""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

from h3_flash_amd import _ext
from h3_flash_amd._build import LIB_PATH

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def consumer_output(tmp_path_factory):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    if not LIB_PATH.is_file():
        pytest.skip("library not built")
    exe = tmp_path_factory.mktemp("c_consumer") / "consumer"
    rocm_lib = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "lib"
    subprocess.run(
        [cc, "-std=c11", "-Wall", "-Werror", "-I", str(ROOT / "include"), str(ROOT / "tests" / "c" / "consumer.c"),
         "-L", str(LIB_PATH.parent), "-lh3attn", f"-Wl,-rpath,{LIB_PATH.parent}", f"-Wl,-rpath,{rocm_lib}",
         "-o", str(exe)],
        check=True,
    )
    run = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=120)
    return dict(line.split(" ", 1) for line in run.stdout.splitlines())


def test_version_matches_the_header(consumer_output):
    library, header = consumer_output["abi"].split()
    assert int(library) == int(header) == _ext.ABI_VERSION


def test_errors_reach_a_c_caller(consumer_output):
    assert int(consumer_output["null_args"]) == _ext.H3A_EINVAL
    assert consumer_output["null_args_message"] == "1"
    assert int(consumer_output["head_dim_64"]) == _ext.H3A_EUNSUPPORTED
    assert consumer_output["head_dim_64_message"] == "1"
    assert int(consumer_output["odd_rotary"]) == _ext.H3A_EINVAL
    assert consumer_output["odd_rotary_message"] == "1"


def test_workspace_query_from_c(consumer_output):
    assert consumer_output["workspace_ok"] == "1"
