"""The drop-in patch (gemma4.c_amd/host/gemma4c.patch) against the reference's
gemma4.c: it only adds lines, it applies to the reference's source, and the
patched program compiles with the reference's flags and links against
libg4.so (with -DG4_MI355X) or stays the CPU program (without).  CPU only: the
GPU run of the patched program is tests/test_gpu_integration.py.
"""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PATCH = os.path.join(ROOT, "gemma4.c_amd", "host", "gemma4c.patch")
REFERENCE = os.environ.get("G4_REFERENCE_DIR", "/root/reference")
LIBG4 = os.path.join(ROOT, "gemma4.c_amd", "libg4.so")
# the reference's Makefile:2 flags, -march=native replaced as in oracle/Makefile
REF_FLAGS = ["-std=c11", "-O3", "-Wall", "-Wextra", "-march=x86-64-v4", "-mavx512vnni", "-fopenmp"]

needs_reference = pytest.mark.skipif(not os.path.exists(os.path.join(REFERENCE, "gemma4.c")),
                                     reason="the reference checkout is not here")


def test_patch_only_adds_lines():
    """No line of the reference is removed or rewritten: the CPU forward() and
    logits() stay under #ifndef G4_MI355X, so the patch carries no reference
    text besides its hunk positions."""
    with open(PATCH) as f:
        lines = f.read().splitlines()
    assert lines[0] == "--- a/gemma4.c" and lines[1] == "+++ b/gemma4.c"
    body = lines[2:]
    assert body and all(line.startswith(("@@", "+")) for line in body)
    added = [line[1:] for line in body if line.startswith("+")]
    text = "\n".join(added)
    for needed in ("g4_init(", "g4_forward(", "g4_logits(", "g4_shutdown()", "#ifdef G4_MI355X"):
        assert needed in text, needed


def _patched_copy(tmp_path) -> str:
    shutil.copy(os.path.join(REFERENCE, "gemma4.c"), tmp_path / "gemma4.c")
    subprocess.run(["patch", "-s", "-p1", "-i", PATCH], cwd=tmp_path, check=True)
    return str(tmp_path / "gemma4.c")


@needs_reference
def test_patched_reference_links_against_libg4(tmp_path):
    if not os.path.exists(LIBG4):
        pytest.skip("libg4.so is not built")
    src = _patched_copy(tmp_path)
    exe = str(tmp_path / "run")
    out = subprocess.run(["gcc", *REF_FLAGS, "-DG4_MI355X", "-Werror", f"-I{ROOT}/include", src, "-o", exe,
                          f"-L{ROOT}/gemma4.c_amd", "-lg4", "-Wl,-rpath-link,/opt/rocm/lib", "-lm"],
                         capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
    symbols = subprocess.run(["nm", "-D", exe], capture_output=True, text=True, check=True).stdout
    undefined = {line.split()[-1] for line in symbols.splitlines() if " U " in line}
    assert {"g4_init", "g4_forward", "g4_logits", "g4_shutdown", "g4_last_error"} <= undefined


@needs_reference
def test_patched_reference_without_the_flag_is_the_cpu_program(tmp_path):
    src = _patched_copy(tmp_path)
    exe = str(tmp_path / "run_cpu")
    out = subprocess.run(["gcc", *REF_FLAGS, "-Werror", src, "-o", exe, "-lm"], capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
    symbols = subprocess.run(["nm", exe], capture_output=True, text=True, check=True).stdout
    assert "g4_" not in symbols
    assert " T forward" in symbols and " T logits" in symbols
