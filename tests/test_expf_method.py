"""The device softmax's expf (gemma4.c:403-407 calls the host libm's expf)
is pinned against the host libm itself, on every float of its main path."""

from __future__ import annotations

import os
import re
import subprocess

import pytest

from helpers import ROOT

SRC = os.path.join(ROOT, "tests", "csrc", "expf_method_check.c")
DEVICE = os.path.join(ROOT, "gemma4.c_amd", "csrc", "g4_reference_order.hip")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("expf") / "expf_check")
    subprocess.run(["gcc", "-std=gnu11", "-O2", "-ffp-contract=off", "-march=x86-64-v3", "-fopenmp",
                    SRC, "-o", exe, "-lm"], check=True)
    return exe


def test_device_table_is_the_definition(checker):
    """The 32 constants in the device source equal 2^(i/32) rounded to double
    (minus i << 47), recomputed in exact integer arithmetic."""
    out = subprocess.run([checker, "table"], check=True, capture_output=True, text=True).stdout.split()
    src = open(DEVICE).read()
    block = src[src.index("kExp2Table[32]"):]
    block = block[:block.index("};")]
    device = re.findall(r"0x([0-9a-f]{16})ull", block)
    assert [f"0x{d}" for d in device] == out


def test_method_equals_host_libm_exhaustively(checker):
    res = subprocess.run([checker], capture_output=True, text=True, timeout=600)
    bad, tested = map(int, res.stdout.split())
    assert tested > 2_000_000_000
    assert bad == 0, f"{bad} of {tested} inputs differ from the host libm"
