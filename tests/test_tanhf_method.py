"""The soft cap's tanhf (gemma4.c:518-519 calls the host libm's tanhf) is
pinned against the host libm itself, on every float below 22 in magnitude
(above, tanhf is +-1); the device restatement (tanhf_libm in g4_kernels.hip)
carries the same constants, and the GPU model tests compare its logits with
the oracle's bit for bit."""

from __future__ import annotations

import os
import re
import subprocess

import pytest

from helpers import ROOT

SRC = os.path.join(ROOT, "tests", "csrc", "tanhf_method_check.c")
DEVICE = os.path.join(ROOT, "gemma4.c_amd", "csrc", "g4_kernels.hip")


def _build(tmp_path_factory, name, *defines):
    exe = str(tmp_path_factory.mktemp(name) / name)
    subprocess.run(["gcc", "-std=gnu11", "-O2", "-ffp-contract=off", "-march=x86-64-v3", "-fopenmp", *defines,
                    SRC, "-o", exe, "-lm"], check=True)
    return exe


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    return _build(tmp_path_factory, "tanhf_check")


def test_device_constants_are_the_checked_ones(checker):
    """Q1..Q5, ln2_hi, ln2_lo and 1/ln2 in tanhf_libm are the checker's."""
    out = subprocess.run([checker, "constants"], check=True, capture_output=True, text=True).stdout.split()
    src = open(DEVICE).read()
    block = src[src.index("float expm1f_libm(float x)"):]
    block = block[:block.index("const float Q1")]
    names = ["kQ1", "kQ2", "kQ3", "kQ4", "kQ5", "kLn2Hi", "kLn2Lo", "kInvLn2"]
    device = [re.search(rf"{n} = (0x[0-9a-f]{{8}})u", block).group(1) for n in names]
    assert device == out


def test_method_equals_host_libm_exhaustively(checker):
    res = subprocess.run([checker], capture_output=True, text=True, timeout=600)
    bad, tested = map(int, res.stdout.split())
    assert tested == 2 * 0x41B00000
    assert bad == 0, f"{bad} of {tested} inputs differ from the host libm"


def test_a_one_ulp_constant_error_is_caught(tmp_path_factory):
    """Q1 one ulp off changes 246 results: the comparison sees such slips."""
    planted = _build(tmp_path_factory, "tanhf_planted", "-DPLANT_ERROR")
    res = subprocess.run([planted], capture_output=True, text=True, timeout=600)
    bad, _ = map(int, res.stdout.split())
    assert bad > 0
