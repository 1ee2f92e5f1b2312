"""The reference's own program, patched onto libg4.so (oracle/_ref/run_g4, built
by `make -C oracle run_g4` where the reference checkout is), run on the GPU:
its unchanged loader mmaps a synthetic E2B .bin file, fixes up the offsets,
hands the records to g4_init, and its unchanged benchmark() drives forward()
and logits() through the library (gemma4.c:627-645).
"""

from __future__ import annotations

import os
import re
import subprocess

import pytest

from conftest import MODEL_SEED

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RUN_G4 = os.path.join(ROOT, "oracle", "_ref", "run_g4")


@pytest.mark.gpu
def test_reference_cli_bench_runs_on_the_gpu(pkg, torch_gpu, tmp_path):
    if not os.path.exists(RUN_G4):
        pytest.skip("oracle/_ref/run_g4 is not built (needs the reference checkout at build time)")
    path = str(tmp_path / "synthetic-e2b.bin")
    img = pkg.img()
    assert img.g4img_write_file(path.encode(), MODEL_SEED, 0, 16) == 0, img.g4img_last_error()
    print(f"running {RUN_G4} -m {path} --bench 600 8", flush=True)
    out = subprocess.run([RUN_G4, "-m", path, "--bench", "600", "8"], capture_output=True, text=True,
                         timeout=180)
    os.remove(path)
    assert out.returncode == 0, out.stderr
    # benchmark()'s two lines: pp600 (two chunks through forward, one logits)
    # and tg8@d600 (eight one-token forward + logits steps)
    prefill = re.search(r"^pp600 ([0-9.]+) tok/s$", out.stdout, re.M)
    decode = re.search(r"^tg8@d600 ([0-9.]+) tok/s$", out.stdout, re.M)
    assert prefill and decode, out.stdout
    print(out.stdout.strip(), flush=True)
    # the CPU build reaches ~600 tok/s prefill on 16 cores; the GPU is far above
    assert float(prefill.group(1)) > 5000.0
    assert float(decode.group(1)) > 50.0
