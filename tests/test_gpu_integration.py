"""The reference's own program, patched onto libg4.so (oracle/_ref/run_g4, built
by `make -C oracle run_g4` where the reference checkout is), run on the GPU:
its unchanged loader mmaps a synthetic E2B .bin file, fixes up the offsets,
hands the records to g4_init, and its unchanged benchmark() and generate()
drive forward() and logits() through the library (gemma4.c:563-608, 627-645).
The unpatched program (oracle/_ref/run_ref, the reference's CPU build) is the
checker for the logit dump.
"""

from __future__ import annotations

import hashlib
import os
import re
import subprocess

import pytest

from conftest import MODEL_SEED

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RUN_G4 = os.path.join(ROOT, "oracle", "_ref", "run_g4")
RUN_REF = os.path.join(ROOT, "oracle", "_ref", "run_ref")
VOCAB = 262144


@pytest.fixture(scope="module")
def model_file(pkg, tmp_path_factory):
    if not os.path.exists(RUN_G4):
        pytest.skip("oracle/_ref/run_g4 is not built (needs the reference checkout at build time)")
    path = str(tmp_path_factory.mktemp("bin") / "synthetic-e2b.bin")
    img = pkg.img()
    assert img.g4img_write_file(path.encode(), MODEL_SEED, 0, 16) == 0, img.g4img_last_error()
    yield path
    os.remove(path)


@pytest.mark.gpu
def test_reference_cli_bench_runs_on_the_gpu(torch_gpu, model_file):
    print(f"running {RUN_G4} -m {model_file} --bench 600 8", flush=True)
    out = subprocess.run([RUN_G4, "-m", model_file, "--bench", "600", "8"], capture_output=True, text=True,
                         timeout=180)
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


def _dump_digest(cmd: list[str], log: str) -> tuple[int, str]:
    """Runs `cmd`, hashing its stdout as it streams (about 1 MiB a row)."""
    print("running " + " ".join(cmd[:3]) + f" --dump-logits <{len(cmd[-1])} bytes>  [{log}]", flush=True)
    digest, size = hashlib.sha256(), 0
    with subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE) as proc:
        while True:
            piece = proc.stdout.read(1 << 22)
            if not piece:
                break
            digest.update(piece)
            size += len(piece)
        err = proc.stderr.read().decode(errors="replace")
        rc = proc.wait(timeout=300)
    assert rc == 0, (log, rc, err)
    return size, digest.hexdigest()


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_reference_cli_dump_logits_matches_cpu_build(torch_gpu, model_file):
    """`./run --dump-logits "<prompt>"` (gemma4.c:575-595 -> prefill with dump,
    563-572): the patched program's stdout equals, byte for byte, the
    unpatched CPU program's on the same .bin and prompt.  The synthetic image's
    tokenizer block is zeroed, so both tokenize the ASCII prompt by byte
    fallback (gemma4.c:96-104): <bos>, a byte token per byte and three for
    each space's U+2581, 63 tokens here; one logits() row is written per
    position (the CPU program's lm_head takes ~0.2 s a row)."""
    if not os.path.exists(RUN_REF):
        pytest.skip("oracle/_ref/run_ref is not built (needs the reference checkout at build time)")
    prompt = "Why is the sky blue? Air scatters short waves."
    spaces = prompt.count(" ")
    tokens = 1 + len(prompt) - spaces + 3 * spaces  # <bos>, one byte token a byte, U+2581 as 3
    assert tokens == 63
    gpu = _dump_digest([RUN_G4, "-m", model_file, "--dump-logits", prompt], "patched, GPU")
    cpu = _dump_digest([RUN_REF, "-m", model_file, "--dump-logits", prompt], "reference, CPU")
    print(f"{tokens} rows: gpu {gpu[0]} bytes sha256 {gpu[1][:16]}, cpu {cpu[0]} bytes sha256 {cpu[1][:16]}",
          flush=True)
    assert gpu[0] == cpu[0] == tokens * VOCAB * 4
    assert gpu[1] == cpu[1]
