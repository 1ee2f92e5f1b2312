"""Build recipe for the gemma4.c_amd libraries (in-tree, no build system).

    python gemma4.c_amd/build.py            # everything
    python gemma4.c_amd/build.py --no-ref   # skip the reference library

Products (all in-tree, git-ignored):
  gemma4.c_amd/libg4.so      HIP kernels + C ABI (hipcc, gfx950)
  gemma4.c_amd/libg4img.so   model-image loader / synthetic writer (gcc)
Test infrastructure built alongside:
  oracle/liboracle.so        CPU restatement (make -C oracle)
  oracle/_ref/libgemma4ref.so  the reference's own gemma4.c, when its
                             checkout is present (make -C oracle ref)
  oracle/_ref/run_g4         the reference's program with
                             gemma4.c_amd/host/gemma4c.patch, linked to
                             libg4.so (make -C oracle run_g4)
"""

from __future__ import annotations

import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, "include")
ORACLE = os.path.join(ROOT, "oracle")
REFERENCE = os.environ.get("G4_REFERENCE_DIR", "/root/reference")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -ffp-contract=off: the reference is built -std=c11 (no contraction), so the
# elementwise kernels round every multiply and add exactly as it does.
# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 anywhere in this library.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-munsafe-fp-atomics",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: the int8 fold reads them with no accvgpr moves
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-function",
    f"-I{INCLUDE}",
]
C_FLAGS = ["-std=c11", "-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fno-math-errno",
           "-fopenmp", "-fPIC", "-Wall", "-Wextra", f"-I{INCLUDE}"]


def run(cmd: list[str], cwd: str | None = None) -> None:
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, cwd=cwd, check=True)


def build_hip() -> str:
    sources = sorted(glob.glob(os.path.join(PKG, "csrc", "*.hip")))
    out = os.path.join(PKG, "libg4.so")
    tmp = out + ".tmp"
    run([HIPCC, *HIP_FLAGS, *sources, "-o", tmp])
    os.replace(tmp, out)
    return out


def build_img() -> str:
    out = os.path.join(PKG, "libg4img.so")
    run(["gcc", *C_FLAGS, "-shared", os.path.join(PKG, "host", "g4img.c"), "-o", out, "-lm"])
    return out


def build_oracle(with_ref: bool = True) -> None:
    run(["make", "-s", "-C", ORACLE, "all"])
    if with_ref and os.path.exists(os.path.join(REFERENCE, "gemma4.c")):
        run(["make", "-s", "-C", ORACLE, "ref", f"REF={REFERENCE}"])
        # the reference's program patched onto libg4.so (the drop-in check)
        run(["make", "-s", "-C", ORACLE, "run_g4", f"REF={REFERENCE}"])


def build_test_bins() -> None:
    """Test programs that run library code the C ABI does not reach (the
    exact-sum engine in every block shape): built with the library's device
    flags, linked to libg4.so, into tests/_bin/."""
    out_dir = os.path.join(ROOT, "tests", "_bin")
    os.makedirs(out_dir, exist_ok=True)
    flags = [f for f in HIP_FLAGS if f not in ("-shared", "-fPIC")]
    out = os.path.join(out_dir, "esum_fuzz")
    run([HIPCC, *flags, f"-I{os.path.join(PKG, 'csrc')}", os.path.join(ROOT, "tests", "esum_fuzz.hip"),
         "-o", out + ".tmp", f"-L{PKG}", "-lg4", "-Wl,-rpath,$ORIGIN/../../gemma4.c_amd"])
    os.replace(out + ".tmp", out)


def build_all(with_ref: bool = True) -> None:
    build_img()
    build_hip()
    build_test_bins()
    build_oracle(with_ref)


if __name__ == "__main__":
    build_all(with_ref="--no-ref" not in sys.argv)
