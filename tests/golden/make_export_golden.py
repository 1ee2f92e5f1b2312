"""Golden vectors for the checkpoint writer, made by the reference's own
exporter.py, imported from its checkout.  Nothing else pins these functions'
output (the reference ships no exported image), so their results are kept here
as data:

  export_tokenizer.json  compile_tokenizer (exporter.py:197-259) on the
                         fabricated tokenizer.json (tests/helpers.py): the
                         block's SHA-256 and size and its three counts;
  export_pack.npz        quantize + write_tensor's tile packing
                         (exporter.py:267-273, 282-316) of a seeded 48 x 192
                         fp32 matrix: the input, the packed int8 bytes and the
                         fp16 scale bytes;
  export_tables.json     SHA-256 of gelu_table() and of the four rope_tables()
                         arrays (exporter.py:73-92) for the E2B configuration.

    python tests/golden/make_export_golden.py [REFERENCE_DIR]
"""

from __future__ import annotations

import hashlib
import io
import json
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))  # tests/


def pack_input() -> np.ndarray:
    """48 x 192 (3 row blocks x 3 groups): N(0, 0.02) values rounded to
    bfloat16 (as a BF16 checkpoint holds them), plus groups that reach the
    quantizer's corners -- all zeros, all below the fp16 scale floor
    (absmax / 127 < 6.104e-5), a single nonzero value, exact halves of the
    scale, and a wide dynamic range."""
    gen = np.random.default_rng(20261202)
    x = (gen.standard_normal((48, 192)) * 0.02).astype(np.float32)
    x = ((x.view(np.uint32) + 0x7FFF + ((x.view(np.uint32) >> 16) & 1)) & 0xFFFF0000).view(np.float32)
    x[0, 0:64] = 0.0
    x[1, 64:128] = (gen.standard_normal(64) * 1e-6).astype(np.float32)
    x[2, 128:192] = 0.0
    x[2, 140] = -0.375
    s = np.float32(np.float16(np.float32(0.5) / np.float32(127.0)))
    x[3, 0:64] = s * (np.arange(64, dtype=np.float32) - np.float32(31.5))
    x[3, 0] = np.float32(0.5)
    x[4, 64:128] = (gen.standard_normal(64) * np.exp(gen.uniform(-12, 2, 64))).astype(np.float32)
    return x


def main() -> int:
    reference = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    from helpers import fabricated_config, fabricated_tokenizer
    sys.path.insert(0, reference)
    import exporter  # the reference's exporter.py

    block = exporter.compile_tokenizer(fabricated_tokenizer())
    merges, encode, specials = struct.unpack_from("<3i", block, 0)
    out = {"sha256": hashlib.sha256(block).hexdigest(), "size": len(block),
           "merges": merges, "encode": encode, "specials": specials}
    with open(os.path.join(HERE, "export_tokenizer.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(out)

    # write_tensor's quantize-and-pack branch, into a buffer: the data at 0,
    # the scales after it (64-byte aligned, as the cursor walk places them)
    x = pack_input()
    rows, cols = x.shape
    data_bytes = rows * cols
    scales_at = exporter.align64(data_bytes)
    sink = io.BytesIO(bytes(scales_at + rows * cols // 64 * 2))

    class Quiet:
        def update(self, n):
            pass

    exporter.write_tensor(sink, None, {"synthetic": x, "shape": (rows, cols), "data": 0, "scales": scales_at,
                                       "path": "golden"}, Quiet())
    raw = sink.getvalue()
    np.savez_compressed(os.path.join(HERE, "export_pack.npz"), input=x,
                        packed=np.frombuffer(raw[:data_bytes], np.int8),
                        scales=np.frombuffer(raw[scales_at:scales_at + rows * cols // 64 * 2], np.uint16))

    tables = {"gelu": hashlib.sha256(exporter.gelu_table().tobytes()).hexdigest()}
    names = ("sliding_cos", "sliding_sin", "global_cos", "global_sin")
    for name, array in zip(names, exporter.rope_tables(fabricated_config()["text_config"])):
        tables[name] = hashlib.sha256(np.ascontiguousarray(array, dtype=np.float32).tobytes()).hexdigest()
        tables[name + "_shape"] = list(array.shape)
    tables["numpy"] = np.__version__
    with open(os.path.join(HERE, "export_tables.json"), "w") as f:
        json.dump(tables, f, indent=1)
        f.write("\n")
    print(tables)
    return 0


if __name__ == "__main__":
    sys.exit(main())
