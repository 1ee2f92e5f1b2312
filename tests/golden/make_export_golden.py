"""Golden vectors for the checkpoint writer's tokenizer block: the reference's
own compile_tokenizer (exporter.py:197-259), imported from its checkout, run
on the fabricated tokenizer.json (tests/helpers.py: fabricated_tokenizer).
Nothing else pins that function's output (the reference ships no exported
image), so its result is kept here as data: the block's SHA-256 and size and
its three counts.

    python tests/golden/make_export_golden.py [REFERENCE_DIR]   # -> tests/golden/export_tokenizer.json
"""

from __future__ import annotations

import hashlib
import json
import os
import struct
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))  # tests/


def main() -> int:
    reference = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    from helpers import fabricated_tokenizer
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
    return 0


if __name__ == "__main__":
    sys.exit(main())
