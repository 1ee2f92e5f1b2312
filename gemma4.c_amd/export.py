"""Gemma 4 E2B checkpoint -> the .bin image gemma4.c loads (exporter.py's job).

    python gemma4.c_amd/export.py CHECKPOINT_DIR -o gemma4-E2B-int8.bin

CHECKPOINT_DIR is a Hugging Face snapshot: config.json, tokenizer.json and
model.safetensors (weights in BF16, F16 or F32).  The image has the exporter's
layout byte for byte (exporter.py:29-37, 95-150, 262-367): "MOG\\0", the
compiled tokenizer (exporter.py:197-259), 671 tensor records, then every
tensor 64-byte aligned in the exporter's cursor order; matrices quantized with
its rule (absmax / 127 as an fp16 scale floored at 6.104e-5, rint, clip to
+-127; exporter.py:267-273) and packed in 16-row x 64-column tiles
(exporter.py:304-316); the shared RoPE tables and the GELU table from its
formulas (exporter.py:73-92), evaluated with numpy's float32 functions in the
exporter's operation order, so they are the exporter's bits.

The layout and the quantize-and-pack step are libg4img.so's (the same code
writes the seeded synthetic image), so a checkpoint holding the synthetic
generator's values exports to the synthetic image exactly outside the tables
(tests/test_export.py); the synthetic image computes its tables with the C
library's powf/sinf/cosf/tanhf instead, which differ from numpy's in the last
bits of some entries.  This module reads the checkpoint without torch: the
safetensors header is JSON, the tensors are mapped from the file.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import struct
import sys

import numpy as np

if __package__ in (None, ""):  # run as a script: import the package by path
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import __graft_entry__

    _pkg = __graft_entry__.load_package()
else:
    _pkg = sys.modules[__package__]

N_LAYERS, N_KV_LAYERS, VOCAB = 35, 15, 262144
TOKEN_MAX, SPECIAL_MAX, ENCODE_MAX, MERGES_MAX = 94, 256, 32768, 514906
BYTE_TOKEN_BASE = 238

# gemma4.c's LayerWeights field order (gemma4.c:125-145) -> the checkpoint's
# tensor name under model.language_model.layers.{l}. (exporter.py:108-130);
# None: a table the image computes (RoPE)
LAYER_FIELDS = [
    "input_layernorm.weight", "layer_scalar", "pre_feedforward_layernorm.weight",
    "post_attention_layernorm.weight", "post_feedforward_layernorm.weight",
    "post_per_layer_input_norm.weight", "per_layer_input_gate.weight", "per_layer_projection.weight",
    "self_attn.q_norm.weight", "self_attn.k_norm.weight", "self_attn.q_proj.weight",
    "self_attn.k_proj.weight", "self_attn.v_proj.weight", "self_attn.o_proj.weight",
    "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight", None, None,
]
TOP = "model.language_model."
GLOBAL_RECORDS = {0: "embed_tokens.weight", 1: "embed_tokens_per_layer.weight", 667: "norm.weight",
                  668: "per_layer_model_projection.weight", 669: "per_layer_projection_norm.weight"}


def record_tensor(record: int) -> str | None:
    """The checkpoint tensor behind a record (None for the computed tables)."""
    if record in GLOBAL_RECORDS:
        return TOP + GLOBAL_RECORDS[record]
    if 2 <= record < 2 + N_LAYERS * 19:
        layer, field = divmod(record - 2, 19)
        name = LAYER_FIELDS[field]
        return None if name is None else f"{TOP}layers.{layer}.{name}"
    return None


class ExportError(ValueError):
    pass


# ---------------------------------------------------------------------------
# config.json: the checkpoint must be Gemma 4 E2B (exporter.py:153-175)

def check_config(model: dict) -> dict:
    if model.get("model_type") != "gemma4":
        raise ExportError("checkpoint is not Gemma 4")
    t = model["text_config"]
    shape = (t["hidden_size"], t["vocab_size"], t["num_hidden_layers"],
             t["num_hidden_layers"] - t["num_kv_shared_layers"], t["num_key_value_heads"], t["head_dim"],
             t["global_head_dim"], t["intermediate_size"], t["use_double_wide_mlp"])
    if shape != (1536, VOCAB, N_LAYERS, N_KV_LAYERS, 1, 256, 512, 6144, True):
        raise ExportError(f"expected Gemma 4 E2B, got {shape}")
    if (t["max_position_embeddings"], t["sliding_window"], t["hidden_size_per_layer_input"]) != (131072, 512, 256):
        raise ExportError("expected the E2B context, window and per-layer width")
    if (np.float32(t["rms_norm_eps"]) != np.float32(float.fromhex("0x1.0c6f7ap-20"))
            or np.float32(t["final_logit_softcapping"]) != np.float32(30.0)):
        raise ExportError("expected the E2B norm epsilon and soft cap")
    if t["layer_types"] != (["sliding_attention"] * 4 + ["full_attention"]) * 7:
        raise ExportError("expected four sliding layers then one global, seven times")
    # the RoPE tables the image computes are E2B's (exporter.py:78-92)
    rope = t["rope_parameters"]
    if (float(rope["sliding_attention"]["rope_theta"]) != 10000.0
            or float(rope["full_attention"]["rope_theta"]) != 1000000.0
            or float(rope["full_attention"]["partial_rotary_factor"]) != 0.25):
        raise ExportError("expected E2B's RoPE parameters")
    return t


# ---------------------------------------------------------------------------
# tokenizer.json -> the fixed 33,429,932-byte block gemma4.c reads
# (gemma4.c:36-113; exporter.py:197-259)

def _payload(token_id: int, token: str, specials: set[int]) -> bytes:
    """What gemma4.c prints for a token: nothing for a special one, the byte
    of a <0xHH> byte token, else the text with the word marker as a space."""
    if token_id in specials:
        return b""
    if (len(token) == 6 and token.startswith("<0x") and token.endswith(">")
            and all(ch in "0123456789abcdefABCDEF" for ch in token[3:5])):
        return bytes([int(token[3:5], 16)])
    out = token.replace("▁", " ").encode("utf-8")
    if b"\0" in out or len(out) >= TOKEN_MAX:
        raise ExportError(f"token {token_id} does not fit char[{TOKEN_MAX}]")
    return out


def compile_tokenizer(data: dict) -> bytes:
    vocab = dict(data["model"]["vocab"])
    added = data["added_tokens"]
    for entry in added:
        if vocab.get(entry["content"], entry["id"]) != entry["id"]:
            raise ExportError(f"token {entry['content']!r} has two ids")
        vocab[entry["content"]] = entry["id"]
    by_id: list[str | None] = [None] * VOCAB
    for token, token_id in vocab.items():
        if not 0 <= token_id < VOCAB or by_id[token_id] is not None:
            raise ExportError("token ids must be unique and in [0, 262144)")
        by_id[token_id] = token
    if any(t is None for t in by_id):
        raise ExportError("token ids must be dense")

    # merges: (left id, right id) -> result id, in rank order
    merges, merge_results, seen_pairs = [], set(), set()
    for rank, merge in enumerate(data["model"]["merges"]):
        left, right = merge if isinstance(merge, list) else merge.split(" ", 1)
        pair = (vocab[left], vocab[right])
        if pair in seen_pairs or left + right not in vocab:
            raise ExportError(f"invalid merge {merge!r}")
        seen_pairs.add(pair)
        merge_results.add(left + right)
        merges.append((struct.pack("<2i", *pair), vocab[left + right], rank))
    # specials, longest first (then by bytes): the tokenizer's greedy match order
    specials = sorted(((e["id"], e["content"]) for e in added if e["special"]),
                      key=lambda s: (-len(s[1].encode()), s[1].encode()))
    special_ids = {i for i, _ in specials}
    special_text = {t for _, t in specials}
    for b in range(256):
        token = f"<0x{b:02X}>"
        if vocab.get(token) != BYTE_TOKEN_BASE + b or token in special_text or token in merge_results:
            raise ExportError("byte tokens must be ids 238..493, neither special nor merge results")
    # direct lookups: short tokens that are neither special nor built by a merge
    encode = [(t.encode().ljust(8, b"\0"), i, 0) for i, t in enumerate(by_id)
              if t not in special_text and t not in merge_results and len(t.encode()) <= 4]
    if len(specials) > SPECIAL_MAX or len(encode) > ENCODE_MAX or len(merges) > MERGES_MAX:
        raise ExportError("tokenizer exceeds the image's fixed tables")

    block = bytearray(_pkg.TOKENIZER_SPAN)
    struct.pack_into("<3i", block, 0, len(merges), len(encode), len(specials))
    for token_id, token in enumerate(by_id):
        text = _payload(token_id, token, special_ids)
        at = 12 + token_id * TOKEN_MAX
        block[at:at + len(text)] = text
    special_at = 12 + VOCAB * TOKEN_MAX
    encode_at = special_at + SPECIAL_MAX * 100
    merge_at = encode_at + ENCODE_MAX * 16
    for n, (token_id, token) in enumerate(specials):
        text = token.encode()
        if b"\0" in text or len(text) >= TOKEN_MAX:
            raise ExportError(f"special token {token!r} does not fit char[{TOKEN_MAX}]")
        block[special_at + n * 100:special_at + n * 100 + len(text)] = text
        struct.pack_into("<i", block, special_at + n * 100 + 96, token_id)
    for at, table in ((encode_at, encode), (merge_at, merges)):
        for n, entry in enumerate(sorted(table)):
            struct.pack_into("<8sii", block, at + n * 16, *entry)
    return bytes(block)


# ---------------------------------------------------------------------------
# The computed tables (exporter.py:73-92), float32 throughout: numpy's
# float32 tanh/cos/sin/power give the exporter's bits, which the C library's
# functions do not always match.

GELU_POINTS, GELU_LOWER, GELU_UPPER = 4096, -8.0, 8.0


def gelu_values() -> np.ndarray:
    """The tanh-form GELU at 4096 evenly spaced points of [-8, 8]; the
    products are taken left to right, as the exporter writes them."""
    x = np.linspace(GELU_LOWER, GELU_UPPER, GELU_POINTS, dtype=np.float32)
    inner = x + np.float32(0.044715) * x * x * x
    return (np.float32(0.5) * x * (np.float32(1.0) + np.tanh(np.float32(0.7978845608) * inner))).astype(np.float32)


def rope_values(head_dim: int, rotary_fraction: float, theta: float, positions: int):
    """(cos, sin) [positions x pairs] of angle = pos * theta^(-2j / head_dim)
    over the first int(head_dim * rotary_fraction) / 2 pairs."""
    pairs = int(head_dim * rotary_fraction) // 2
    inverse = np.float32(1) / np.power(np.float32(theta),
                                       np.arange(pairs, dtype=np.float32) * np.float32(2) / np.float32(head_dim))
    angle = np.arange(positions, dtype=np.float32)[:, None] * inverse
    return np.cos(angle), np.sin(angle)


def table_values(it, text_config: dict) -> np.ndarray:
    """The float32 values of a RoPE or GELU table item."""
    if it.kind == _pkg.ITEM_GELU:
        return gelu_values()
    rope = text_config["rope_parameters"]
    if it.global_rope:
        full = rope["full_attention"]
        cos, sin = rope_values(text_config["global_head_dim"], float(full["partial_rotary_factor"]),
                               float(full["rope_theta"]), it.rows)
    else:
        cos, sin = rope_values(text_config["head_dim"], 1.0, float(rope["sliding_attention"]["rope_theta"]),
                               it.rows)
    return cos if it.kind == _pkg.ITEM_ROPE_COS else sin


# ---------------------------------------------------------------------------
# model.safetensors, mapped (no torch)

_DTYPES = {"F32": (_pkg.DTYPE_F32, np.float32), "BF16": (_pkg.DTYPE_BF16, np.uint16),
           "F16": (_pkg.DTYPE_F16, np.uint16)}


class SafeTensors:
    def __init__(self, path: str):
        with open(path, "rb") as f:
            (n,) = struct.unpack("<Q", f.read(8))
            self.header = json.loads(f.read(n))
        self.header.pop("__metadata__", None)
        self.base = 8 + n
        self.map = np.memmap(path, dtype=np.uint8, mode="r")

    def entry(self, name: str, shape: tuple[int, ...]):
        """(dtype code, view of the bytes) of a tensor of the expected shape."""
        if name not in self.header:
            raise ExportError(f"checkpoint has no tensor {name}")
        e = self.header[name]
        if e["dtype"] not in _DTYPES:
            raise ExportError(f"{name}: dtype {e['dtype']} is not BF16, F16 or F32")
        if tuple(e["shape"]) != shape:
            raise ExportError(f"{name}: shape {tuple(e['shape'])}, expected {shape}")
        begin, end = e["data_offsets"]
        code, np_type = _DTYPES[e["dtype"]]
        if end - begin != int(np.prod(shape)) * np.dtype(np_type).itemsize or self.base + end > self.map.size:
            raise ExportError(f"{name}: data offsets do not match its shape")
        return code, self.map[self.base + begin:self.base + end]

    def floats(self, name: str, shape: tuple[int, ...]) -> np.ndarray:
        code, raw = self.entry(name, shape)
        if code == _pkg.DTYPE_F32:
            return raw.view(np.float32).copy()
        bits = raw.view(np.uint16)
        if code == _pkg.DTYPE_BF16:
            return (bits.astype(np.uint32) << 16).view(np.float32)
        return bits.view(np.float16).astype(np.float32)


# ---------------------------------------------------------------------------

def export(checkpoint: str, out_path: str, threads: int = 0) -> None:
    img = _pkg.img()
    with open(os.path.join(checkpoint, "config.json"), encoding="utf-8") as f:
        text_config = check_config(json.load(f))
    with open(os.path.join(checkpoint, "tokenizer.json"), encoding="utf-8") as f:
        tokenizer = compile_tokenizer(json.load(f))
    weights = SafeTensors(os.path.join(checkpoint, "model.safetensors"))

    items = (_pkg.ImageItem * 700)()
    count = img.g4img_layout(0, items, 700)
    if count < 0:
        raise ExportError(img.g4img_last_error().decode())
    size = img.g4img_size(0)
    tmp = out_path + ".partial"
    out = np.memmap(tmp, dtype=np.uint8, mode="w+", shape=(size,))  # zero-filled
    base = out.ctypes.data

    def check(rc):
        if rc != 0:
            raise ExportError(img.g4img_last_error().decode())

    check(img.g4img_write_header(base, size, 0))
    out[4:4 + len(tokenizer)] = np.frombuffer(tokenizer, np.uint8)
    for i in range(count):
        it = items[i]
        if it.kind in (_pkg.ITEM_ROPE_COS, _pkg.ITEM_ROPE_SIN, _pkg.ITEM_GELU):
            values = table_values(it, text_config)
            if values.size != it.rows * it.cols:
                raise ExportError(f"table item {i}: {values.size} values for {it.rows} x {it.cols}")
            out[it.data:it.data + 4 * values.size] = values.reshape(-1).view(np.uint8)
            continue
        name = record_tensor(it.record)
        if it.kind == _pkg.ITEM_QUANT:
            code, raw = weights.entry(name, (it.rows, it.cols))
            check(img.g4img_pack_matrix(raw.ctypes.data, code, it.rows, it.cols, base + it.data,
                                        base + it.scales, threads))
        else:  # norm weights (and layer_scalar): fp32 as they are
            values = weights.floats(name, (it.rows,))
            out[it.data:it.data + 4 * it.rows] = values.view(np.uint8)
    out.flush()
    del out
    os.replace(tmp, out_path)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("checkpoint")
    ap.add_argument("-o", "--out", required=True)
    ap.add_argument("--threads", type=int, default=0)
    args = ap.parse_args()
    export(args.checkpoint, args.out, args.threads)
    print(f"wrote {args.out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
