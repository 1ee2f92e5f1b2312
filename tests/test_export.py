"""The checkpoint writer (gemma4.c_amd/export.py, exporter.py's job): a
fabricated Gemma-4-E2B-shaped checkpoint whose BF16 weights are the synthetic
generator's seeded values exports to the synthetic image byte for byte outside
the computed tables (the generator with G4IMG_BF16_VALUES quantizes the same
bf16-rounded values).  Its tokenizer block, its quantize-and-pack step and its
RoPE/GELU tables are the reference exporter's own output (golden vectors in
tests/golden/ written by exporter.py's compile_tokenizer, quantize +
write_tensor, rope_tables and gelu_table).  Plus the dtypes of the packing step
and the writer's refusals.
"""

from __future__ import annotations

import ctypes
import hashlib
import importlib
import json
import os
import shutil
import struct
import tempfile

import numpy as np
import pytest

from conftest import MODEL_SEED
from helpers import GOLDEN, fabricated_config, fabricated_tokenizer


@pytest.fixture(scope="module")
def export(pkg):
    return importlib.import_module("gemma4_c_amd.export")


def _scratch_dir(need_bytes: int) -> str:
    """/dev/shm when it has room (memory speed), else the temp directory."""
    shm = "/dev/shm"
    if os.path.isdir(shm) and shutil.disk_usage(shm).free > need_bytes * 1.2:
        return tempfile.mkdtemp(prefix="g4export-", dir=shm)
    return tempfile.mkdtemp(prefix="g4export-")


def write_checkpoint(pkg, export, directory: str, seed: int, flags: int, dtype: str = "BF16") -> None:
    """config.json, tokenizer.json and model.safetensors holding the synthetic
    generator's values (rounded to bfloat16 with G4IMG_BF16_VALUES) under the
    checkpoint's tensor names."""
    img = pkg.img()
    with open(os.path.join(directory, "config.json"), "w") as f:
        json.dump(fabricated_config(), f)
    with open(os.path.join(directory, "tokenizer.json"), "w") as f:
        json.dump(fabricated_tokenizer(), f)
    items = (pkg.ImageItem * 700)()
    count = img.g4img_layout(0, items, 700)
    width = 2 if dtype == "BF16" else 4
    entries, offset = [], 0
    for i in range(count):
        it = items[i]
        name = export.record_tensor(it.record)
        if name is None:
            continue
        shape = (it.rows, it.cols) if it.kind == pkg.ITEM_QUANT else (it.rows,)
        n = int(np.prod(shape))
        entries.append((name, shape, i, offset, n))
        offset += n * width
    header = {"__metadata__": {"format": "pt"}}
    header.update({name: {"dtype": dtype, "shape": list(shape), "data_offsets": [o, o + n * width]}
                   for name, shape, _, o, n in entries})
    raw = json.dumps(header).encode()
    raw += b" " * (-len(raw) % 8)
    path = os.path.join(directory, "model.safetensors")
    out = np.memmap(path, dtype=np.uint8, mode="w+", shape=(8 + len(raw) + offset,))
    out[:8] = np.frombuffer(struct.pack("<Q", len(raw)), np.uint8)
    out[8:8 + len(raw)] = np.frombuffer(raw, np.uint8)
    data = out.ctypes.data + 8 + len(raw)
    code = pkg.DTYPE_BF16 if dtype == "BF16" else pkg.DTYPE_F32
    for name, shape, i, o, n in entries:  # straight into the mapped file
        assert img.g4img_draw(seed, flags, ctypes.byref(items[i]), data + o, code, 0) == 0, name
    out.flush()
    del out


def test_tokenizer_block_is_the_references(export):
    gold = json.load(open(os.path.join(GOLDEN, "export_tokenizer.json")))
    block = export.compile_tokenizer(fabricated_tokenizer())
    assert len(block) == gold["size"]
    assert struct.unpack_from("<3i", block, 0) == (gold["merges"], gold["encode"], gold["specials"])
    assert hashlib.sha256(block).hexdigest() == gold["sha256"]


def test_pack_matrix_is_the_exporters(pkg):
    """g4img_pack_matrix (the quantize-and-pack step of both writers) against
    exporter.py's quantize + write_tensor on a 48 x 192 matrix with
    bf16-rounded values, a zero group, a group under the fp16 scale floor, a
    lone value, exact halves of the scale and a wide dynamic range: int8
    bytes and fp16 scale bytes identical."""
    with np.load(os.path.join(GOLDEN, "export_pack.npz"), allow_pickle=False) as z:
        x, want_q, want_s = z["input"], z["packed"], z["scales"]
    rows, cols = x.shape
    q = np.zeros(rows * cols, np.int8)
    s = np.zeros(rows * cols // 64, np.uint16)
    assert pkg.img().g4img_pack_matrix(np.ascontiguousarray(x).ctypes.data, pkg.DTYPE_F32, rows, cols,
                                       q.ctypes.data, s.ctypes.data, 2) == 0
    assert np.array_equal(s, want_s), np.flatnonzero(s != want_s)[:8]
    assert np.array_equal(q, want_q), np.flatnonzero(q != want_q)[:8]


def test_pack_golden_catches_the_unrounded_scale():
    """The fixture tells the exporter's rule (divide by the fp16-rounded scale)
    from a plausible slip (divide by the fp32 scale before its rounding)."""
    with np.load(os.path.join(GOLDEN, "export_pack.npz"), allow_pickle=False) as z:
        x, want_q = z["input"], z["packed"]
    groups = x.reshape(-1, 64)
    scale = np.maximum(np.abs(groups).max(axis=1) / np.float32(127.0), np.float32(6.104e-05))
    slip = np.rint(groups / scale[:, None]).clip(-127, 127).astype(np.int8)
    blocks, ng = x.shape[0] // 16, x.shape[1] // 64
    packed = slip.reshape(blocks, 16, ng, 16, 4).transpose(0, 2, 3, 1, 4).reshape(-1)
    assert not np.array_equal(packed, want_q)


def test_tables_are_the_exporters(export):
    """export.py's GELU and RoPE tables against the SHA-256 of exporter.py's
    gelu_table() and rope_tables() for the E2B configuration (the same numpy
    float32 functions, so the same bits)."""
    gold = json.load(open(os.path.join(GOLDEN, "export_tables.json")))
    digest = lambda a: hashlib.sha256(np.ascontiguousarray(a, dtype=np.float32).tobytes()).hexdigest()
    note = f"golden written with numpy {gold['numpy']}, this is {np.__version__}"
    assert digest(export.gelu_values()) == gold["gelu"], note
    t = fabricated_config()["text_config"]
    rope = t["rope_parameters"]
    tables = {"sliding": export.rope_values(t["head_dim"], 1.0, rope["sliding_attention"]["rope_theta"], 131072),
              "global": export.rope_values(t["global_head_dim"], rope["full_attention"]["partial_rotary_factor"],
                                           rope["full_attention"]["rope_theta"], 131072)}
    for kind, (cos, sin) in tables.items():
        assert list(cos.shape) == gold[f"{kind}_cos_shape"]
        assert digest(cos) == gold[f"{kind}_cos"], (kind, note)
        assert digest(sin) == gold[f"{kind}_sin"], (kind, note)


def test_checkpoint_exports_to_the_synthetic_image(pkg, export):
    flags = pkg.BF16_VALUES
    size = pkg.img().g4img_size(flags)
    directory = _scratch_dir(size * 3)
    try:
        write_checkpoint(pkg, export, directory, MODEL_SEED, flags)
        out_path = os.path.join(directory, "e2b.bin")
        export.export(directory, out_path)
        out = np.memmap(out_path, dtype=np.uint8, mode="r")
        assert out.size == size
        synthetic = pkg.Image.synthetic(seed=MODEL_SEED, flags=flags)
        ref = np.frombuffer(synthetic.buf, dtype=np.uint8, count=size)
        t0, t1 = 4, 4 + pkg.TOKENIZER_SPAN
        assert bytes(out[:t0]) == bytes(ref[:t0]) == b"MOG\0"
        # the computed tables: the exporter's numpy values (pinned by
        # test_tables_are_the_exporters) in the file.  The synthetic image's
        # come from the C library (powf, cosf, sinf, tanhf): some RoPE
        # frequencies differ from numpy's by an ulp, which a position of up to
        # 131071 turns into angles up to ~2 ulp of 1 apart (|d| <= 2^-5 on
        # cos/sin, measured 0.0156); the GELU entries within a few ulp
        items = (pkg.ImageItem * 700)()
        count = pkg.img().g4img_layout(flags, items, 700)
        tables = []
        for i in range(count):
            it = items[i]
            if it.kind in (pkg.ITEM_ROPE_COS, pkg.ITEM_ROPE_SIN, pkg.ITEM_GELU):
                n = it.rows * it.cols
                want = export.table_values(it, fabricated_config()["text_config"]).reshape(-1)
                got = np.asarray(out[it.data:it.data + 4 * n]).view(np.float32)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), i
                syn = np.asarray(ref[it.data:it.data + 4 * n]).view(np.float32)
                bound = 2.0 ** -5 if it.kind != pkg.ITEM_GELU else 4 * np.spacing(np.abs(want).max())
                assert np.abs(syn - want).max() <= bound, (i, float(np.abs(syn - want).max()))
                tables.append((it.data, it.data + 4 * n))
        # records and every other tensor (4.77 GB): the same bytes, in 512 MiB pieces
        step, at = 1 << 29, t1
        for begin, end in sorted(tables) + [(size, size)]:
            for piece in range(at, begin, step):
                stop = min(piece + step, begin)
                assert np.array_equal(out[piece:stop], ref[piece:stop]), piece
            at = max(at, end)
        gold = json.load(open(os.path.join(GOLDEN, "export_tokenizer.json")))
        assert hashlib.sha256(out[t0:t1].tobytes()).hexdigest() == gold["sha256"]
        del out, ref, synthetic
    finally:
        shutil.rmtree(directory, ignore_errors=True)


@pytest.mark.parametrize("dtype", ["BF16", "F16"])
def test_pack_matrix_reads_each_dtype_as_its_fp32_value(pkg, dtype):
    """A 16-bit source packs exactly as the fp32 matrix of its values."""
    img = pkg.img()
    gen = np.random.default_rng(7)
    rows, cols = 32, 128
    x = (gen.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    if dtype == "BF16":
        src = (x.view(np.uint32) >> 16).astype(np.uint16)
        wide = (src.astype(np.uint32) << 16).view(np.float32)
        code = pkg.DTYPE_BF16
    else:
        src = x.astype(np.float16).view(np.uint16)
        wide = src.view(np.float16).astype(np.float32)
        code = pkg.DTYPE_F16
    outs = []
    for data, c in ((src, code), (np.ascontiguousarray(wide), pkg.DTYPE_F32)):
        q = np.zeros(rows * cols, np.int8)
        s = np.zeros(rows * cols // 64, np.uint16)
        assert img.g4img_pack_matrix(data.ctypes.data, c, rows, cols, q.ctypes.data, s.ctypes.data, 2) == 0
        outs.append((q, s))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])


def test_pack_matrix_refuses_nan_and_bad_shapes(pkg):
    img = pkg.img()
    x = np.zeros((16, 64), np.float32)
    q = np.zeros(16 * 64, np.int8)
    s = np.zeros(16, np.uint16)
    x[3, 5] = np.nan
    assert img.g4img_pack_matrix(x.ctypes.data, pkg.DTYPE_F32, 16, 64, q.ctypes.data, s.ctypes.data, 1) != 0
    assert img.g4img_pack_matrix(x.ctypes.data, pkg.DTYPE_F32, 15, 64, q.ctypes.data, s.ctypes.data, 1) != 0


def test_export_refuses_other_checkpoints(pkg, export, tmp_path):
    config = fabricated_config()
    config["text_config"]["num_hidden_layers"] = 26
    with pytest.raises(export.ExportError):
        export.check_config(config)
    # a tensor of the wrong shape is named in the error
    (tmp_path / "config.json").write_text(json.dumps(fabricated_config()))
    (tmp_path / "tokenizer.json").write_text(json.dumps(fabricated_tokenizer()))
    header = {"model.language_model.embed_tokens.weight": {"dtype": "BF16", "shape": [16, 64],
                                                           "data_offsets": [0, 2048]}}
    raw = json.dumps(header).encode()
    raw += b" " * (-len(raw) % 8)
    (tmp_path / "model.safetensors").write_bytes(struct.pack("<Q", len(raw)) + raw + bytes(2048))
    with pytest.raises(export.ExportError, match="embed_tokens.weight: shape"):
        export.export(str(tmp_path), str(tmp_path / "out.bin"))
    assert not (tmp_path / "out.bin").exists()
