"""The model image: exporter layout (exporter.py:29-70, 95-150, 262-273,
304-367) of the synthetic writer, and the validating loader."""

from __future__ import annotations

import ctypes
import mmap

import numpy as np
import pytest

from helpers import image_digest, load_golden

N_LAYERS = 35


def exporter_layout(ffn_6144: bool = False):
    """The exporter's cursor walk restated in Python (exporter.py:42-70,
    95-150, 333): a second, independent computation of every record's
    (data, scales, shape) and of the file size."""
    cursor = (4 + 33_429_932 + 55_008 + 63) & ~63

    def align(v):
        return (v + 63) & ~63

    def tensor(shape, quantized):
        nonlocal cursor
        count = int(np.prod(shape))
        rec = {"data": cursor, "scales": 0, "shape": shape}
        cursor = align(cursor + count * (1 if quantized else 4))
        if quantized:
            rec["scales"] = cursor
            cursor = align(cursor + count // 64 * 2)
        return rec

    slots = [tensor((262144, 1536), True), tensor((262144, 8960), True)]
    rope = {}
    for layer in range(N_LAYERS):
        full = layer % 5 == 4
        hd = 512 if full else 256
        kv = layer < 15
        ffn = 6144 if (layer < 15 or ffn_6144) else 12288
        row = [tensor((1536,), False), tensor((1,), False), tensor((1536,), False),
               tensor((1536,), False), tensor((1536,), False), tensor((1536,), False),
               tensor((256, 1536), True), tensor((1536, 256), True), tensor((hd,), False),
               tensor((hd,), False) if kv else None, tensor((8 * hd, 1536), True),
               tensor((hd, 1536), True) if kv else None, tensor((hd, 1536), True) if kv else None,
               tensor((1536, 8 * hd), True), tensor((ffn, 1536), True), tensor((ffn, 1536), True),
               tensor((1536, ffn), True)]
        key = 2 if full else 0
        pairs = 64 if full else 128
        for t in (0, 1):
            if key + t not in rope:
                rope[key + t] = tensor((131072, pairs), False)
            row.append(rope[key + t])
        slots += row
    gelu = tensor((4096,), False)
    gelu["shape"] = (4096, -8, 8)
    slots += [tensor((1536,), False), tensor((8960, 1536), True), tensor((256,), False), gelu]
    return slots, cursor


def test_size_matches_exporter_walk(pkg):
    for flags, ffn in ((0, False), (pkg.FFN_6144, True)):
        _, size = exporter_layout(ffn)
        assert pkg.img().g4img_size(flags) == size
    assert exporter_layout()[1] == 5_008_891_264  # E2B image size


def test_records_match_exporter_walk(pkg, image):
    slots, _ = exporter_layout()
    assert len(slots) == 671
    raw = np.frombuffer(image.buf, dtype=np.uint8, count=33_429_936 + 671 * 32)
    if image.fixed_inplace:
        pytest.skip("record table rewritten in place by an earlier test")
    assert bytes(raw[:4]) == b"MOG\0"
    table = raw[33_429_936:].view(np.dtype([("d", "<u8"), ("s", "<u8"), ("shape", "<i4", 4)]))
    for i, slot in enumerate(slots):
        if slot is None:
            assert table[i]["d"] == 0 and table[i]["s"] == 0
            continue
        assert table[i]["d"] == slot["data"], i
        assert table[i]["s"] == slot["scales"], i
        shape = list(slot["shape"]) + [0] * (4 - len(slot["shape"]))
        assert list(table[i]["shape"]) == shape, i
        assert slot["data"] % 64 == 0 and slot["scales"] % 64 == 0


def test_shared_rope_and_null_kv(pkg, image):
    r = image.records
    for layer in range(N_LAYERS):
        base = 2 + layer * 19
        ref_layer = 4 if layer % 5 == 4 else 0
        assert r[base + 17].data == r[2 + ref_layer * 19 + 17].data
        assert r[base + 18].data == r[2 + ref_layer * 19 + 18].data
        for field in (9, 11, 12):  # k_norm, k_proj, v_proj
            assert bool(r[base + field].data) == (layer < 15)


def test_weight_quantizer_invariants(pkg, image):
    """exporter.py:267-273: fp16 scale >= the fp16 floor, |q| <= 127, and a
    group whose scale is above the floor reaches |q| = 127."""
    floor = np.float32(np.float16(np.float32(6.104e-05)))
    for index in (0, pkg.layer_record(3, "q_proj"), pkg.layer_record(20, "down_proj"), 668):
        data, scales = image.packed(index)
        n, k = image.records[index].shape[0], image.records[index].shape[1]
        rows = min(n, 64)
        w = pkg.unpack_weight(data[: rows * k], rows, k)
        s = scales[: rows * k // 64].astype(np.float32).reshape(rows // 16, k // 64, 16)
        s = s.transpose(0, 2, 1).reshape(rows, k // 64)
        assert (s >= floor).all()
        assert np.abs(w.astype(np.int32)).max() <= 127
        gmax = np.abs(w.astype(np.int32)).reshape(rows, k // 64, 64).max(axis=2)
        assert (gmax[s > floor] == 127).all()
        # N(0, 0.02) before quantization: dequantized std close to 0.02
        deq = w.reshape(rows, k // 64, 64).astype(np.float32) * s[:, :, None]
        assert 0.017 < float(deq.std()) < 0.023


def test_tables(pkg, image):
    gelu = image.array(pkg.GELU_TABLE)
    assert gelu.shape == (4096,)
    x = np.linspace(-8, 8, 4096)
    ref = 0.5 * x * (1 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))
    assert np.abs(gelu - ref).max() < 1e-5
    cos = image.array(pkg.layer_record(0, "rope_cos"))
    sin = image.array(pkg.layer_record(0, "rope_sin"))
    assert cos.shape == (131072, 128)
    pos = np.array([0, 1, 511, 4096])[:, None]
    freq = 1.0 / 10000.0 ** (2 * np.arange(128) / 256)
    assert np.abs(cos[pos[:, 0]] - np.cos(pos * freq)).max() < 2e-3  # fp32 angle rounding
    assert np.abs(sin[1] - np.sin(freq)).max() < 1e-6
    gcos = image.array(pkg.layer_record(4, "rope_cos"))
    assert gcos.shape == (131072, 64)
    gfreq = 1.0 / 1e6 ** (2 * np.arange(64) / 512)
    assert np.abs(gcos[3] - np.cos(3 * gfreq)).max() < 1e-6


def test_image_digest_is_pinned(image):
    """The writer produces the same bytes as when the golden vectors were made."""
    gold = load_golden("model.npz")
    assert bytes(image_digest(image)) == bytes(gold["image_digest"])


def test_generator_is_thread_independent(pkg):
    """Regenerate with one thread into a second buffer and compare a digest."""
    size = pkg.img().g4img_size(pkg.FFN_6144)
    a = mmap.mmap(-1, size)
    b = mmap.mmap(-1, size)
    pa = ctypes.addressof(ctypes.c_char.from_buffer(a))
    pb = ctypes.addressof(ctypes.c_char.from_buffer(b))
    assert pkg.img().g4img_generate(pa, size, 99, pkg.FFN_6144, 8) == 0
    assert pkg.img().g4img_generate(pb, size, 99, pkg.FFN_6144, 3) == 0
    va = np.frombuffer(a, dtype=np.uint64)
    vb = np.frombuffer(b, dtype=np.uint64)
    assert np.array_equal(va[::4099], vb[::4099])
    assert np.array_equal(va[-100000:], vb[-100000:])
    del va, vb
    a.close()
    b.close()


def _records(pkg, buf, size):
    out = pkg.Records()
    base = ctypes.addressof(ctypes.c_char.from_buffer(buf))
    return pkg.img().g4img_records(base, size, out), pkg.img().g4img_last_error().decode()


def test_loader_rejects_bad_images(pkg):
    size = 33_429_936 + 671 * 32 + 4096
    buf = mmap.mmap(-1, size)
    rc, msg = _records(pkg, buf, size)
    assert rc == -1 and "bad model file" in msg  # gemma4.c:680
    buf[:4] = b"MOG\0"
    rc, _ = _records(pkg, buf, size)
    assert rc == 0  # all-null record table is well formed
    # a record whose data runs past the end of the image
    rec = np.frombuffer(buf, dtype=np.uint8)[33_429_936:33_429_936 + 32]
    rec[:] = np.frombuffer(np.array([size - 100, 0], "<u8").tobytes() + np.array([1536, 0, 0, 0], "<i4").tobytes(), np.uint8)
    rc, msg = _records(pkg, buf, size)
    assert rc == -1 and "outside the image" in msg
    # an unpackable quantized shape
    rec[:] = np.frombuffer(np.array([40_000_000 // 64 * 64, 40_000_000 // 64 * 64 + 4096], "<u8").tobytes() + np.array([17, 64, 0, 0], "<i4").tobytes(), np.uint8)
    rc, msg = _records(pkg, buf, size)
    assert rc == -1 and "packable" in msg
    del rec
    # truncated below the record table
    rc, msg = _records(pkg, buf, 1000)
    assert rc == -1 and "smaller" in msg
    buf.close()
