"""Test plumbing: packed weights as host (numpy) or device (torch) records."""

from __future__ import annotations

import ctypes
import hashlib
import os
import re

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")


def gelu_table_exporter() -> np.ndarray:
    """exporter.py:73-75 in float32 (numpy's tanh)."""
    x = np.linspace(-8.0, 8.0, 4096, dtype=np.float32)
    return (0.5 * x * (1.0 + np.tanh(0.7978845608 * (x + 0.044715 * x * x * x)))).astype(np.float32)


def aligned(a: np.ndarray, alignment: int = 64) -> np.ndarray:
    """Copy of `a` whose data starts on an `alignment`-byte boundary (the
    reference's VNNI kernel uses aligned 64-byte loads, gemma4.c:207)."""
    a = np.ascontiguousarray(a)
    raw = np.empty(a.nbytes + alignment, dtype=np.uint8)
    off = (-raw.ctypes.data) % alignment
    out = raw[off:off + a.nbytes].view(a.dtype).reshape(a.shape)
    out[...] = a
    return out


class HostWeight:
    """A packed int8 matrix with fp16 scales in host memory plus its record."""

    def __init__(self, pkg, w: np.ndarray, s: np.ndarray):
        self.w, self.s = w, s
        self.n, self.k = w.shape
        self.packed = aligned(pkg.pack_weight(w))
        self.scales = aligned(pkg.pack_scales(s.astype(np.float16)).view(np.uint16))
        self.record = pkg.Tensor()
        self.record.data = self.packed.ctypes.data
        self.record.scales = self.scales.ctypes.data
        self.record.shape[0], self.record.shape[1] = self.n, self.k


class HostF32:
    """An fp32 record (norm weights, tables) in host memory."""

    def __init__(self, pkg, a: np.ndarray, shape=None):
        self.a = np.ascontiguousarray(a, dtype=np.float32)
        self.record = pkg.Tensor()
        self.record.data = self.a.ctypes.data
        self.record.scales = None
        shp = shape if shape is not None else self.a.shape
        for i, v in enumerate(shp):
            self.record.shape[i] = v


class DeviceWeight:
    """The same packed matrix copied to the GPU (torch memory)."""

    def __init__(self, pkg, torch, host: HostWeight):
        self.data = torch.from_numpy(host.packed.copy()).cuda()
        self.scales = torch.from_numpy(host.scales.view(np.int16).copy()).cuda()
        self.record = pkg.Tensor()
        self.record.data = self.data.data_ptr()
        self.record.scales = self.scales.data_ptr()
        self.record.shape[0], self.record.shape[1] = host.n, host.k


def header_functions(path: str) -> list[str]:
    """Function names declared in a C header (for the export check)."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\**\s*(g4[a-z_0-9]*)\s*\(", text, flags=re.M)


def load_golden(name: str) -> dict[str, np.ndarray]:
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def stream_ptr(torch) -> int:
    return torch.cuda.current_stream().cuda_stream


def ptr(t) -> int:
    return t.data_ptr()


def as_tensor_record(pkg, data_ptr: int, scales_ptr: int, n: int, k: int):
    rec = pkg.Tensor()
    rec.data = data_ptr
    rec.scales = scales_ptr
    rec.shape[0], rec.shape[1] = n, k
    return rec


def c_float_p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def record_sizes(t, index: int) -> tuple[int, int]:
    """(data bytes, scales bytes) of a record (exporter.py:61-70)."""
    if not t.data:
        return 0, 0
    if t.scales:
        count = t.shape[0] * t.shape[1]
        return count, count // 32
    if index == 670:  # GELU table: shape (4096, lo, hi)
        return t.shape[0] * 4, 0
    return t.shape[0] * max(t.shape[1], 1) * 4, 0


def image_digest(image) -> np.ndarray:
    """SHA-256 over every record's shape, data/scales offsets and the first
    4 KiB (at most) of its data and of its scales: pins the synthetic writer's
    bytes across hosts without hashing 5 GB."""
    h = hashlib.sha256()
    for i in range(671):
        t = image.records[i]
        h.update(np.array(list(t.shape), dtype=np.int32).tobytes())
        for p, size in zip((t.data, t.scales), record_sizes(t, i)):
            if not p:
                continue
            h.update(np.int64(p - image.base).tobytes())
            h.update(ctypes.string_at(p, min(size, 4096)))
    return np.frombuffer(h.digest(), dtype=np.uint8)


def sample_cases(vocab: int = 4096):
    """Logits rows, temperatures and generator states for the sampler
    (gemma4.c:527-561): rows chosen to exercise the top-64 list's ordering
    (ties at and around the 64th place, +0 against -0), the soft-capped
    range, one dominant logit, a flat top, and a row whose 64 highest are
    all equal."""
    g = np.random.default_rng(42)
    rows = []
    rows.append((g.standard_normal(vocab) * 3.0).astype(np.float32))
    rows.append(g.integers(-20, 21, vocab).astype(np.float32))                      # many ties
    z = np.where(g.random(vocab) < 0.5, np.float32(0.0), np.float32(-0.0))
    z[g.choice(vocab, 40, replace=False)] = g.standard_normal(40).astype(np.float32)
    rows.append(z.astype(np.float32))                                               # +0 / -0
    rows.append((30.0 * np.tanh(g.standard_normal(vocab) * 10.0 / 30.0)).astype(np.float32))
    d = (g.standard_normal(vocab)).astype(np.float32)
    d[1234] = 40.0
    rows.append(d)                                                                  # dominant
    f = (g.standard_normal(vocab) - 10.0).astype(np.float32)
    f[g.choice(vocab, 100, replace=False)] = np.float32(5.0)
    rows.append(f)                                                                  # 100-way tie
    temps = [0.0, 0.3, 1.0, 2.5]
    states = [42, 0x9E3779B97F4A7C15]
    return rows, temps, states


# ---------------------------------------------------------------------------
# A fabricated Gemma 4 E2B checkpoint (for the checkpoint writer's tests and
# the golden tokenizer block)

def fabricated_config() -> dict:
    """config.json with the E2B text configuration the exporter accepts
    (exporter.py:153-175)."""
    return {
        "model_type": "gemma4",
        "text_config": {
            "hidden_size": 1536, "vocab_size": 262144, "num_hidden_layers": 35, "num_kv_shared_layers": 20,
            "num_key_value_heads": 1, "head_dim": 256, "global_head_dim": 512, "intermediate_size": 6144,
            "use_double_wide_mlp": True, "max_position_embeddings": 131072, "sliding_window": 512,
            "hidden_size_per_layer_input": 256, "rms_norm_eps": 1e-6, "final_logit_softcapping": 30.0,
            "layer_types": (["sliding_attention"] * 4 + ["full_attention"]) * 7,
            "rope_parameters": {"sliding_attention": {"rope_theta": 10000.0},
                                "full_attention": {"rope_theta": 1000000.0, "partial_rotary_factor": 0.25}},
        },
    }


def fabricated_tokenizer() -> dict:
    """tokenizer.json of 262144 ids that the exporter's rules accept: ids 0-5
    and 105/106 special (turn markers included), the byte tokens <0x00>..<0xFF>
    at 238-493, the 26 letters (direct lookups), their 676 two-letter
    concatenations built by merges, a few multi-byte and word-marker tokens,
    and filler words elsewhere."""
    specials = {0: "<pad>", 1: "<eos>", 2: "<bos>", 3: "<unk>", 4: "<mask>", 5: "[multimodal]",
                105: "<|turn>", 106: "<turn|>"}
    vocab = {}
    for b in range(256):
        vocab[f"<0x{b:02X}>"] = 238 + b
    letters = [chr(ord("a") + i) for i in range(26)]
    for i, ch in enumerate(letters):
        vocab[ch] = 494 + i
    merges = []
    n = 520
    for a in letters:
        for b in letters:
            vocab[a + b] = n
            merges.append(f"{a} {b}")
            n += 1
    extra = ["▁", "▁the", "é", "ß", "€", "日本", "▁▁", "\t", "x▁y"]
    for t in extra:
        vocab[t] = n
        n += 1
    used = set(vocab.values()) | set(specials)
    for i in range(262144):
        if i not in used:
            vocab[f"▁w{i}"] = i
    added = [{"id": i, "content": t, "special": True} for i, t in sorted(specials.items())]
    return {"model": {"vocab": vocab, "merges": merges}, "added_tokens": added}
