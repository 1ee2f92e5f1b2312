"""ctypes binding of the oracle (liboracle.so) and of the compiled reference
(oracle/_ref/libgemma4ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the CPU baseline, never
as the product path.
"""

from __future__ import annotations

import ctypes
import mmap
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_ORACLE = os.path.join(HERE, "liboracle.so")
LIB_REF = os.path.join(HERE, "_ref", "libgemma4ref.so")

VOCAB = 262144
HIDDEN = 1536

_p = ctypes.c_void_p
_sz = ctypes.c_size_t
_i = ctypes.c_int
_f = ctypes.c_float

# name in the oracle, name in the reference, restype, argtypes
_KERNELS = [
    ("orc_quantize", "quantize", None, [_p, _p, _p, _sz, _sz]),
    ("orc_matmul_int8", "matmul_int8", None, [_p, _p, _p, _p, _sz]),
    ("orc_attention_scores", "attention_scores", None, [_p, _p, _p, _i, _i, _i, _i]),
    ("orc_softmax", "softmax", None, [_p, _i]),
    ("orc_weighted_value_sum", "weighted_value_sum", None, [_p, _p, _p, _i, _i, _i, _i]),
    ("orc_geglu", "geglu", None, [_p, _p, _i, _i, _i, _p]),
    ("orc_embedding", "embedding", None, [_p, _p, _p, _sz, _f]),
    ("orc_rmsnorm", "rmsnorm", None, [_p, _p, _p, _i, _f, _sz]),
    ("orc_add_and_scale", "add_and_scale", None, [_p, _p, _sz, _f]),
    ("orc_apply_rope", "apply_rope", None, [_p, _p, _p, _i, _i, _i, _sz]),
    ("orc_forward", "forward", None, [_p, _p, _p, _sz, _i]),
    ("orc_logits", "logits", ctypes.POINTER(ctypes.c_float), [_p, _p, _sz]),
]

_ORACLE_EXTRA = {
    "orc_state_new": (_p, []),
    "orc_state_free": (None, [_p]),
    "orc_state_reset": (None, [_p]),
    "orc_state_cache": (ctypes.POINTER(ctypes.c_float), [_p, _i, ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "orc_state_residual": (ctypes.POINTER(ctypes.c_float), [_p]),
    "orc_state_hidden": (ctypes.POINTER(ctypes.c_float), [_p]),
    "orc_attention_layer": (None, [_p, _p, _i, _i, _sz]),
    "orc_set_threads": (None, [_i]),
    "orc_threads": (_i, []),
    "orc_set_fast": (None, [_i]),
    "orc_fast_available": (_i, []),
    "orc_f16_to_f32": (_f, [ctypes.c_uint16]),
    "orc_attend": (None, [_p, _p, _p, _p, _i, _i, _i, _i, _i, _sz]),
    "orc_sample": (_i, [_p, _i, _f, ctypes.POINTER(ctypes.c_uint64)]),
}

_REF_EXTRA = {
    "ref_state_size": (_sz, []),
    "ref_off_residual": (_sz, []),
    "ref_off_hidden": (_sz, []),
    "ref_off_sliding": (_sz, []),
    "ref_off_full": (_sz, []),
    "ref_model_weights_offset": (_sz, []),
    "attention": (None, [_p, _p, _i, _i, _sz, _p]),
    "ref_thread_count": (_i, []),
    "sample": (_i, [_p, _i, _f]),
}

_cache: dict[str, ctypes.CDLL] = {}


def _load(path: str, which: int, extra: dict) -> ctypes.CDLL:
    if path in _cache:
        return _cache[path]
    if not os.path.exists(path):
        raise FileNotFoundError(path)
    lib = ctypes.CDLL(path)
    for entry in _KERNELS:
        fn = getattr(lib, entry[which])
        fn.restype, fn.argtypes = entry[2], entry[3]
    for name, (restype, argtypes) in extra.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = restype, argtypes
    _cache[path] = lib
    return lib


def oracle() -> ctypes.CDLL:
    return _load(LIB_ORACLE, 0, _ORACLE_EXTRA)


def ref_available() -> bool:
    return os.path.exists(LIB_REF)


def ref() -> ctypes.CDLL:
    return _load(LIB_REF, 1, _REF_EXTRA)


def ptr(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


class Kernels:
    """Uniform numpy-level calls into either the oracle or the reference."""

    def __init__(self, use_ref: bool = False):
        self.is_ref = use_ref
        self.lib = ref() if use_ref else oracle()
        self.n = 1 if use_ref else 0

    def _fn(self, index: int):
        return getattr(self.lib, _KERNELS[index][self.n])

    def quantize(self, x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, width = x.shape
        q = np.empty((rows, width), np.int8)
        s = np.empty((rows, width // 64), np.float32)
        self._fn(0)(ptr(q), ptr(s), ptr(x), rows, width)
        return q, s

    def matmul(self, xq: np.ndarray, xs: np.ndarray, tensor, n: int) -> np.ndarray:
        rows = xq.shape[0]
        out = np.empty((rows, n), np.float32)
        self._fn(1)(ptr(out), ptr(xq), ptr(xs), ctypes.addressof(tensor), rows)
        return out

    def scores(self, q, kc, first, num, mask, hd):
        out = np.empty(num, np.float32)
        self._fn(2)(ptr(out), ptr(q), ptr(kc), first, num, mask, hd)
        return out

    def softmax(self, v: np.ndarray) -> np.ndarray:
        v = np.array(v, dtype=np.float32)
        self._fn(3)(ptr(v), v.size)
        return v

    def value_sum(self, p, vc, first, num, mask, hd):
        out = np.empty(hd, np.float32)
        self._fn(4)(ptr(out), ptr(p), ptr(vc), first, num, mask, hd)
        return out

    def geglu(self, gate, up, up_stride, table_tensor):
        gate = np.array(gate, dtype=np.float32)
        rows, width = gate.shape
        self._fn(5)(ptr(gate), ptr(up), rows, width, up_stride, ctypes.addressof(table_tensor))
        return gate

    def embedding(self, table_tensor, tokens, mult):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty((tokens.size, table_tensor.shape[1]), np.float32)
        self._fn(6)(ptr(out), ctypes.addressof(table_tensor), ptr(tokens), tokens.size, mult)
        return out

    def rmsnorm(self, x, weight_tensor, width, eps):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty_like(x)
        rows = x.size // width
        w = ctypes.addressof(weight_tensor) if weight_tensor is not None else None
        self._fn(7)(ptr(out), ptr(x), w, width, eps, rows)
        return out

    def add_and_scale(self, out, add, scale):
        out = np.array(out, dtype=np.float32)
        self._fn(8)(ptr(out), ptr(np.ascontiguousarray(add, dtype=np.float32)), out.size, scale)
        return out

    def rope(self, cos_t, sin_t, v, heads, hd, start_pos):
        v = np.array(v, dtype=np.float32)
        n = v.size // (heads * hd)
        self._fn(9)(ctypes.addressof(cos_t), ctypes.addressof(sin_t), ptr(v), heads, hd, start_pos, n)
        return v


class Model:
    """forward()/logits() of either the oracle or the compiled reference over
    one model image, with that implementation's own state."""

    def __init__(self, image, use_ref: bool = False):
        self.image = image
        self.is_ref = use_ref
        if use_ref:
            self.lib = ref()
            # The reference reads a fixed-up Model in place (gemma4.c:681-685).
            image.fixup_inplace()
            self.model = image.base
            size = self.lib.ref_state_size()
            self._state_buf = mmap.mmap(-1, size)
            self.state = ctypes.addressof(ctypes.c_char.from_buffer(self._state_buf))
            self._fwd, self._lg = self.lib.forward, self.lib.logits
        else:
            self.lib = oracle()
            self.model = ctypes.addressof(image.records)
            self.state = self.lib.orc_state_new()
            if not self.state:
                raise MemoryError("orc_state_new")
            self._fwd, self._lg = self.lib.orc_forward, self.lib.orc_logits

    def forward(self, tokens, start_pos: int) -> None:
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        assert 1 <= tokens.size <= 512
        self._fwd(self.model, self.state, ptr(tokens), tokens.size, start_pos)

    def logits(self, row: int) -> np.ndarray:
        p = self._lg(self.model, self.state, row)
        return np.ctypeslib.as_array(p, shape=(VOCAB,)).copy()

    def fill_kv_random(self, positions: int, seed: int) -> None:
        """Fill rows 0 .. positions - 1 of the three global KV caches and every
        row of the twelve sliding rings with N(0,1) values: a stand-in for a
        long prefill where only the timing of later steps matters (the cache
        rows the model writes are RMS-normalized, so of that scale).  The
        compiled reference's own state layout (gemma4.c:157-167)."""
        assert self.is_ref and 0 < positions <= 131072
        rng = np.random.default_rng(seed)
        full = self.lib.ref_off_full()
        ring = 131072 * 512
        for owner in range(3):
            for part in range(2):  # keys, then values
                at = full + (owner * 2 * ring + part * ring) * 4
                view = np.frombuffer(self._state_buf, np.float32, positions * 512, at)
                view[:] = rng.standard_normal(positions * 512, dtype=np.float32)
        sliding = self.lib.ref_off_sliding()
        count = 12 * 2 * 1024 * 256
        np.frombuffer(self._state_buf, np.float32, count, sliding)[:] = rng.standard_normal(count, dtype=np.float32)

    def residual(self, rows: int) -> np.ndarray:
        if self.is_ref:
            off = self.lib.ref_off_residual()
            p = ctypes.cast(self.state + off, ctypes.POINTER(ctypes.c_float))
        else:
            p = self.lib.orc_state_residual(self.state)
        return np.ctypeslib.as_array(p, shape=(rows * HIDDEN,)).reshape(rows, HIDDEN).copy()

    def hidden(self, rows: int) -> np.ndarray:
        """Writable view of the state's first `rows` hidden rows (the input
        and output of attention(), gemma4.c:483-484)."""
        if self.is_ref:
            p = ctypes.cast(self.state + self.lib.ref_off_hidden(), ctypes.POINTER(ctypes.c_float))
        else:
            p = self.lib.orc_state_hidden(self.state)
        return np.ctypeslib.as_array(p, shape=(rows * HIDDEN,)).reshape(rows, HIDDEN)

    def cache(self, owner: int) -> tuple[np.ndarray, np.ndarray]:
        """Writable (keys, values) views of cache owner `owner` (0..14):
        [cache_len x head_dim] each, as the implementation holds them
        (gemma4.c:164-165, 421-422)."""
        full = owner % 5 == 4
        cache_len, hd = (131072, 512) if full else (1024, 256)
        if self.is_ref:
            if full:
                at = self.lib.ref_off_full() + (owner // 5) * 2 * cache_len * hd * 4
            else:
                at = self.lib.ref_off_sliding() + ((owner // 5) * 4 + owner % 5) * 2 * cache_len * hd * 4
            p = ctypes.cast(self.state + at, ctypes.POINTER(ctypes.c_float))
        else:
            cl, d = ctypes.c_int(), ctypes.c_int()
            p = self.lib.orc_state_cache(self.state, owner, ctypes.byref(cl), ctypes.byref(d))
            assert (cl.value, d.value) == (cache_len, hd)
        both = np.ctypeslib.as_array(p, shape=(2 * cache_len * hd,)).reshape(2, cache_len, hd)
        return both[0], both[1]

    def attention_layer(self, layer: int, start_pos: int, n: int) -> None:
        """attention() of one layer over the first n hidden rows (gemma4.c:411-461)."""
        if self.is_ref:  # its orphaned `omp for` runs on this one thread
            layers = self.model + self.lib.ref_model_weights_offset() + 2 * 32
            scores = np.empty(start_pos + n, np.float32)
            self.lib.attention(self.state, layers, layer, start_pos, n, ptr(scores))
        else:
            self.lib.orc_attention_layer(self.model, self.state, layer, start_pos, n)

    def close(self) -> None:
        if not self.is_ref and self.state:
            self.lib.orc_state_free(self.state)
            self.state = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
