"""gemma4.c_amd -- MI355X (gfx950) W8A8 forward path for gemma4.c.

Python view of the C ABI in include/g4.h (libg4.so, hipcc-built HIP kernels)
and include/g4img.h (libg4img.so, the model-image loader and synthetic
writer).  The C host in host/ uses the same two libraries directly; this module
exists for the tests and bench.py.

The directory name is not a Python identifier, so load it with ``load()`` in
__graft_entry__.py (or importlib with this file as the package's __init__).

Nothing here falls back to a CPU implementation: if libg4.so is missing or was
built for another target, ``lib()`` raises.
"""

from __future__ import annotations

import ctypes
import mmap
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_G4 = os.path.join(PKG_DIR, "libg4.so")
LIB_IMG = os.path.join(PKG_DIR, "libg4img.so")

LAYERS = 35
HIDDEN = 1536
VOCAB = 262144
MAX_CONTEXT = 131072
WINDOW = 512
BATCH = 512
PLE = 256
HEADS = 8
RECORDS = 671

FFN_6144 = 1
UNIT_NORMS = 2
BF16_VALUES = 4

ORDER_REFERENCE = 0
ORDER_PARALLEL = 1

# Record indices (field order of gemma4.c:125-155).
EMBED, EMBED_PER_LAYER = 0, 1
NORM, PER_LAYER_MODEL_PROJECTION, PER_LAYER_PROJECTION_NORM, GELU_TABLE = 667, 668, 669, 670
FIELDS = (
    "input_layernorm", "layer_scalar", "pre_ffn_layernorm", "post_attn_layernorm",
    "post_ffn_layernorm", "post_per_layer_input_norm", "per_layer_input_gate",
    "per_layer_projection", "q_norm", "k_norm", "q_proj", "k_proj", "v_proj", "o_proj",
    "gate_proj", "up_proj", "down_proj", "rope_cos", "rope_sin",
)


def layer_record(layer: int, field: str) -> int:
    return 2 + layer * 19 + FIELDS.index(field)


class Tensor(ctypes.Structure):
    """The 32-byte tensor record (gemma4.c:119-123 / g4_tensor)."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("shape", ctypes.c_int32 * 4),
    ]


Records = Tensor * RECORDS

_c_p = ctypes.c_void_p
_c_sz = ctypes.c_size_t
_c_i = ctypes.c_int
_c_f = ctypes.c_float

_G4_SIGNATURES = {
    "g4_last_error": (ctypes.c_char_p, []),
    "g4_init": (_c_i, [ctypes.POINTER(Tensor), _c_i]),
    "g4_forward": (_c_i, [_c_p, _c_sz, _c_i]),
    "g4_logits": (_c_i, [_c_sz, _c_p]),
    "g4_logits_all": (_c_i, [_c_p]),
    "g4_argmax": (_c_i, [_c_sz, ctypes.POINTER(_c_i)]),
    "g4_sample": (_c_i, [_c_sz, ctypes.c_float, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(_c_i)]),
    "g4_sample_logits": (_c_i, [_c_p, _c_p, _c_i, ctypes.c_float, ctypes.POINTER(ctypes.c_uint64),
                                ctypes.POINTER(_c_i)]),
    "g4_shutdown": (None, []),
    "g4_stream": (_c_p, []),
    "g4_set_order": (_c_i, [_c_i]),
    "g4_softmax": (_c_i, [_c_p, _c_p, _c_i, _c_sz]),
    "g4_quantize": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_sz, _c_sz]),
    "g4_matmul_int8": (_c_i, [_c_p, _c_p, _c_p, _c_p, ctypes.POINTER(Tensor), _c_sz]),
    "g4_rmsnorm": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_i, _c_f, _c_sz]),
    "g4_add_and_scale": (_c_i, [_c_p, _c_p, _c_p, _c_sz, _c_f]),
    "g4_apply_rope": (_c_i, [_c_p, _c_p, _c_p, _c_i, _c_p, _c_i, _c_i, _c_i, _c_sz]),
    "g4_geglu": (_c_i, [_c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_p, _c_i, _c_f, _c_f]),
    "g4_embedding": (_c_i, [_c_p, _c_p, ctypes.POINTER(Tensor), _c_p, _c_sz, _c_f]),
    "g4_attend": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_i, _c_i, _c_sz]),
    "g4_attend_noalloc": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_i, _c_i, _c_sz]),
    "g4_attention_layer": (_c_i, [_c_p, _c_p, _c_sz, _c_i, ctypes.POINTER(Tensor), _c_p, _c_i, _c_i]),
}

class ImageItem(ctypes.Structure):
    """g4img_item (include/g4img.h): one distinct tensor of the image."""
    _fields_ = [("record", ctypes.c_int), ("kind", ctypes.c_int), ("rows", ctypes.c_int),
                ("cols", ctypes.c_int), ("global_rope", ctypes.c_int),
                ("data", ctypes.c_uint64), ("scales", ctypes.c_uint64)]


ITEM_QUANT, ITEM_VECTOR, ITEM_SCALAR, ITEM_ROPE_COS, ITEM_ROPE_SIN, ITEM_GELU = range(6)
DTYPE_F32, DTYPE_BF16, DTYPE_F16 = range(3)
TOKENIZER_SPAN = 33_429_932
DATA_START = 33_484_992

_IMG_SIGNATURES = {
    "g4img_size": (_c_sz, [ctypes.c_uint]),
    "g4img_layout": (_c_i, [ctypes.c_uint, ctypes.POINTER(ImageItem), _c_i]),
    "g4img_write_header": (_c_i, [_c_p, _c_sz, ctypes.c_uint]),
    "g4img_pack_matrix": (_c_i, [_c_p, _c_i, _c_i, _c_i, _c_p, _c_p, _c_i]),
    "g4img_fill_table": (_c_i, [_c_p, _c_sz, ctypes.POINTER(ImageItem), _c_i]),
    "g4img_draw": (_c_i, [ctypes.c_uint64, ctypes.c_uint, ctypes.POINTER(ImageItem), _c_p, _c_i, _c_i]),
    "g4img_generate": (_c_i, [_c_p, _c_sz, ctypes.c_uint64, ctypes.c_uint, _c_i]),
    "g4img_write_file": (_c_i, [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_uint, _c_i]),
    "g4img_records": (_c_i, [_c_p, _c_sz, ctypes.POINTER(Tensor)]),
    "g4img_fixup_inplace": (_c_i, [_c_p, _c_sz]),
    "g4img_last_error": (ctypes.c_char_p, []),
}

_libs: dict[str, ctypes.CDLL] = {}


def _bind(path: str, signatures: dict) -> ctypes.CDLL:
    if path in _libs:
        return _libs[path]
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run __graft_entry__.build() first")
    lib = ctypes.CDLL(path)
    for name, (restype, argtypes) in signatures.items():
        fn = getattr(lib, name)  # AttributeError names a missing export
        fn.restype = restype
        fn.argtypes = argtypes
    _libs[path] = lib
    return lib


def lib() -> ctypes.CDLL:
    """libg4.so, the HIP path.  Raises if it is not built."""
    return _bind(LIB_G4, _G4_SIGNATURES)


def img() -> ctypes.CDLL:
    """libg4img.so, the model-image tool."""
    return _bind(LIB_IMG, _IMG_SIGNATURES)


def exported_symbols() -> list[str]:
    return list(_G4_SIGNATURES)


class G4Error(RuntimeError):
    pass


def check(status: int) -> None:
    if status != 0:
        raise G4Error(f"g4 status {status}: {lib().g4_last_error().decode()}")


class Image:
    """A model image in anonymous memory (page aligned), synthetic or read
    from a file, with its record table fixed up into pointers."""

    def __init__(self, buf: mmap.mmap, size: int):
        self.buf = buf
        self.size = size
        self.base = ctypes.addressof(ctypes.c_char.from_buffer(buf))
        self.records = Records()
        self.fixed_inplace = False
        if img().g4img_records(self.base, size, self.records) != 0:
            raise G4Error(img().g4img_last_error().decode())

    def fixup_inplace(self) -> None:
        """Also rewrite the image's own record table to pointers, as the
        reference loader does (gemma4.c:681-685), for code that reads the image
        as a fixed-up Model.  self.records is unaffected."""
        if not self.fixed_inplace:
            if img().g4img_fixup_inplace(self.base, self.size) != 0:
                raise G4Error(img().g4img_last_error().decode())
            self.fixed_inplace = True

    @classmethod
    def synthetic(cls, seed: int, flags: int = 0, threads: int = 0) -> "Image":
        size = img().g4img_size(flags)
        buf = mmap.mmap(-1, size)
        base = ctypes.addressof(ctypes.c_char.from_buffer(buf))
        if img().g4img_generate(base, size, seed, flags, threads) != 0:
            raise G4Error(img().g4img_last_error().decode())
        return cls(buf, size)

    @classmethod
    def from_file(cls, path: str) -> "Image":
        size = os.path.getsize(path)
        buf = mmap.mmap(-1, size)
        with open(path, "rb") as f:
            f.readinto(memoryview(buf))
        return cls(buf, size)

    def record(self, index: int) -> Tensor:
        return self.records[index]

    def array(self, index: int, dtype=np.float32) -> np.ndarray:
        """fp32 record as a numpy view (norm weights, tables)."""
        t = self.records[index]
        shape = [s for s in t.shape[:2] if s > 0] or [1]
        if index == GELU_TABLE:
            shape = [t.shape[0]]
        count = int(np.prod(shape))
        ptr = ctypes.cast(t.data, ctypes.POINTER(ctypes.c_float))
        return np.ctypeslib.as_array(ptr, shape=(count,)).reshape(shape)

    def packed(self, index: int) -> tuple[np.ndarray, np.ndarray]:
        """Quantized record as (packed int8 bytes, fp16 scales) numpy views."""
        t = self.records[index]
        n, k = t.shape[0], t.shape[1]
        d = np.ctypeslib.as_array(ctypes.cast(t.data, ctypes.POINTER(ctypes.c_int8)), shape=(n * k,))
        s = np.ctypeslib.as_array(ctypes.cast(t.scales, ctypes.POINTER(ctypes.c_uint16)), shape=(n * k // 64,))
        return d, s.view(np.float16)


def unpack_weight(packed: np.ndarray, n: int, k: int) -> np.ndarray:
    """Packed tiles -> row-major int8 [n x k] (inverse of exporter.py:307-309)."""
    return packed.reshape(n // 16, k // 64, 16, 16, 4).transpose(0, 3, 1, 2, 4).reshape(n, k)


def pack_weight(w: np.ndarray) -> np.ndarray:
    """Row-major int8 [n x k] -> packed tiles (exporter.py:307-309)."""
    n, k = w.shape
    return np.ascontiguousarray(
        w.reshape(n // 16, 16, k // 64, 16, 4).transpose(0, 2, 3, 1, 4)).reshape(-1)


def pack_scales(s: np.ndarray) -> np.ndarray:
    """[n x k/64] fp16 scales -> [block][group][16] (exporter.py:310)."""
    n, g = s.shape
    return np.ascontiguousarray(s.reshape(n // 16, 16, g).transpose(0, 2, 1)).reshape(-1)
