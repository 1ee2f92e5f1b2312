"""The C ABI boundary: libg4.so loads, exports every function include/g4.h
declares, and its host-side argument checks fail with the documented status
before touching a device (no GPU needed)."""

from __future__ import annotations

import ctypes
import os

import numpy as np

from helpers import ROOT, header_functions


def test_header_declares_the_boundary():
    names = header_functions(os.path.join(ROOT, "include", "g4.h"))
    for required in ("g4_init", "g4_forward", "g4_logits", "g4_logits_all", "g4_argmax",
                     "g4_shutdown", "g4_last_error", "g4_stream", "g4_quantize", "g4_matmul_int8",
                     "g4_rmsnorm", "g4_add_and_scale", "g4_apply_rope", "g4_geglu",
                     "g4_embedding", "g4_attend"):
        assert required in names


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg.lib()
    for name in header_functions(os.path.join(ROOT, "include", "g4.h")):
        assert hasattr(lib, name), name
    img = pkg.img()
    for name in header_functions(os.path.join(ROOT, "include", "g4img.h")):
        assert hasattr(img, name), name
    # the Python binding covers the whole header
    assert set(header_functions(os.path.join(ROOT, "include", "g4.h"))) == set(pkg.exported_symbols())


def test_library_is_built_for_gfx950():
    data = open(os.path.join(ROOT, "gemma4.c_amd", "libg4.so"), "rb").read()
    assert b"gfx950" in data


def test_call_order_errors(pkg):
    lib = pkg.lib()
    toks = np.array([1, 2], np.int32)
    assert lib.g4_forward(toks.ctypes.data, 2, 0) == 3  # G4_ERR_STATE
    assert b"g4_init" in lib.g4_last_error()
    out = np.empty(16, np.float32)
    assert lib.g4_logits(0, out.ctypes.data) == 3
    tok = ctypes.c_int()
    assert lib.g4_argmax(0, ctypes.byref(tok)) == 3
    lib.g4_shutdown()  # harmless without init


def test_argument_errors(pkg):
    lib = pkg.lib()
    # the attention layer checks its arguments before any device call
    layer = (pkg.Tensor * 19)()
    assert lib.g4_attention_layer(None, None, 1, 0, layer, 16, 1024, 0) == 1
    assert b"null pointer" in lib.g4_last_error()
    assert lib.g4_attention_layer(None, 16, 0, 0, layer, 16, 1024, 0) == 1
    assert b"rows" in lib.g4_last_error()
    assert lib.g4_attention_layer(None, 16, 1, 0, layer, 16, 1024, 0) == 1  # empty records
    assert b"head_dim" in lib.g4_last_error()
    # width not a multiple of 64
    assert lib.g4_quantize(None, 16, 16, 16, 1, 100) == 1
    assert b"multiple of 64" in lib.g4_last_error()
    t = pkg.Tensor()
    t.data, t.scales = 64, 64
    t.shape[0], t.shape[1] = 17, 64  # not a multiple of 16 rows
    assert lib.g4_matmul_int8(None, 16, 16, 16, ctypes.byref(t), 1) == 1
    assert b"not packable" in lib.g4_last_error()
    assert lib.g4_attend(None, 16, 16, 16, 16, 1024, 128, 8, 0, 0, 1) == 1
    assert lib.g4_attend(None, 16, 16, 16, 16, 1000, 256, 8, 0, 0, 1) == 1  # not a power of two
    assert lib.g4_attend(None, 16, 16, 16, 16, 1024, 256, 8, 0, 600, 600) == 1  # exceeds the ring
    assert lib.g4_init(None, 0) == 1
