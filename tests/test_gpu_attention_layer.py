"""g4_attention_layer (one layer's attention(), gemma4.c:411-461) through the
C ABI against the oracle's attention layer -- itself pinned bit for bit to the
compiled reference's attention() in test_oracle.py -- on the same hidden rows
and prior cache rows: the output rows and the cache owner's rows identical bit
for bit.  Cases: a sliding layer's first chunk (the three projections in one
launch), a later chunk over the wrapped ring, a global layer, and two shared
layers that only read a cache (one decode row, a ragged batch of 3).  The
same cases in G4_ORDER_PARALLEL are held to stated tolerances."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from helpers import record_sizes
from test_oracle import ATTENTION_LAYER_CASES, attention_layer_inputs

pytestmark = pytest.mark.gpu

USED_FIELDS = (8, 9, 10, 11, 12, 13, 17, 18)  # q/k norms, q/k/v/o, RoPE tables


def device_layer(pkg, torch, image, layer: int):
    """The layer's 19 records with the fields attention() reads on the device
    (the others empty); returns the records and the tensors that hold them."""
    recs = (pkg.Tensor * 19)()
    keep = []
    for f in USED_FIELDS:
        index = 2 + layer * 19 + f
        src = image.records[index]
        for i in range(4):
            recs[f].shape[i] = src.shape[i]
        if not src.data:
            continue
        nbytes, sbytes = record_sizes(src, index)
        data = np.ctypeslib.as_array(ctypes.cast(src.data, ctypes.POINTER(ctypes.c_uint8)), shape=(nbytes,))
        d = torch.from_numpy(data.copy()).cuda()
        keep.append(d)
        recs[f].data = d.data_ptr()
        if sbytes:
            sc = np.ctypeslib.as_array(ctypes.cast(src.scales, ctypes.POINTER(ctypes.c_uint8)), shape=(sbytes,))
            ds = torch.from_numpy(sc.copy()).cuda()
            keep.append(ds)
            recs[f].scales = ds.data_ptr()
    return recs, keep


def run_case(pkg, g4lib, torch, image, oracle_lib, layer, start_pos, n):
    """The oracle's attention layer and g4_attention_layer (in the library's
    current order) on one case: (want_hidden, want_cache, got_hidden, got_cache)."""
    owner, hidden, slots, keys, values = attention_layer_inputs(layer, start_pos, n)
    full = owner % 5 == 4
    hd = 512 if full else 256
    cache_len = 4096 if full else 1024  # every position of the cases fits
    print(f"case layer={layer} start_pos={start_pos} n={n}", flush=True)

    # the oracle
    m = oracle_lib.Model(image)
    kc, vc = m.cache(owner)
    kc[slots], vc[slots] = keys, values
    m.hidden(n)[:] = hidden
    m.attention_layer(layer, start_pos, n)
    want_hidden = m.hidden(n).copy()
    want_cache = np.stack([kc[:cache_len], vc[:cache_len]]).copy()
    m.close()

    # the device
    recs, keep = device_layer(pkg, torch, image, layer)
    cache = np.zeros((2, cache_len, hd), np.float32)
    cache[0, slots & (cache_len - 1)], cache[1, slots & (cache_len - 1)] = keys, values
    cache_d = torch.from_numpy(cache).cuda()
    hidden_d = torch.from_numpy(hidden.copy()).cuda()
    stream = torch.cuda.current_stream().cuda_stream
    pkg.check(g4lib.g4_attention_layer(stream, hidden_d.data_ptr(), n, start_pos, recs,
                                       cache_d.data_ptr(), cache_len, int(full)))
    torch.cuda.synchronize()
    got_hidden = hidden_d.cpu().numpy()
    got_cache = cache_d.cpu().numpy()
    del keep
    return want_hidden, want_cache, got_hidden, got_cache


@pytest.mark.parametrize("layer,start_pos,n", ATTENTION_LAYER_CASES)
def test_attention_layer_bitexact(pkg, g4lib, torch_gpu, image, oracle_lib, layer, start_pos, n):
    want_hidden, want_cache, got_hidden, got_cache = run_case(pkg, g4lib, torch_gpu, image, oracle_lib,
                                                              layer, start_pos, n)
    assert np.array_equal(got_hidden.view(np.uint32), want_hidden.view(np.uint32)), \
        f"max |d| {np.abs(got_hidden - want_hidden).max()}"
    assert np.array_equal(got_cache.view(np.uint32), want_cache.view(np.uint32))


# G4_ORDER_PARALLEL against the reference order, per layer.  The cache rows
# written (k_norm + RoPE, the unweighted v norm) differ from the oracle's only
# by the norms' tree sums: a few ulp of the row, bounded here at 1e-5 of its
# RMS.  The output rows pass through the int8 requantization of the attention
# output (k_quantize's rint): where the parallel order moves x / scale across
# a rounding boundary one activation moves by one step, and the whole output
# row by scale x one weight column -- about 5e-4 of the row's RMS a step.
# Bounded at 2e-2 of the row's RMS (dozens of such steps); a wiring mistake
# (another head's query, a RoPE position off by one, a wrong ring slot) moves
# the rows by their own size.
PARALLEL_CACHE_TOL = 1e-5
PARALLEL_OUT_TOL = 2e-2


@pytest.mark.parametrize("layer,start_pos,n", ATTENTION_LAYER_CASES)
def test_attention_layer_parallel_order(pkg, g4lib, torch_gpu, image, oracle_lib, layer, start_pos, n):
    previous = g4lib.g4_set_order(pkg.ORDER_PARALLEL)
    try:
        want_hidden, want_cache, got_hidden, got_cache = run_case(pkg, g4lib, torch_gpu, image, oracle_lib,
                                                                  layer, start_pos, n)
    finally:
        g4lib.g4_set_order(previous)
    flat_want = want_cache.reshape(-1, want_cache.shape[-1])
    flat_got = got_cache.reshape(-1, got_cache.shape[-1])
    rms_c = np.sqrt(np.mean(flat_want.astype(np.float64) ** 2, axis=1, keepdims=True))
    dc = np.abs(flat_got - flat_want)
    assert np.all(dc <= PARALLEL_CACHE_TOL * rms_c + 1e-30), f"cache: max |d| / rms {np.max(dc / (rms_c + 1e-30)):.3g}"
    rms_h = np.sqrt(np.mean(want_hidden.astype(np.float64) ** 2, axis=1, keepdims=True))
    rel = np.abs(got_hidden - want_hidden) / rms_h
    moved = int(np.sum(rel.max(axis=1) > 1e-5))
    print(f"parallel order: cache max |d|/rms {np.max(dc / (rms_c + 1e-30)):.3g}; output max |d|/rms "
          f"{rel.max():.3g}, median {np.median(rel):.3g}; rows moved past 1e-5: {moved}/{n}", flush=True)
    assert rel.max() <= PARALLEL_OUT_TOL


def test_attention_layer_rejects_bad_calls(pkg, g4lib, torch_gpu, image):
    torch = torch_gpu
    recs, keep = device_layer(pkg, torch, image, 0)
    hidden_d = torch.zeros((4, 1536), device="cuda")
    cache_d = torch.zeros((2, 1024, 256), device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    call = lambda *a: g4lib.g4_attention_layer(stream, hidden_d.data_ptr(), *a)
    assert call(0, 0, recs, cache_d.data_ptr(), 1024, 0) == 1          # no rows
    assert call(4, 0, recs, cache_d.data_ptr(), 1000, 0) == 1          # not a power of two
    assert call(4, 1022, recs, cache_d.data_ptr(), 1024, 0) == 0       # the window fits the ring
    assert call(4, 600, recs, cache_d.data_ptr(), 256, 0) == 1         # window + batch exceed the ring
    bad = (pkg.Tensor * 19)()
    ctypes.memmove(bad, recs, ctypes.sizeof(bad))
    bad[8].shape[0] = 128                                              # head_dim 128
    assert call(4, 0, bad, cache_d.data_ptr(), 1024, 0) == 1
    torch.cuda.synchronize()
    del keep
