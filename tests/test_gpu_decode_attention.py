"""One decode token over a global layer (gemma4.c:443-456 with one token, a
full-attention layer) in reference order, bit-exact against the oracle over
score spreads from a flat row (every probability 2^-14) to very peaked rows,
value rows built for exact ties on the fma chain's grid and signed zeros,
values spread over 2^-30 .. 2^30, and key counts from one key to 64K.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def attend(pkg, lib, torch, oracle_lib, kc, vc, q, hd, ring, start):
    ref = np.empty_like(q)
    oracle_lib.oracle().orc_attend(ref.ctypes.data, q.ctypes.data, kc.ctypes.data, vc.ctypes.data,
                                   ring, hd, 8, 1, start, 1)
    out = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    kd, vd, qd = dev(torch, kc), dev(torch, vc), dev(torch, q)
    pkg.check(lib.g4_attend(None, out.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                            ring, hd, 8, 1, start, 1))
    torch.cuda.synchronize()
    return out.cpu().numpy(), ref


# head_dim, ring, position, query scale (the score spread is ~ scale * sqrt(head_dim)), values
CASES = [
    (512, 16384, 16383, 0.0, "normal"),     # a flat row: p = 2^-14 for every key
    (512, 16384, 16383, 0.01, "normal"),    # near-uniform
    (512, 16384, 16383, 0.25, "normal"),
    (512, 16384, 16383, 1.0, "normal"),     # the spread of normalized q.k at head_dim 512
    (512, 16384, 12345, 0.25, "ties"),      # small dyadic values: exact ties in the fma chain
    (512, 16384, 9000, 0.25, "zeros"),      # a third of the values +0 or -0
    (512, 16384, 16383, 0.25, "scaled"),    # values over 2^-30 .. 2^30
    (256, 8192, 5000, 0.25, "normal"),
    (512, 4096, 0, 0.25, "normal"),         # one key
    (512, 4096, 15, 0.25, "normal"),        # under one tile
    (512, 4096, 1023, 0.25, "normal"),      # 16 whole tiles of 64 keys
    (512, 4096, 1030, 0.25, "normal"),      # a partial last tile
    (512, 65536, 65535, 0.25, "normal"),    # 64K keys
]


@pytest.mark.parametrize("hd,ring,start,scale,values", CASES)
def test_decode_attention_bitexact(pkg, g4lib, torch_gpu, oracle_lib, hd, ring, start, scale, values):
    g = rng(1000 + hd + start + int(scale * 100))
    kc = g.standard_normal((ring, hd)).astype(np.float32)
    vc = g.standard_normal((ring, hd)).astype(np.float32)
    if values == "ties":
        vc = (g.integers(-64, 64, (ring, hd)) / 8.0).astype(np.float32)
    elif values == "zeros":
        u = g.random((ring, hd))
        vc[u < 0.2] = 0.0
        vc[(u >= 0.2) & (u < 0.33)] = -0.0
    elif values == "scaled":
        vc = (vc * np.exp2(g.integers(-30, 31, (ring, 1)))).astype(np.float32)
    q = (g.standard_normal((1, 8, hd)) * scale).astype(np.float32)
    o, ref = attend(pkg, g4lib, torch_gpu, oracle_lib, kc, vc, q, hd, ring, start)
    assert np.array_equal(o.view(np.uint32), ref.view(np.uint32)), int((o != ref).sum())
