"""Many-token attention (gemma4.c:443-456 for a prefill chunk) in reference
order, bit-exact against the oracle on inputs that separate a fused
multiply-add chain from any other rounding: the prefill kernels step each
score's 16 chains and each output's chain over the keys on the fp32 matrix
cores (one product a step), so these cases pin that every step rounds once,
like fmaf, with subnormal products, signed zeros and values over 2^-30 .. 2^30,
flat and tied rows, and token counts that leave partial tiles.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def attend(pkg, lib, torch, oracle_lib, kc, vc, q, hd, ring, full, start, n):
    ref = np.empty_like(q)
    oracle_lib.oracle().orc_attend(ref.ctypes.data, q.ctypes.data, kc.ctypes.data, vc.ctypes.data,
                                   ring, hd, 8, full, start, n)
    out = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    kd, vd, qd = dev(torch, kc), dev(torch, vc), dev(torch, q)
    pkg.check(lib.g4_attend(None, out.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                            ring, hd, 8, full, start, n))
    torch.cuda.synchronize()
    return out.cpu().numpy(), ref


# head_dim, ring, full, start, tokens, inputs
CASES = [
    (256, 1024, 0, 0, 61, "subnormal"),    # q.k products below 2^-126 in every chain
    (256, 1024, 0, 470, 77, "zeros"),      # +0 / -0 in queries, keys and values
    (256, 1024, 0, 700, 33, "ties"),       # dyadic values: exact ties in both chains
    (256, 1024, 0, 100, 45, "scaled"),     # values over 2^-30 .. 2^30
    (256, 1024, 0, 300, 29, "flat"),       # q = 0: every score 0, equal probabilities
    (512, 2048, 1, 0, 70, "subnormal"),
    (512, 2048, 1, 555, 38, "zeros"),
    (512, 2048, 1, 1000, 21, "ties"),
    (512, 2048, 1, 900, 53, "scaled"),
    (512, 2048, 1, 64, 9, "flat"),
    # more than 512 tokens in one call: one key block per 4-token group,
    # each block striding over every pass of its keys
    (256, 2048, 0, 100, 1100, "normal"),
    (512, 4096, 1, 0, 700, "normal"),
]


@pytest.mark.parametrize("hd,ring,full,start,n,inputs", CASES)
def test_prefill_attention_bitexact(pkg, g4lib, torch_gpu, oracle_lib, hd, ring, full, start, n, inputs):
    g = rng(2000 + hd + start + n)
    kc = g.standard_normal((ring, hd)).astype(np.float32)
    vc = g.standard_normal((ring, hd)).astype(np.float32)
    q = (g.standard_normal((n, 8, hd)) * 0.25).astype(np.float32)
    if inputs == "subnormal":
        # |q| ~ 2^-70, |k| ~ 2^-60: products ~ 2^-130, below the normal range
        q = (q * np.float32(2.0 ** -70)).astype(np.float32)
        kc = (kc * np.float32(2.0 ** -60)).astype(np.float32)
        vc[:, ::7] = (vc[:, ::7] * np.float32(2.0 ** -140)).astype(np.float32)
    elif inputs == "zeros":
        for a in (q, kc, vc):
            u = g.random(a.shape)
            a[u < 0.2] = 0.0
            a[(u >= 0.2) & (u < 0.33)] = -0.0
    elif inputs == "ties":
        q = (g.integers(-8, 8, q.shape) / 16.0).astype(np.float32)
        kc = (g.integers(-8, 8, kc.shape) / 16.0).astype(np.float32)
        vc = (g.integers(-64, 64, vc.shape) / 8.0).astype(np.float32)
    elif inputs == "scaled":
        vc = (vc * np.exp2(g.integers(-30, 31, (ring, 1)))).astype(np.float32)
        kc = (kc * np.exp2(g.integers(-4, 5, (ring, 1)))).astype(np.float32)
    elif inputs == "flat":
        q[:] = 0.0
    o, ref = attend(pkg, g4lib, torch_gpu, oracle_lib, kc, vc, q, hd, ring, full, start, n)
    assert np.array_equal(o.view(np.uint32), ref.view(np.uint32)), int((o.view(np.uint32) != ref.view(np.uint32)).sum())
