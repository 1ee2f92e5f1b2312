"""g4_attend_noalloc (the allocation-free variant of g4_attend) against
g4_attend itself: bit-identical outputs on two calls in a row, the second
smaller than the first, in both summation orders; oversized calls are refused
before anything is launched."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu

# (head_dim, ring, full, start_pos, n): a long-context decode call, then a
# smaller prefill chunk; a sliding prefill chunk, then a one-token decode
PAIRS = [
    ((512, 16384, 1, 16000, 4), (512, 4096, 1, 1000, 64)),
    ((256, 1024, 0, 700, 301), (256, 1024, 0, 1500, 1)),
]


def _inputs(torch, hd, ring, start, n):
    g = rng(hd * 3 + start + n)
    kc = torch.from_numpy(g.standard_normal((ring, hd)).astype(np.float32)).cuda()
    vc = torch.from_numpy(g.standard_normal((ring, hd)).astype(np.float32)).cuda()
    q = torch.from_numpy((g.standard_normal((n, 8, hd)) * 0.25).astype(np.float32)).cuda()
    return kc, vc, q


def _call(pkg, fn, torch, case, inputs):
    hd, ring, full, start, n = case
    kc, vc, q = inputs
    out = torch.full(q.shape, float("nan"), dtype=torch.float32, device="cuda")
    pkg.check(fn(None, out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), ring, hd, 8, full,
                 start, n))
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("order", [0, 1])
@pytest.mark.parametrize("pair", PAIRS)
def test_noalloc_matches_attend(pkg, g4lib, torch_gpu, order, pair):
    torch = torch_gpu
    previous = g4lib.g4_set_order(order)
    try:
        for case in pair:
            print(f"noalloc case order={order} {case}", flush=True)
            inputs = _inputs(torch, case[0], case[1], case[3], case[4])
            want = _call(pkg, g4lib.g4_attend, torch, case, inputs)
            got = _call(pkg, g4lib.g4_attend_noalloc, torch, case, inputs)
            assert np.isfinite(want).all()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (order, case)
    finally:
        g4lib.g4_set_order(previous)


def test_noalloc_refuses_oversized_calls(pkg, g4lib, torch_gpu):
    """A 512-token chunk at 16K keys needs 512 x 8 x 16384 floats of scores
    (256 MiB) in reference order: refused (status G4_ERR_ARG) before any
    launch, and the output is left untouched."""
    torch = torch_gpu
    hd, ring, n = 512, 32768, 512
    kc = torch.zeros((ring, hd), dtype=torch.float32, device="cuda")
    q = torch.zeros((n, 8, hd), dtype=torch.float32, device="cuda")
    out = torch.full((n, 8, hd), 7.0, dtype=torch.float32, device="cuda")
    status = g4lib.g4_attend_noalloc(None, out.data_ptr(), q.data_ptr(), kc.data_ptr(), kc.data_ptr(),
                                     ring, hd, 8, 1, 16000, n)
    torch.cuda.synchronize()
    assert status == 1, status
    assert b"scratch" in g4lib.g4_last_error()
    assert bool((out == 7.0).all())
