"""The reference's sequential fp32 sums -- the softmax running sum
(gemma4.c:400-408) and the sum of squares of rmsnorm (gemma4.c:366-368) -- on
rows built so that the running sum passes a power of two B one ulp at a time.

The parallel evaluation cuts a row into runs of steps on one grid (the ulp of
a predicted binade) and resolves them against the exact sum.  A prediction
that differs from the exact sum by a few ulps is harmless anywhere but within
a few ulps of a power of two, so these rows keep the sum there for hundreds of
terms: the sum is brought to B - m ulp by a few large terms, then every term
is r ulp, r uniform in [2.05, 2.45], [1.55, 2.45] or [0.55, 0.95]: each
sequential step below B adds exactly R = rint(r) ulps (2, 2, 1), while a
prediction that sums the terms first leads the sequential sum by a quarter
ulp a term, wanders around it, or lags it, so neighbouring threads' predicted
ranges leave gaps or overlap right where the sum passes B; and a term rounded
on the grid of the binade above (rint(r / 2)) differs from R, so a step taken
on the wrong grid changes the sum.  The sum passes B near a chosen term, or
stops just short of it.  Each row goes through every block shape that
evaluates such a sum: per-op softmax rows of 300 and 511 values (64-term
blocks advanced from the exact sum) and of 3000 .. 20000 (16 waves x 4 terms
a thread, 16 x 8 in chunks of 8192), rmsnorm rows of 1536 (4 waves x 6), and
attention over designed scores (q a unit vector, so each score is one key
component exactly): global prefill rows (one wave x 8 terms, or 4 waves x 8
in chunks of 2048), global decode rows of 12001 keys (the split path:
per-chunk predicted starts, then the walk), and sliding-window rows of 512
keys in decode (8 waves x 1) and prefill (one wave x 8).  Bit for bit
against the oracle.
"""

from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

from conftest import rng
from helpers import HostF32

pytestmark = pytest.mark.gpu


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.fixture(scope="module")
def ok(oracle_lib):
    return oracle_lib.Kernels()


# term sizes in ulps: the prediction leads, wanders or lags
RANGES = [(2.05, 2.45), (1.55, 2.45), (0.55, 0.95)]


def crawl_scores(g, length, boundary, cross_at, short_by=0, r=RANGES[0]):
    """Softmax inputs whose running sum reaches `boundary` near term
    `cross_at` (or ends `short_by` ulps below it when short_by > 0).

    x_0 = 0 is the starting maximum (sum 1); boundary - 2 values of 0 add 1
    each; ln(1 - d) brings the sum to boundary - m u (u: the ulp just below
    boundary); every later value is ln(r u), a term of r ulps, which the
    sequential sum rounds to R = rint(r) ulps below boundary."""
    u = boundary * 2.0 ** -24
    ones = boundary - 2
    crawl = length - 2 - ones
    R = round(sum(r) / 2)
    m = R * crawl + short_by if short_by else R * (cross_at - 2 - ones)
    x = np.empty(length, np.float32)
    x[0] = 0.0
    x[1:1 + ones] = 0.0
    x[1 + ones] = np.log1p(-m * u)
    x[2 + ones:] = np.log(g.uniform(r[0], r[1], crawl) * u)
    return x.astype(np.float32)


def softmax_rows(g, length):
    rows = []
    for i in range(18):
        boundary, r = (2, 4, 8)[i % 3], RANGES[(i // 3) % 3]
        if i >= 16:  # ends two or three ulps short
            rows.append(crawl_scores(g, length, boundary, 0, short_by=2 + i % 2, r=r))
        else:
            rows.append(crawl_scores(g, length, boundary, int(g.integers(length // 5, length * 9 // 10)), r=r))
    return rows


@pytest.mark.parametrize("length", [300, 511, 3000, 4096, 6000, 12000, 20000])
def test_softmax_sum_crawls_past_power_of_two(pkg, g4lib, torch_gpu, ok, length):
    g = rng(7100 + length)
    block = np.stack(softmax_rows(g, length))
    d = dev(torch_gpu, block)
    pkg.check(g4lib.g4_softmax(None, d.data_ptr(), length, block.shape[0]))
    torch_gpu.cuda.synchronize()
    out = d.cpu().numpy()
    bad = [r for r in range(block.shape[0])
           if not np.array_equal(out[r].view(np.uint32), ok.softmax(block[r]).view(np.uint32))]
    assert not bad, f"rows {bad} of length {length}"


def test_rmsnorm_sum_of_squares_crawls_past_power_of_two(pkg, g4lib, torch_gpu, ok):
    """Width 1536 (the hidden rows): x_0^2 = B - m u, then squares of r ulps."""
    g = rng(7200)
    w = 1536
    rows = []
    for i in range(96):
        boundary, (lo, hi) = (2.0, 4.0, 1024.0, 2.0 ** -10)[i % 4], RANGES[(i // 4) % 3]
        u = boundary * 2.0 ** -24
        cross = int(g.integers(100, w - 100)) if i % 6 else w + 2  # every sixth ends short
        x = np.empty(w, np.float64)
        R = round((lo + hi) / 2)
        x[0] = np.sqrt(boundary - R * (cross - 1) * u)
        x[1:] = np.sqrt(g.uniform(lo, hi, w - 1) * u)
        x *= np.where(g.random(w) < 0.5, -1.0, 1.0)
        rows.append(x.astype(np.float32))
    x = np.stack(rows)
    wt = g.uniform(0.5, 1.5, w).astype(np.float32)
    xd, wd = dev(torch_gpu, x), dev(torch_gpu, wt)
    pkg.check(g4lib.g4_rmsnorm(None, xd.data_ptr(), xd.data_ptr(), wd.data_ptr(), w, 1e-6, x.shape[0]))
    torch_gpu.cuda.synchronize()
    out = xd.cpu().numpy()
    ref = ok.rmsnorm(x, HostF32(pkg, wt).record, w, 1e-6)
    bad = [r for r in range(x.shape[0]) if not np.array_equal(out[r].view(np.uint32), ref[r].view(np.uint32))]
    assert not bad, f"rows {bad}"


# head_dim, ring, full, tokens, start position, seed
ATTEND = [
    (512, 16384, 1, 64, 3000, 0),   # global prefill rows of 3001 .. 3064 keys: two chunks of 2048
    (512, 16384, 1, 64, 3000, 1),
    (512, 16384, 1, 32, 800, 2),    # one wave a row
    (512, 16384, 1, 1, 12000, 0),   # global decode over 12001 keys: the split path
    (512, 16384, 1, 1, 12000, 1),
    (512, 16384, 1, 3, 12000, 2),
    (256, 1024, 0, 1, 5000, 0),     # window decode: rows of 512 keys
    (256, 1024, 0, 1, 5000, 1),
    (256, 1024, 0, 2, 5000, 2),
    (256, 1024, 0, 16, 900, 3),     # window prefill
]


@pytest.mark.parametrize("hd,ring,full,n,start,seed", ATTEND)
def test_attention_softmax_crawls_past_power_of_two(pkg, g4lib, torch_gpu, oracle_lib, hd, ring, full, n,
                                                    start, seed):
    """Head h's query is the unit vector e_h, so its scores are component h
    of the keys, which holds a crawling row (a different crossing a head),
    laid out from the first key token 0 sees (later tokens see it shifted)."""
    heads = 8
    g = rng(7300 + 10 * seed + n + start)
    first = 0 if full else start - 511
    keys = start + n - first
    slots = (first + np.arange(keys)) % ring
    kc = np.zeros((ring, hd), np.float32)
    for h in range(heads):
        boundary, r = (2, 4, 8)[(h + seed) % 3], RANGES[(h + 2 * seed) % 3]
        if h == 7:  # ends short
            kc[slots, h] = crawl_scores(g, keys, boundary, 0, short_by=3, r=r)
        else:
            kc[slots, h] = crawl_scores(g, keys, boundary, int(g.integers(min(keys, start) // 5, min(keys, start))), r=r)
    vc = g.standard_normal((ring, hd)).astype(np.float32)
    q = np.zeros((n, heads, hd), np.float32)
    for h in range(heads):
        q[:, h, h] = 1.0
    ref = np.empty_like(q)
    oracle_lib.oracle().orc_attend(ref.ctypes.data, q.ctypes.data, kc.ctypes.data, vc.ctypes.data,
                                   ring, hd, heads, full, start, n)
    out = torch_gpu.empty(q.shape, dtype=torch_gpu.float32, device="cuda")
    kd, vd, qd = dev(torch_gpu, kc), dev(torch_gpu, vc), dev(torch_gpu, q)
    pkg.check(g4lib.g4_attend(None, out.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                              ring, hd, heads, full, start, n))
    torch_gpu.cuda.synchronize()
    o = out.cpu().numpy()
    bad = [(t, h) for t in range(n) for h in range(heads)
           if not np.array_equal(o[t, h].view(np.uint32), ref[t, h].view(np.uint32))]
    assert not bad, f"(token, head) {bad[:16]}"


FUZZ = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_bin", "esum_fuzz")


def test_engine_in_every_block_shape_against_the_sequential_loop(torch_gpu):
    """The engine itself (tests/esum_fuzz.hip, built by build(): it includes
    the library's source), one row of 64 NW J terms a block, in every block
    shape the kernels use and both modes, over 45,600 generated rows (random
    magnitudes, sums crawling past powers of two, peaked rows, a new maximum
    at every step, ties, zeros, subnormal and huge terms), against the plain
    sequential fp32 loop on the host, bit for bit.  The engine as it was
    before the thread-boundary rule fails rows of every shape here."""
    assert os.path.exists(FUZZ), "tests/_bin/esum_fuzz is missing: run __graft_entry__.build()"
    run = subprocess.run([FUZZ], capture_output=True, text=True, timeout=120)
    print(run.stdout)
    assert run.returncode == 0, run.stdout[-3000:] + run.stderr[-2000:]
    assert "all rows equal" in run.stdout
