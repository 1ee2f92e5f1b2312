"""Per-op parity of the HIP kernels (through the C ABI) with the oracle and
with the reference's golden vectors.

Bars: bit-exact for quantize, matmul_int8 (int32 group dots + ordered fold),
rope, geglu, embedding, add_and_scale, and -- in the default reference
summation order -- rmsnorm, softmax and attention.  In the parallel order,
rmsnorm is held within 1e-5 and attention within 2e-5 of the output scale.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import random_weight, rng
from helpers import DeviceWeight, HostF32, HostWeight, load_golden

pytestmark = pytest.mark.gpu


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


@pytest.fixture(scope="module")
def ok(oracle_lib):
    return oracle_lib.Kernels()


def gpu_quantize(pkg, lib, torch, x):
    xd = dev(torch, x)
    q = torch.empty(x.shape, dtype=torch.int8, device="cuda")
    s = torch.empty((x.shape[0], x.shape[1] // 64), dtype=torch.float32, device="cuda")
    pkg.check(lib.g4_quantize(None, q.data_ptr(), s.data_ptr(), xd.data_ptr(), x.shape[0], x.shape[1]))
    torch.cuda.synchronize()
    return host(q), host(s)


def gpu_matmul(pkg, lib, torch, dw, xq, xs):
    rows = xq.shape[0]
    out = torch.empty((rows, dw.record.shape[0]), dtype=torch.float32, device="cuda")
    xqd, xsd = dev(torch, xq), dev(torch, xs)  # keep both alive until the kernel has run
    pkg.check(lib.g4_matmul_int8(None, out.data_ptr(), xqd.data_ptr(), xsd.data_ptr(), dw.record, rows))
    torch.cuda.synchronize()
    return host(out)


def test_quantize_bitexact(pkg, g4lib, torch_gpu, ok):
    g = rng(41)
    x = (g.standard_normal((37, 2048)) * g.uniform(1e-3, 1e3, (37, 1))).astype(np.float32)
    x[2] = 0
    x[3, 5] = 3e4
    q, s = gpu_quantize(pkg, g4lib, torch_gpu, x)
    q0, s0 = ok.quantize(x)
    assert np.array_equal(q, q0) and np.array_equal(s, s0)


def test_quantize_golden(pkg, g4lib, torch_gpu):
    gold = load_golden("ops.npz")
    q, s = gpu_quantize(pkg, g4lib, torch_gpu, gold["quant_x"])
    assert np.array_equal(q, gold["quant_q"]) and np.array_equal(s, gold["quant_s"])


def test_matmul_golden(pkg, g4lib, torch_gpu):
    gold = load_golden("ops.npz")
    for name in ("mm_a", "mm_b"):
        hw = HostWeight(pkg, gold[f"{name}_w"], gold[f"{name}_ws"])
        y = gpu_matmul(pkg, g4lib, torch_gpu, DeviceWeight(pkg, torch_gpu, hw), gold[f"{name}_xq"], gold[f"{name}_xs"])
        assert np.array_equal(y, gold[f"{name}_y"]), name


# Every linear shape of a Gemma-4-E2B layer (N x K) plus the lm_head.
DECODE_SHAPES = [(2048, 1536), (4096, 1536), (256, 1536), (512, 1536), (1536, 2048), (1536, 4096),
                 (6144, 1536), (12288, 1536), (1536, 6144), (1536, 12288), (256, 1536), (1536, 256),
                 (8960, 1536), (262144, 1536)]


@pytest.mark.parametrize("n,k", DECODE_SHAPES)
def test_matmul_decode_shapes_bitexact(pkg, g4lib, torch_gpu, ok, n, k):
    g = rng(n + k)
    w, s = random_weight(g, n, k)
    hw = HostWeight(pkg, w, s)
    dw = DeviceWeight(pkg, torch_gpu, hw)
    xq, xs = ok.quantize(g.standard_normal((1, k)).astype(np.float32))
    y = gpu_matmul(pkg, g4lib, torch_gpu, dw, xq, xs)
    assert np.array_equal(y, ok.matmul(xq, xs, hw.record, n))
    # a second call on the same buffers gives the same bits (no state carried over)
    assert np.array_equal(gpu_matmul(pkg, g4lib, torch_gpu, dw, xq, xs), y)


@pytest.mark.parametrize("rows", [1, 2, 3, 5, 8, 9, 17, 64, 100, 512])
def test_matmul_row_counts_bitexact(pkg, g4lib, torch_gpu, ok, rows):
    g = rng(rows)
    n, k = 1536, 2048
    w, s = random_weight(g, n, k)
    hw = HostWeight(pkg, w, s)
    xq, xs = ok.quantize(g.standard_normal((rows, k)).astype(np.float32))
    y = gpu_matmul(pkg, g4lib, torch_gpu, DeviceWeight(pkg, torch_gpu, hw), xq, xs)
    assert np.array_equal(y, ok.matmul(xq, xs, hw.record, n))


# Prefill products of a layer: grids of up to 256 blocks take 8-wave blocks,
# larger ones 4-wave blocks (launch_matmul).
@pytest.mark.parametrize("rows,n,k", [(512, 256, 1536), (512, 2048, 1536), (200, 1536, 6144),
                                      (64, 1536, 12288), (1000, 512, 1536), (512, 1536, 2048),
                                      (300, 1536, 4096)])
def test_matmul_prefill_shapes_bitexact(pkg, g4lib, torch_gpu, ok, rows, n, k):
    g = rng(rows * 7 + n + k)
    w, s = random_weight(g, n, k)
    hw = HostWeight(pkg, w, s)
    xq, xs = ok.quantize(g.standard_normal((rows, k)).astype(np.float32))
    y = gpu_matmul(pkg, g4lib, torch_gpu, DeviceWeight(pkg, torch_gpu, hw), xq, xs)
    assert np.array_equal(y, ok.matmul(xq, xs, hw.record, n))


def test_matmul_prefill_config_bitexact(pkg, g4lib, torch_gpu, ok):
    """The prefill GEMM workload: X [512 x 1536] N(0,1), W [6144 x 1536]."""
    g = rng(2026)
    w, s = random_weight(g, 6144, 1536)
    hw = HostWeight(pkg, w, s)
    xq, xs = ok.quantize(g.standard_normal((512, 1536)).astype(np.float32))
    y = gpu_matmul(pkg, g4lib, torch_gpu, DeviceWeight(pkg, torch_gpu, hw), xq, xs)
    assert np.array_equal(y, ok.matmul(xq, xs, hw.record, 6144))


@pytest.fixture
def order(pkg, g4lib, request):
    """Run a test under one summation order and restore the default after."""
    previous = g4lib.g4_set_order(request.param)
    yield request.param
    g4lib.g4_set_order(previous)


def gpu_rmsnorm(pkg, lib, torch, x, w, width):
    xd = dev(torch, x)
    wd = dev(torch, w) if w is not None else None
    pkg.check(lib.g4_rmsnorm(None, xd.data_ptr(), xd.data_ptr(), wd.data_ptr() if wd is not None else None,
                             width, 1e-6, x.size // width))
    torch.cuda.synchronize()
    return host(xd)


@pytest.mark.parametrize("order", [0], indirect=True)
def test_rmsnorm_reference_order_bitexact(pkg, g4lib, torch_gpu, ok, order):
    """The reference's sequential fp32 sum of squares, bit for bit."""
    g = rng(43)
    for width, rows, weighted in ((1536, 33, True), (256, 280, True), (512, 9, False), (2048, 3, True)):
        x = (g.standard_normal((rows, width)) * 4).astype(np.float32)
        w = g.uniform(0.5, 1.5, width).astype(np.float32)
        out = gpu_rmsnorm(pkg, g4lib, torch_gpu, x, w if weighted else None, width)
        ref = ok.rmsnorm(x, HostF32(pkg, w).record if weighted else None, width, 1e-6)
        assert np.array_equal(out, ref), width


@pytest.mark.parametrize("order", [0], indirect=True)
def test_rmsnorm_reference_order_adversarial(pkg, g4lib, torch_gpu, ok, order):
    """Rows that stress the exact parallel evaluation of the sequential sum of
    squares: many exact half-ulp ties (1 + k 2^-12 squared), leading and
    scattered zeros, magnitudes spread over 2^-60 .. 2^60, tiny values,
    all-equal rows, a single nonzero at the end -- bit for bit."""
    g = rng(47)
    w = 1536
    rows = [
        (1.0 + g.integers(0, 4, w) * 2.0 ** -12).astype(np.float32),
        (1.0 + g.integers(0, 64, w) * 2.0 ** -12).astype(np.float32),
        np.where(g.random(w) < 0.9, 0.0, g.standard_normal(w)).astype(np.float32),
        np.concatenate([np.zeros(700), g.standard_normal(w - 700)]).astype(np.float32),
        (g.standard_normal(w) * np.exp2(g.uniform(-60, 60, w))).astype(np.float32),
        (g.standard_normal(w) * 1e-20).astype(np.float32),
        np.full(w, 3.0, np.float32),
        np.concatenate([np.zeros(w - 1), [5.0]]).astype(np.float32),
        np.exp2(np.arange(w) % 40 - 20).astype(np.float32),
        np.exp2(-(np.arange(w) % 40)).astype(np.float32),
    ]
    x = np.stack(rows)
    wt = g.uniform(0.5, 1.5, w).astype(np.float32)
    out = gpu_rmsnorm(pkg, g4lib, torch_gpu, x, wt, w)
    ref = ok.rmsnorm(x, HostF32(pkg, wt).record, w, 1e-6)
    for i in range(len(rows)):
        assert np.array_equal(out[i], ref[i]), i


def test_rmsnorm_golden(pkg, g4lib, torch_gpu):
    gold = load_golden("ops.npz")
    out = gpu_rmsnorm(pkg, g4lib, torch_gpu, gold["rms_x"], gold["rms_w"], 1536)
    assert np.array_equal(out, gold["rms_out"])
    assert np.array_equal(gpu_rmsnorm(pkg, g4lib, torch_gpu, gold["rms_xh"], None, 256), gold["rms_outh"])


@pytest.mark.parametrize("order", [1], indirect=True)
def test_rmsnorm_parallel_order(pkg, g4lib, torch_gpu, ok, order):
    """Tree-ordered sums: close to the exact value, within 1e-5 of the reference."""
    g = rng(44)
    for width, rows, weighted in ((1536, 33, True), (256, 280, True), (512, 9, False)):
        x = (g.standard_normal((rows, width)) * 4).astype(np.float32)
        w = g.uniform(0.5, 1.5, width).astype(np.float32)
        out = gpu_rmsnorm(pkg, g4lib, torch_gpu, x, w if weighted else None, width)
        ref = ok.rmsnorm(x, HostF32(pkg, w).record if weighted else None, width, 1e-6)
        x64 = x.astype(np.float64)
        exact = (w if weighted else 1.0) * x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6)
        assert np.abs(out - exact).max() <= 2e-6 * np.abs(exact).max()
        assert np.allclose(out, ref, rtol=1e-5, atol=1e-6)


def test_softmax_bitexact(pkg, g4lib, torch_gpu, ok):
    """gemma4.c:400-408 with the host libm's expf: random rows, rising rows
    (a new maximum at every step), ties, huge ranges that underflow."""
    torch = torch_gpu
    g = rng(45)
    rows = [
        (g.standard_normal(1000) * 16).astype(np.float32),
        np.linspace(-50, 50, 777).astype(np.float32),
        np.linspace(50, -50, 130).astype(np.float32),
        np.full(300, 3.25, np.float32),
        (g.standard_normal(4096) * 200).astype(np.float32),
        np.array([0.0], np.float32),
        (g.uniform(-1e-3, 1e-3, 65)).astype(np.float32),
        # long rows (a block per row, in chunks of 16384 values): three chunks,
        # a new maximum at every one of 5000 steps, a long falling row
        (g.standard_normal(40000) * 8).astype(np.float32),
        np.linspace(-30, 30, 5000).astype(np.float32),
        np.linspace(30, -30, 20000).astype(np.float32),
        np.full(1500, -2.0, np.float32),
    ]
    for v in rows:
        d = dev(torch, v)
        pkg.check(g4lib.g4_softmax(None, d.data_ptr(), v.size, 1))
        torch.cuda.synchronize()
        assert np.array_equal(host(d), ok.softmax(v)), v.size
    # many rows at once, arguments spread over the whole negative range
    block = (g.standard_normal((64, 2048)) * g.uniform(0.1, 300, (64, 1))).astype(np.float32)
    d = dev(torch, block)
    pkg.check(g4lib.g4_softmax(None, d.data_ptr(), 2048, 64))
    torch.cuda.synchronize()
    out = host(d)
    for r in range(64):
        assert np.array_equal(out[r], ok.softmax(block[r])), r


def test_softmax_golden(pkg, g4lib, torch_gpu):
    gold = load_golden("ops.npz")
    d = dev(torch_gpu, gold["att_scores"])
    pkg.check(g4lib.g4_softmax(None, d.data_ptr(), gold["att_scores"].size, 1))
    torch_gpu.cuda.synchronize()
    assert np.array_equal(host(d), gold["att_p"])


def test_elementwise_golden_bitexact(pkg, g4lib, torch_gpu):
    gold = load_golden("ops.npz")
    torch = torch_gpu
    # rope, both table widths
    for name, hd in (("rope_s", 256), ("rope_g", 512)):
        v = dev(torch, gold[f"{name}_v"])
        c, s = dev(torch, gold[f"{name}_cos"]), dev(torch, gold[f"{name}_sin"])
        pkg.check(g4lib.g4_apply_rope(None, c.data_ptr(), s.data_ptr(), gold[f"{name}_cos"].shape[1],
                                      v.data_ptr(), 2, hd, 5, 3))
        torch.cuda.synchronize()
        assert np.array_equal(host(v), gold[f"{name}_out"]), name
    # geglu
    gate, up, table = gold["geglu_gate"], gold["geglu_up"], gold["geglu_table"]
    gd, ud, td = dev(torch, gate), dev(torch, up), dev(torch, table)
    pkg.check(g4lib.g4_geglu(None, gd.data_ptr(), ud.data_ptr(), gate.shape[0], gate.shape[1], up.shape[1],
                             td.data_ptr(), 4096, -8.0, 8.0))
    torch.cuda.synchronize()
    assert np.array_equal(host(gd), gold["geglu_out"])
    # embedding
    hw = HostWeight(pkg, gold["emb_w"], gold["emb_ws"])
    dw = DeviceWeight(pkg, torch, hw)
    toks = dev(torch, gold["emb_tokens"])
    out = torch.empty(gold["emb_out"].shape, dtype=torch.float32, device="cuda")
    pkg.check(g4lib.g4_embedding(None, out.data_ptr(), dw.record, toks.data_ptr(), toks.numel(),
                                 float(np.sqrt(np.float32(1536)))))
    torch.cuda.synchronize()
    assert np.array_equal(host(out), gold["emb_out"])
    # add_and_scale
    a, b = dev(torch, gold["add_a"]), dev(torch, gold["add_b"])
    pkg.check(g4lib.g4_add_and_scale(None, a.data_ptr(), b.data_ptr(), a.numel(), 0.7071067))
    torch.cuda.synchronize()
    assert np.array_equal(host(a), gold["add_out"])


def test_geglu_table_edges_bitexact(pkg, g4lib, torch_gpu, image, ok):
    """The GELU table's boundaries (gemma4.c:319-327): at and around lower and
    upper, the top interpolation cell (x just below upper, whose position can
    round to the last entry), +-inf, signed zeros and tiny values."""
    torch = torch_gpu
    below_upper = np.nextafter(np.float32(8.0), np.float32(0.0))
    edges = np.array([-8.0, np.nextafter(np.float32(-8.0), np.float32(0.0)),
                      np.nextafter(np.float32(-8.0), np.float32(-9.0)), 8.0, below_upper,
                      np.nextafter(below_upper, np.float32(0.0)), 7.9999, 7.998, -7.998,
                      0.0, -0.0, 1e-30, -1e-30, np.inf, -np.inf, 100.0, -100.0, 3.0e38], np.float32)
    gate = np.tile(edges, (3, 1))
    up = np.random.default_rng(5).standard_normal(gate.shape).astype(np.float32)
    width = gate.shape[1]
    table = image.array(pkg.GELU_TABLE)
    gd, ud, td = dev(torch, gate), dev(torch, up), dev(torch, table)
    pkg.check(g4lib.g4_geglu(None, gd.data_ptr(), ud.data_ptr(), 3, width, width, td.data_ptr(), 4096, -8.0, 8.0))
    torch.cuda.synchronize()
    want = ok.geglu(gate, up, width, image.records[pkg.GELU_TABLE])
    # where x + 8 rounds to 16 the position is the last entry and the fraction
    # 0: the reference reads one float past the table and multiplies it by 0,
    # which gives table[4095] for a finite neighbour (the oracle reads whatever
    # follows its copy of the table, so that case is stated directly)
    with np.errstate(over="ignore", invalid="ignore"):  # 3e38 and inf overflow: outside anyway
        position = (gate - np.float32(-8.0)) * np.float32(4095.0 / 16.0)
    last = (gate < np.float32(8.0)) & (gate > np.float32(-8.0)) & (position >= np.float32(4095.0))
    assert last.any()  # the case is exercised
    want = np.where(last, np.float32(table[4095]) * up, want).astype(np.float32)
    got = host(gd)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (edges, got[0], want[0])


def test_model_tables_bitexact(pkg, g4lib, torch_gpu, image, ok):
    """geglu with the image's GELU table; embeddings and RoPE from the image."""
    torch = torch_gpu
    g = rng(47)
    gate = (g.standard_normal((7, 12288)) * 3).astype(np.float32)
    up = g.standard_normal((7, 12288)).astype(np.float32)
    table = image.array(pkg.GELU_TABLE)
    gd, ud, td = dev(torch, gate), dev(torch, up), dev(torch, table)
    pkg.check(g4lib.g4_geglu(None, gd.data_ptr(), ud.data_ptr(), 7, 12288, 12288, td.data_ptr(), 4096, -8.0, 8.0))
    torch.cuda.synchronize()
    assert np.array_equal(host(gd), ok.geglu(gate, up, 12288, image.records[pkg.GELU_TABLE]))
    cos = image.array(pkg.layer_record(4, "rope_cos"))
    sin = image.array(pkg.layer_record(4, "rope_sin"))
    v = g.standard_normal((5, 8, 512)).astype(np.float32)
    vd = dev(torch, v)
    cd, sd = dev(torch, cos[:200000 // 2]), dev(torch, sin[:200000 // 2])
    pkg.check(g4lib.g4_apply_rope(None, cd.data_ptr(), sd.data_ptr(), 64, vd.data_ptr(), 8, 512, 99990, 5))
    torch.cuda.synchronize()
    ref = ok.rope(image.records[pkg.layer_record(4, "rope_cos")], image.records[pkg.layer_record(4, "rope_sin")],
                  v, 8, 512, 99990)
    assert np.array_equal(host(vd), ref)


ATTN_CASES = [
    # head_dim, ring, full, start_pos, n
    (256, 1024, 0, 0, 8),
    (256, 1024, 0, 1500, 1),      # window wraps the ring
    (256, 1024, 0, 600, 300),     # a prefill chunk straddling the window edge
    (512, 4096, 1, 0, 16),
    (512, 4096, 1, 3000, 1),
    (512, 4096, 1, 1000, 64),
    # token counts that leave a partial last block of 4 (taken first)
    (256, 1024, 0, 0, 5),
    (256, 1024, 0, 700, 301),
    (512, 4096, 1, 37, 13),
    # decode (one to four tokens)
    (512, 4096, 1, 63, 1),        # the row ends on a tile edge
    (512, 4096, 1, 4, 3),         # under one tile, three tokens
    (512, 4096, 1, 4095, 1),      # every cache row; prefetches run past the end of the cache
    (256, 1024, 0, 100, 2),       # sliding window before it fills
    (256, 1024, 0, 1019, 4),      # four tokens whose windows wrap the ring
    # long context: the depth of the 16K decode benchmark and beyond
    (512, 16384, 1, 16383, 1),    # every row of a 16K ring
    (512, 32768, 1, 16380, 4),    # four decode tokens crossing 16K in a grown ring
    (512, 32768, 1, 16000, 64),   # a prefill chunk at 16K keys
    (256, 1024, 0, 16380, 4),     # the sliding window deep in a sequence
    (512, 65536, 1, 40000, 1),    # more key blocks than one pass of the score grid
]


def run_attention(pkg, lib, torch, oracle_lib, hd, ring, full, start, n):
    g = rng(hd + start + n)
    kc = g.standard_normal((ring, hd)).astype(np.float32)
    vc = g.standard_normal((ring, hd)).astype(np.float32)
    q = (g.standard_normal((n, 8, hd)) * 0.25).astype(np.float32)
    ref = np.empty_like(q)
    oracle_lib.oracle().orc_attend(ref.ctypes.data, q.ctypes.data, kc.ctypes.data, vc.ctypes.data,
                                   ring, hd, 8, full, start, n)
    out = torch.empty(q.shape, dtype=torch.float32, device="cuda")
    kd, vd, qd = dev(torch, kc), dev(torch, vc), dev(torch, q)
    pkg.check(lib.g4_attend(None, out.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                            ring, hd, 8, full, start, n))
    torch.cuda.synchronize()
    return host(out), ref


@pytest.mark.parametrize("order", [0], indirect=True)
@pytest.mark.parametrize("hd,ring,full,start,n", ATTN_CASES)
def test_attention_reference_order_bitexact(pkg, g4lib, torch_gpu, oracle_lib, order, hd, ring, full, start, n):
    o, ref = run_attention(pkg, g4lib, torch_gpu, oracle_lib, hd, ring, full, start, n)
    assert np.array_equal(o, ref)


def exact_attention(hd, ring, full, start, n):
    """gemma4.c:443-456 in float64 on run_attention's inputs (same seed)."""
    g = rng(hd + start + n)
    kc = g.standard_normal((ring, hd)).astype(np.float32).astype(np.float64)
    vc = g.standard_normal((ring, hd)).astype(np.float32).astype(np.float64)
    q = (g.standard_normal((n, 8, hd)) * 0.25).astype(np.float32).astype(np.float64)
    out = np.empty((n, 8, hd))
    for t in range(n):
        pos = start + t
        rows = np.arange(0 if full else max(0, pos - 511), pos + 1) & (ring - 1)
        s = kc[rows] @ q[t].T  # keys x heads
        p = np.exp(s - s.max(axis=0))
        out[t] = (p / p.sum(axis=0)).T @ vc[rows]
    return out


@pytest.mark.parametrize("order", [1], indirect=True)
@pytest.mark.parametrize("hd,ring,full,start,n", ATTN_CASES)
def test_attention_parallel_order(pkg, g4lib, torch_gpu, oracle_lib, order, hd, ring, full, start, n):
    """Split-KV flash decoding: within 2e-5 of the output scale of the exact
    (float64) attention, and of the oracle within 2e-5 plus the oracle's own
    recursive-summation bound, (keys - 1) * 2^-24 relative: its sequential
    fp32 softmax sum (gemma4.c:400-408) absorbs terms below half an ulp of the
    running sum, which over 16K keys moves it by ~1e-5 (measured)."""
    o, ref = run_attention(pkg, g4lib, torch_gpu, oracle_lib, hd, ring, full, start, n)
    exact = exact_attention(hd, ring, full, start, n)
    scale = np.abs(exact).max()
    assert np.abs(o - exact).max() <= 2e-5 * scale, float(np.abs(o - exact).max() / scale)
    keys = start + n if full else min(start + n, 512)
    bound = 2e-5 + (keys - 1) * 2.0 ** -24
    assert np.abs(o - ref).max() <= bound * scale, float(np.abs(o - ref).max() / scale)


# --- the sampler (gemma4.c:527-561) -------------------------------------------

def gpu_sample(pkg, lib, torch, row: np.ndarray, temp: float, state: int) -> tuple[int, int]:
    import ctypes

    d = dev(torch, row)
    st = ctypes.c_uint64(state)
    tok = ctypes.c_int(-1)
    pkg.check(lib.g4_sample_logits(None, d.data_ptr(), row.size, float(temp), ctypes.byref(st),
                                   ctypes.byref(tok)))
    return tok.value, st.value


def orc_sample(oracle_lib, row: np.ndarray, temp: float, state: int) -> tuple[int, int]:
    import ctypes

    st = ctypes.c_uint64(state)
    tok = oracle_lib.oracle().orc_sample(row.ctypes.data, row.size, float(temp), ctypes.byref(st))
    return int(tok), st.value


def test_sample_golden(pkg, g4lib, torch_gpu):
    """The reference's own sample() outputs (tests/golden/sample.npz): the
    token and the generator state after each of several consecutive draws."""
    d = load_golden("sample.npz")
    for r in range(d["rows"].shape[0]):
        row = np.ascontiguousarray(d["rows"][r])
        for t, temp in enumerate(d["temps"]):
            for s0, start in enumerate(d["states"]):
                state = int(start)
                for k in range(d["tokens"].shape[3]):
                    tok, after = gpu_sample(pkg, g4lib, torch_gpu, row, float(temp), state)
                    if temp > 0:
                        state = after
                    assert tok == d["tokens"][r, t, s0, k], (r, float(temp), s0, k)
                    assert state == int(d["states_after"][r, t, s0, k]), (r, float(temp), s0, k)


def test_sample_full_vocab(pkg, g4lib, torch_gpu, oracle_lib):
    """Model-sized rows against the oracle: soft-capped logits with ties
    planted at the 64th place, a row with a NaN (the reference's insertion
    loop then decides), and a row that is -inf outside 70 entries."""
    g = rng(77)
    rows = []
    for _ in range(3):
        row = (30.0 * np.tanh(g.standard_normal(pkg.VOCAB) * 8.0 / 30.0)).astype(np.float32)
        row[g.choice(pkg.VOCAB, 12, replace=False)] = np.sort(row)[::-1][63]
        rows.append(row)
    nan_row = rows[0].copy()
    nan_row[g.integers(0, pkg.VOCAB)] = np.nan
    rows.append(nan_row)
    sparse = np.full(pkg.VOCAB, -np.inf, np.float32)
    sparse[g.choice(pkg.VOCAB, 70, replace=False)] = g.standard_normal(70).astype(np.float32)
    rows.append(sparse)
    for i, row in enumerate(rows):
        for temp in (0.0, 0.5, 1.0, 1.7):
            state = int(g.integers(1, 2**63))
            for _ in range(3):
                want = orc_sample(oracle_lib, row, temp, state)
                got = gpu_sample(pkg, g4lib, torch_gpu, row, temp, state)
                if temp > 0:
                    assert got == want, (i, temp)
                    state = want[1]
                else:
                    assert got[0] == want[0], (i, temp)
