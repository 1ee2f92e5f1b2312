"""Pins the oracle (oracle/oracle.c, the CPU restatement of gemma4.c:178-522):

1. against the golden vectors written by the reference's own compiled
   gemma4.c (tests/golden/*.npz), bit for bit -- this holds anywhere;
2. against the compiled reference itself (oracle/_ref) on fresh inputs,
   bit for bit -- where the reference checkout exists;
3. against closed forms computed independently in float64 (integer dot
   products, the GELU and rotation formulas, a float64 softmax), so a dropped
   term, wrong index or transposed operand fails even if both 1 and 2 were
   wrong the same way.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import HostF32, HostWeight, load_golden

from conftest import random_weight, rng


@pytest.fixture(scope="module")
def gold():
    return load_golden("ops.npz")


@pytest.fixture(scope="module", params=["fast", "scalar"])
def ok(request, oracle_lib):
    """Oracle kernels with the VNNI matmul on and off."""
    lib = oracle_lib.oracle()
    lib.orc_set_fast(1 if request.param == "fast" else 0)
    yield oracle_lib.Kernels()
    lib.orc_set_fast(1)


def _ref_or_skip(oracle_lib):
    if not oracle_lib.ref_available():
        pytest.skip("reference library not built here")
    return oracle_lib.Kernels(use_ref=True)


# --- 1. golden vectors ------------------------------------------------------

def test_golden_quantize(ok, gold):
    q, s = ok.quantize(gold["quant_x"])
    assert np.array_equal(q, gold["quant_q"]) and np.array_equal(s, gold["quant_s"])


def test_golden_matmul(pkg, ok, gold):
    for name in ("mm_a", "mm_b"):
        hw = HostWeight(pkg, gold[f"{name}_w"], gold[f"{name}_ws"])
        y = ok.matmul(gold[f"{name}_xq"], gold[f"{name}_xs"], hw.record, hw.n)
        assert np.array_equal(y, gold[f"{name}_y"]), name


def test_golden_attention_primitives(ok, gold):
    ring = gold["att_k"].shape[0]
    hd = gold["att_q"].size
    first, num = int(gold["att_first"]), int(gold["att_num"])
    sc = ok.scores(gold["att_q"], gold["att_k"], first, num, ring - 1, hd)
    assert np.array_equal(sc, gold["att_scores"])
    p = ok.softmax(sc)
    assert np.array_equal(p, gold["att_p"])
    o = ok.value_sum(p, gold["att_v"], first, num, ring - 1, hd)
    assert np.array_equal(o, gold["att_o"])


def test_golden_elementwise(pkg, ok, gold):
    tab = HostF32(pkg, gold["geglu_table"], shape=(4096, -8, 8))
    assert np.array_equal(ok.geglu(gold["geglu_gate"], gold["geglu_up"], 320, tab.record), gold["geglu_out"])
    hw = HostWeight(pkg, gold["emb_w"], gold["emb_ws"])
    emb = ok.embedding(hw.record, gold["emb_tokens"], float(np.sqrt(np.float32(1536))))
    assert np.array_equal(emb, gold["emb_out"])
    rw = ok.rmsnorm(gold["rms_x"], HostF32(pkg, gold["rms_w"]).record, 1536, 1e-6)
    assert np.array_equal(rw, gold["rms_out"])
    assert np.array_equal(ok.rmsnorm(gold["rms_xh"], None, 256, 1e-6), gold["rms_outh"])
    assert np.array_equal(ok.add_and_scale(gold["add_a"], gold["add_b"], 0.7071067), gold["add_out"])
    for name, hd in (("rope_s", 256), ("rope_g", 512)):
        r = ok.rope(HostF32(pkg, gold[f"{name}_cos"]).record, HostF32(pkg, gold[f"{name}_sin"]).record,
                    gold[f"{name}_v"], 2, hd, 5)
        assert np.array_equal(r, gold[f"{name}_out"]), name


# --- 2. the compiled reference on fresh inputs --------------------------------

@pytest.mark.parametrize("n,k,rows", [(16, 64, 1), (256, 1536, 3), (96, 2048, 8), (64, 12288, 13), (6144, 1536, 17)])
def test_reference_matmul(pkg, ok, oracle_lib, n, k, rows):
    ref = _ref_or_skip(oracle_lib)
    g = rng(n * 7 + k + rows)
    w, s = random_weight(g, n, k)
    hw = HostWeight(pkg, w, s)
    xq, xs = ref.quantize(g.standard_normal((rows, k)).astype(np.float32))
    assert np.array_equal(ok.matmul(xq, xs, hw.record, n), ref.matmul(xq, xs, hw.record, n))


def test_reference_kernels_fresh(pkg, ok, oracle_lib):
    ref = _ref_or_skip(oracle_lib)
    g = rng(5)
    x = (g.standard_normal((33, 2048)) * g.uniform(0.01, 100, (33, 1))).astype(np.float32)
    q1, s1 = ok.quantize(x)
    q2, s2 = ref.quantize(x)
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)
    for hd in (256, 512):
        ring = 1024
        kc = g.standard_normal((ring, hd)).astype(np.float32)
        qv = g.standard_normal(hd).astype(np.float32)
        a = ok.scores(qv, kc, 900, 400, ring - 1, hd)
        assert np.array_equal(a, ref.scores(qv, kc, 900, 400, ring - 1, hd))
        assert np.array_equal(ok.softmax(a * 3), ref.softmax(a * 3))
        vc = g.standard_normal((ring, hd)).astype(np.float32)
        p = ref.softmax(a)
        assert np.array_equal(ok.value_sum(p, vc, 900, 400, ring - 1, hd),
                              ref.value_sum(p, vc, 900, 400, ring - 1, hd))
    w = g.uniform(0.5, 1.5, 512).astype(np.float32)
    xr = g.standard_normal((9, 512)).astype(np.float32)
    assert np.array_equal(ok.rmsnorm(xr, HostF32(pkg, w).record, 512, 1e-6),
                          ref.rmsnorm(xr, HostF32(pkg, w).record, 512, 1e-6))


def test_reference_model_tables(pkg, image, ok, oracle_lib):
    """Kernels that read the image's own tables (GELU, RoPE, embeddings)."""
    ref = _ref_or_skip(oracle_lib)
    g = rng(11)
    gate = (g.standard_normal((5, 6144)) * 3).astype(np.float32)
    up = g.standard_normal((5, 6144)).astype(np.float32)
    t = image.records[pkg.GELU_TABLE]
    assert np.array_equal(ok.geglu(gate, up, 6144, t), ref.geglu(gate, up, 6144, t))
    toks = g.integers(0, 262144, 7).astype(np.int32)
    e = image.records[pkg.EMBED_PER_LAYER]
    assert np.array_equal(ok.embedding(e, toks, 16.0), ref.embedding(e, toks, 16.0))
    c, s = image.records[pkg.layer_record(4, "rope_cos")], image.records[pkg.layer_record(4, "rope_sin")]
    v = g.standard_normal((3, 8, 512)).astype(np.float32)
    assert np.array_equal(ok.rope(c, s, v, 8, 512, 77777), ref.rope(c, s, v, 8, 512, 77777))


# --- 3. closed forms ------------------------------------------------------------

def test_quantize_invariants(ok):
    g = rng(3)
    x = (g.standard_normal((4, 640)) * 5).astype(np.float32)
    x[1, 64:128] = 0
    q, s = ok.quantize(x)
    grp = x.reshape(4, 10, 64)
    qg = q.reshape(4, 10, 64).astype(np.int32)
    assert s[1, 1] == 0 and not qg[1, 1].any()  # zero group -> scale 0, q 0
    amax = np.abs(grp).max(axis=2)
    nz = amax > 0
    assert np.array_equal(np.abs(qg).max(axis=2)[nz], np.full(nz.sum(), 127))  # the max maps to +-127
    assert np.allclose(s, amax / 127, rtol=1e-7)
    err = np.abs(qg * s[:, :, None].astype(np.float64) - grp)
    assert (err <= s[:, :, None] * 0.5001 + 1e-30).all()  # round to nearest


def test_matmul_integer_closed_form(pkg, ok):
    """Y = sum_g ws[n,g] xs[m,g] sum_{k in g} xq[m,k] w[n,k], brute force in
    exact integers then float64 (no packing, no fold order)."""
    g = rng(17)
    n, k, rows = 32, 512, 3
    w, s = random_weight(g, n, k)
    hw = HostWeight(pkg, w, s)
    xq, xs = ok.quantize(g.standard_normal((rows, k)).astype(np.float32))
    y = ok.matmul(xq, xs, hw.record, n)
    dots = np.einsum("mgk,ngk->mng", xq.reshape(rows, k // 64, 64).astype(np.int64),
                     w.reshape(n, k // 64, 64).astype(np.int64))
    expect = (dots * xs[:, None, :].astype(np.float64) * s[None, :, :].astype(np.float64)).sum(axis=2)
    assert np.allclose(y, expect, rtol=2e-6, atol=1e-6 * np.abs(expect).max())


def test_attention_closed_form(ok):
    g = rng(19)
    hd, ring = 512, 1024
    kc = g.standard_normal((ring, hd)).astype(np.float32)
    vc = g.standard_normal((ring, hd)).astype(np.float32)
    qv = (g.standard_normal(hd) * 0.1).astype(np.float32)
    first, num = 1000, 50  # wraps past the ring end
    rows = (first + np.arange(num)) & (ring - 1)
    sc = ok.scores(qv, kc, first, num, ring - 1, hd)
    exact = kc[rows].astype(np.float64) @ qv.astype(np.float64)
    assert np.allclose(sc, exact, rtol=1e-5, atol=1e-5)
    p = ok.softmax(sc)
    e = np.exp(sc.astype(np.float64) - sc.max())
    assert np.allclose(p, e / e.sum(), rtol=1e-5)
    o = ok.value_sum(p, vc, first, num, ring - 1, hd)
    assert np.allclose(o, p.astype(np.float64) @ vc[rows].astype(np.float64), rtol=1e-4, atol=1e-5)


def test_elementwise_closed_forms(pkg, ok):
    g = rng(23)
    # rmsnorm: w * x / sqrt(mean(x^2) + eps)
    x = g.standard_normal((3, 1536)).astype(np.float32)
    w = g.uniform(0.5, 1.5, 1536).astype(np.float32)
    y = ok.rmsnorm(x, HostF32(pkg, w).record, 1536, 1e-6)
    x64 = x.astype(np.float64)
    assert np.allclose(y, w * x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6), rtol=1e-5)
    # rope: rotation of (x_j, x_{j+hd/2}) by the table angle, untouched beyond pairs
    ang = g.uniform(-3, 3, (8, 64))
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    v = g.standard_normal((2, 1, 512)).astype(np.float32)
    r = ok.rope(HostF32(pkg, c).record, HostF32(pkg, s).record, v, 1, 512, 3)
    a, b = v[:, 0, :64].astype(np.float64), v[:, 0, 256:320].astype(np.float64)
    cc, ss = c[3:5].astype(np.float64), s[3:5].astype(np.float64)
    assert np.allclose(r[:, 0, :64], a * cc - b * ss, atol=1e-6)
    assert np.allclose(r[:, 0, 256:320], b * cc + a * ss, atol=1e-6)
    assert np.array_equal(r[:, 0, 64:256], v[:, 0, 64:256])
    # geglu: tanh-GELU(x) * up within the table's interpolation error
    table = (lambda t: (0.5 * t * (1 + np.tanh(0.7978845608 * (t + 0.044715 * t ** 3)))).astype(np.float32))(
        np.linspace(-8, 8, 4096, dtype=np.float32))
    tab = HostF32(pkg, table, shape=(4096, -8, 8))
    gate = np.concatenate([g.uniform(-9, 9, 1000), [-8.0, 8.0, 20.0, -20.0]]).astype(np.float32)[None]
    up = g.uniform(-2, 2, gate.shape).astype(np.float32)
    out = ok.geglu(gate, up, gate.shape[1], tab.record)
    t = gate.astype(np.float64)
    gelu = 0.5 * t * (1 + np.tanh(0.7978845608 * (t + 0.044715 * t ** 3)))
    gelu = np.where(t <= -8, table[0], np.where(t >= 8, t, gelu))
    assert np.allclose(out, gelu * up, atol=2e-4)


def test_sliding_equals_global_inside_window(oracle_lib):
    """While every query sees all keys (positions < 512), sliding and full
    attention agree exactly (gemma4.c:448)."""
    lib = oracle_lib.oracle()
    g = rng(29)
    hd, heads, n = 256, 8, 40
    kc = g.standard_normal((1024, hd)).astype(np.float32)
    vc = g.standard_normal((1024, hd)).astype(np.float32)
    q = g.standard_normal((n, heads, hd)).astype(np.float32)
    outs = []
    for full in (0, 1):
        o = np.empty_like(q)
        lib.orc_attend(o.ctypes.data, q.ctypes.data, kc.ctypes.data, vc.ctypes.data, 1024, hd, heads, full, 300, n)
        outs.append(o)
    assert np.array_equal(outs[0], outs[1])


# --- the whole step -------------------------------------------------------------

def test_oracle_model_matches_golden(image, oracle_lib):
    """forward()/logits() of the oracle reproduce the reference's logits rows
    bit for bit (SHA-256 of all 262144 floats) and its greedy tokens."""
    from helpers import load_golden
    import hashlib
    gold = load_golden("model.npz")
    m = oracle_lib.Model(image)
    m.forward(gold["tokens"], 0)
    for r in (0, 7):
        lg = m.logits(r)
        assert hashlib.sha256(lg.tobytes()).digest() == bytes(gold[f"row{r}_sha"]), r
    lg = m.logits(7)
    pos = gold["tokens"].size
    for step, tok in enumerate(gold["decode_tokens"]):
        assert int(np.argmax(lg)) == int(tok)
        m.forward(np.array([tok], np.int32), pos)
        pos += 1
        lg = m.logits(0)
        assert hashlib.sha256(lg.tobytes()).digest() == bytes(gold["decode_sha"][step])
    m.close()


def test_oracle_matches_reference_beyond_the_window(image, oracle_lib):
    """forward()/logits() of the oracle and of the compiled reference over
    1100 tokens (the sliding rings wrap at 1024, the window clamp of
    gemma4.c:448 is active from position 512, global layers attend past 512)
    and 3 greedy decode steps: every compared logits row identical bit for bit
    (SHA-256 of all 262144 floats)."""
    import hashlib
    if not oracle_lib.ref_available():
        pytest.skip("reference library not built here")
    tokens = rng(59).integers(0, 262144, 1100).astype(np.int32)
    models = [oracle_lib.Model(image), oracle_lib.Model(image, use_ref=True)]
    digests = [[], []]
    for i, m in enumerate(models):
        for pos in range(0, tokens.size, 512):
            m.forward(tokens[pos:pos + 512], pos)
        row = (tokens.size - 1) % 512
        for r in (0, 37, row):
            digests[i].append(hashlib.sha256(m.logits(r).tobytes()).hexdigest())
        pos = tokens.size
        for _ in range(3):
            lg = m.logits(row)
            m.forward(np.array([int(np.argmax(lg))], np.int32), pos)
            pos += 1
            row = 0
            digests[i].append(hashlib.sha256(m.logits(0).tobytes()).hexdigest())
        m.close()
    assert digests[0] == digests[1]


@pytest.mark.parametrize("full,ring,pos", [
    (0, 1024, 510), (0, 1024, 511), (0, 1024, 512), (0, 1024, 1023), (0, 1024, 1024),
    (0, 1024, 1535), (0, 1024, 16380), (1, 8192, 700), (1, 8192, 5000)])
def test_window_and_ring_brute_force(oracle_lib, full, ring, pos):
    """Attention of one query at `pos` against a brute-force float64
    restatement of gemma4.c:443-456: sliding layers see exactly the 512
    positions max(0, pos - 511) .. pos (gemma4.c:448), global layers 0 .. pos,
    and position p lives in ring row p & (ring - 1).  One key too many or too
    few moves the output by ~2% of its scale, far above the tolerance."""
    lib = oracle_lib.oracle()
    g = rng(pos + ring)
    hd, heads = 256, 2
    kc = g.standard_normal((ring, hd)).astype(np.float32)
    vc = g.standard_normal((ring, hd)).astype(np.float32)
    # small queries: near-uniform weights, so every key counts (~2% of the
    # output's scale for one key more or less, or a ring row off by one)
    q = (g.standard_normal((1, heads, hd)) * 0.02).astype(np.float32)
    out = np.empty_like(q)
    lib.orc_attend(out.ctypes.data, q.ctypes.data, kc.ctypes.data, vc.ctypes.data, ring, hd, heads,
                   full, pos, 1)
    first = 0 if full else max(0, pos - 511)
    rows = np.arange(first, pos + 1) & (ring - 1)
    k64, v64 = kc[rows].astype(np.float64), vc[rows].astype(np.float64)
    for h in range(heads):
        s = k64 @ q[0, h].astype(np.float64)
        p = np.exp(s - s.max())
        want = (p / p.sum()) @ v64
        assert np.abs(out[0, h] - want).max() <= 2e-5 * np.abs(want).max(), (h, pos)


def test_oracle_thread_count_independent(image, oracle_lib):
    lib = oracle_lib.oracle()
    toks = np.array([5, 6, 7], np.int32)
    rows = []
    for threads in (1, 5):
        lib.orc_set_threads(threads)
        m = oracle_lib.Model(image)
        m.forward(toks, 0)
        rows.append(m.logits(2))
        m.close()
    lib.orc_set_threads(0)
    assert np.array_equal(rows[0], rows[1])


# --- the sampler (gemma4.c:527-561) -------------------------------------------

def _orc_sample(oracle_lib, row: np.ndarray, temp: float, state: int) -> tuple[int, int]:
    import ctypes

    st = ctypes.c_uint64(state)
    tok = oracle_lib.oracle().orc_sample(row.ctypes.data, row.size, float(temp), ctypes.byref(st))
    return int(tok), int(st.value)


def test_sample_golden(oracle_lib):
    """orc_sample against the reference's own sample() (tests/golden/sample.npz):
    tokens and generator states over consecutive draws."""
    d = load_golden("sample.npz")
    rows, temps, states = d["rows"], d["temps"], d["states"]
    for r in range(rows.shape[0]):
        row = np.ascontiguousarray(rows[r])
        for t, temp in enumerate(temps):
            for s0, start in enumerate(states):
                state = int(start)
                for k in range(d["tokens"].shape[3]):
                    tok, state = _orc_sample(oracle_lib, row, float(temp), state)
                    assert tok == d["tokens"][r, t, s0, k], (r, t, s0, k)
                    assert state == int(d["states_after"][r, t, s0, k]), (r, t, s0, k)


def test_sample_reference_full_vocab(oracle_lib):
    """orc_sample against the compiled reference at the model's vocabulary,
    soft-capped logits with ties planted at the 64th place."""
    import ctypes

    if not oracle_lib.ref_available():
        pytest.skip("reference library not built here")
    lib = oracle_lib.ref()
    state = ctypes.c_ulonglong.in_dll(lib, "rng_state")
    g = np.random.default_rng(5)
    for case in range(3):
        row = (30.0 * np.tanh(g.standard_normal(262144) * 8.0 / 30.0)).astype(np.float32)
        top = np.sort(row)[::-1]
        row[g.choice(262144, 12, replace=False)] = top[63]  # equal to the 64th
        for temp in (0.0, 0.7, 1.0):
            s = int(g.integers(1, 2**63))
            state.value = s
            want = lib.sample(row.ctypes.data, row.size, temp)
            tok, after = _orc_sample(oracle_lib, row, temp, s)
            assert tok == want and after == state.value, (case, temp)


def _uniform(state: int) -> tuple[float, int]:
    """xorshift64* as published (Vigna): shifts 12, 25, 27, multiplier
    0x2545F4914F6CDD1D; the top 24 bits of the product over 2^24."""
    m = (1 << 64) - 1
    x = state
    x ^= x >> 12
    x = (x ^ (x << 25)) & m
    x ^= x >> 27
    return ((x * 0x2545F4914F6CDD1D) & m) >> 40, x


def test_sample_closed_forms(oracle_lib):
    """Cases whose answer follows from the definition alone: temperature 0
    is the first maximum; one logit 40 above the rest is always drawn; a row
    whose 64 highest are equal has p = 1/64 each (weights exactly 1), a 95%
    prefix of ceil(0.95 * 64) = 61 entries, and draws entry ceil(x) - 1 of
    the 64 lowest-indexed maxima, x = u * 61 in float32 (x = 0: the first),
    for the generator's next u."""
    g = np.random.default_rng(9)
    row = g.standard_normal(5000).astype(np.float32)
    row[[77, 3000]] = 9.0
    assert _orc_sample(oracle_lib, row, 0.0, 1)[0] == 77
    row[1234] = 49.0
    assert all(_orc_sample(oracle_lib, row, 1.0, s)[0] == 1234 for s in (1, 42, 2**40 + 7))
    flat = np.full(5000, -3.0, np.float32)
    idx = np.sort(g.choice(5000, 90, replace=False))
    flat[idx] = 2.5  # 90 equal maxima: the list holds the 64 with the lowest indices
    state = 42
    for _ in range(20):
        top24, nxt = _uniform(state)
        x = float(np.float32(np.float32(top24) / np.float32(16777216.0)) * np.float32(61.0))
        want = idx[max(0, min(60, int(np.ceil(x)) - 1))]
        tok, state = _orc_sample(oracle_lib, flat, 1.0, state)
        assert state == nxt
        assert tok == want, (tok, want)


# (layer, start_pos, n): a sliding layer's first chunk and a later chunk over a
# wrapped ring, a global layer, and two shared layers (layers 15..34 read the
# caches of owners 13 and 14 without writing, gemma4.c:419-421, 432) in
# decode and a ragged batch
ATTENTION_LAYER_CASES = [(0, 0, 512), (3, 1536, 512), (4, 512, 64), (16, 700, 1), (19, 2000, 3)]


def attention_layer_inputs(layer: int, start_pos: int, n: int):
    """The hidden rows and the owner's prior cache rows of one case (N(0,1)):
    rows start_pos - 1023 .. start_pos - 1 of a sliding ring, 0 .. start_pos - 1
    of a global one."""
    owner = layer if layer < 15 else (14 if layer % 5 == 4 else 13)
    full = owner % 5 == 4
    g = rng(1000 * layer + start_pos + n)
    hidden = g.standard_normal((n, 1536)).astype(np.float32)
    rows = start_pos if full else min(start_pos, 1024)
    keys = g.standard_normal((rows, 512 if full else 256)).astype(np.float32)
    values = g.standard_normal(keys.shape).astype(np.float32)
    slots = np.arange(start_pos - rows, start_pos) & ((131072 if full else 1024) - 1)
    return owner, hidden, slots, keys, values


@pytest.mark.parametrize("layer,start_pos,n", ATTENTION_LAYER_CASES)
def test_oracle_attention_layer_matches_reference(image, oracle_lib, layer, start_pos, n):
    """orc_attention_layer against the compiled reference's own attention()
    (gemma4.c:411-461) on the same hidden rows and prior cache: the output rows
    and the whole cache owner identical bit for bit."""
    if not oracle_lib.ref_available():
        pytest.skip("reference library not built here")
    owner, hidden, slots, keys, values = attention_layer_inputs(layer, start_pos, n)
    out = []
    for use_ref in (False, True):
        m = oracle_lib.Model(image, use_ref=use_ref)
        kc, vc = m.cache(owner)
        kc[slots], vc[slots] = keys, values
        m.hidden(n)[:] = hidden
        m.attention_layer(layer, start_pos, n)
        used = max(start_pos + n, 1024) if owner % 5 == 4 else 1024
        out.append((m.hidden(n).copy(), kc[:used].copy(), vc[:used].copy()))
        m.close()
    for a, b in zip(*out):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # the layer did its work: new output rows, and the new cache rows written
    assert np.all(np.isfinite(out[0][0])) and not np.array_equal(out[0][0], hidden)
    if layer < 15:
        new = np.arange(start_pos, start_pos + n) & (out[0][1].shape[0] - 1)
        assert np.all(np.abs(out[0][1][new]).sum(axis=1) > 0)
