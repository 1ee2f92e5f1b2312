"""The exact-sum engine's algorithm (exact_sum_events in
gemma4.c_amd/csrc/g4_reference_order.hip), restated in numpy and checked
against the plain sequential fp32 loop it replaces: the rmsnorm sum of squares
(gemma4.c:366-368) and the softmax running sum with its new-maximum step
(gemma4.c:400-408).

The model follows the kernel pass for pass: lane-major terms (thread T holds
terms J T .. J T + J - 1), a predicted prefix whose binade marks events
(binade change, tie, new maximum, out-of-range value), integer run sums
saturating at 2^29, at most 63 events per pass, the chain computed before the
checks, and the two ways a run can fail (predicted binade wrong; run leaves
its binade early).  The prediction has the kernel's structure: each thread's
start comes from its own J-term map composed over lanes and waves by scans,
and the thread then runs its J steps from that start, so the start and the
previous thread's end are two evaluations of one prefix in different orders.
A thread's first step takes the binade of the previous thread's end (lane
l - 1's; for a wave's lane 0, its start's unless that lies within 2^-12 of a
power of two, then an event), as the kernel does.  The GPU kernels are held
to the oracle bit for bit by the GPU tests; this test pins the method itself
on inputs chosen to hit every branch (ties, zeros, huge dynamic range,
overflow to inf, many events per pass, sums that pass a power of two an ulp
at a time) and shows that the first-step rule is needed."""

import numpy as np

f32 = np.float32
CAP = 1 << 29
EVENTS = 63


def biased_exponent(x):
    return (np.asarray(x, np.float32).view(np.uint32).astype(np.int64) >> 23) & 0xFF


def plain(s, t, special):
    return f32(f32(s * t) + f32(1)) if special else f32(s + t)


def sequential(t, spec, s=0.0):
    s = f32(s)
    for k in range(len(t)):
        s = plain(s, t[k], spec[k])
    return s


def fma32(a, b, c):
    """fp32 a * b + c (the product exact in float64, then one rounding to
    float64 and one to float32: a prediction, so a rare double rounding does
    not matter)."""
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(np.float32)


def predict(t, spec, s, k0, J, rule, softmax):
    """A_prev, A_cur per term (the prediction before and after each step),
    the binade each thread's first step is taken on and its start's."""
    n = len(t)
    nt = -(-n // J)
    tt = np.concatenate([t, np.zeros(nt * J - n, np.float32)])
    sp = np.concatenate([spec, np.zeros(nt * J - n, bool)])
    act = np.arange(nt * J) >= k0
    idx = np.arange(nt) * J
    # each thread's map x -> la x + lb over its J terms
    la, lb = np.ones(nt, np.float32), np.zeros(nt, np.float32)
    for j in range(J):
        i = idx + j
        a = np.where(act[i] & sp[i], tt[i], f32(1)).astype(np.float32)
        b = np.where(act[i], np.where(sp[i], f32(1), tt[i]), f32(0)).astype(np.float32)
        lb = fma32(lb, a, b)
        la = (la * a).astype(np.float32)
    # inclusive scan over the 64 lanes of each wave (Hillis-Steele), then the
    # waves' maps in order: the start of each thread
    nw = -(-nt // 64)
    A = np.ones(nw * 64, np.float32)
    B = np.zeros(nw * 64, np.float32)
    A[:nt], B[:nt] = la, lb
    A, B = A.reshape(nw, 64), B.reshape(nw, 64)
    for sh in (1, 2, 4, 8, 16, 32):
        pa = np.concatenate([np.ones((nw, sh), np.float32), A[:, :-sh]], axis=1)
        pb = np.concatenate([np.zeros((nw, sh), np.float32), B[:, :-sh]], axis=1)
        B = fma32(pb, A, B)
        A = (pa * A).astype(np.float32)
    x = np.empty(nw, np.float32)
    xv = f32(s)
    for w in range(nw):
        x[w] = xv
        xv = fma32(xv, A[w, 63], B[w, 63])
    ex_a = np.concatenate([np.ones((nw, 1), np.float32), A[:, :-1]], axis=1).reshape(-1)[:nt]
    ex_b = np.concatenate([np.zeros((nw, 1), np.float32), B[:, :-1]], axis=1).reshape(-1)[:nt]
    c = fma32(np.repeat(x, 64)[:nt], ex_a, ex_b)
    # each thread's J steps from its start
    A_prev = np.empty(nt * J, np.float32)
    A_cur = np.empty(nt * J, np.float32)
    a = c.copy()
    for j in range(J):
        i = idx + j
        A_prev[i] = a
        nxt = np.where(sp[i], fma32(a, tt[i], 1), (a + tt[i]).astype(np.float32))
        a = np.where(act[i], nxt, a).astype(np.float32)
        A_cur[i] = a
    e_first = biased_exponent(c)
    if rule == "thread":
        end = biased_exponent(a)  # each thread's predicted end
        lane0 = (np.arange(nt) % 64) == 0
        e_first = np.where(lane0, e_first, np.concatenate([[0], end[:-1]]))
        m = c.view(np.uint32) & 0x7FFFFF
        near = ((m < (1 << 11)) & ~(softmax & (biased_exponent(c) == 127))) | (m >= (1 << 23) - (1 << 12))
        e_first = np.where(lane0 & (np.arange(nt) > 0) & (idx > k0) & near, -1, e_first)
    return A_prev[:n], A_cur[:n], e_first, biased_exponent(c)


def one_pass(t, spec, s, k0, J=8, rule="thread", softmax=False):
    """Returns (s, k0, done), as esum_pass does.  rule "thread": a thread's
    first step takes the binade the previous thread's prediction ends in;
    "start": its own start's (the rule without the thread boundary).
    softmax: the engine's new-maximum mode (s >= 1 throughout)."""
    n = len(t)
    k = np.arange(n)
    act = k >= k0
    # 1. predicted prefix
    A_prev, A_cur, e_first, e_start = predict(t, spec, s, k0, J, rule, softmax)
    ep, ec = biased_exponent(A_prev), biased_exponent(A_cur)
    with np.errstate(over="ignore", invalid="ignore"):
        T = np.minimum(np.ldexp(t.astype(np.float32), (150 - ep).astype(np.int32)).astype(np.float32),
                       f32(1 << 24))
    R = np.rint(T)
    ev = act & (spec | (ep != ec) | ((ep - 27) > 200) | ((ep - 27) < 0) | (np.abs(T - R) == 0.5)
                | ~(t <= f32(3.40282347e38)))
    # a thread's first step on another grid than the run's: an event
    first = k[k % J == 0]
    ev[first] |= act[first] & (e_first[first // J] != e_start[first // J])
    # 3. run sums (segmented at events, saturating)
    P = np.zeros(n, np.int64)
    run = 0
    for i in range(n):
        run = 0 if ev[i] else min(run + (int(R[i]) if act[i] else 0), CAP)
        P[i] = run
    events = np.nonzero(ev)[0]
    more = len(events) > EVENTS
    events = events[:EVENTS]
    # entries: (d before the event, k, term, special, predicted exponent after)
    entries = [(int(P[e - 1]) if e > 0 else 0, int(e), t[e], bool(spec[e]), int(ec[e])) for e in events]
    if not more:
        entries.append((int(P[n - 1]), n, f32(0), False, 0))
    starts, e_runs = [], []
    for i, (d, kk, te, sp, e_after) in enumerate(entries):
        starts.append(k0 if i == 0 else entries[i - 1][1] + 1)
        e_runs.append(int(biased_exponent(f32(s))) if i == 0 else entries[i - 1][4])
    # 5. the chain, then the checks
    sv = f32(s)
    at_start, at_end = [], []
    for i, (d, kk, te, sp, _) in enumerate(entries):
        nonempty = kk > starts[i]
        du = f32(np.ldexp(f32(d), e_runs[i] - 150)) if nonempty else f32(0)
        at_start.append(sv)
        sv = f32(sv + du)
        at_end.append(sv)
        fa, fb = (te, f32(1)) if sp else (f32(1), te)
        sv = f32(f32(sv * fa) + fb)
    bad = [i for i, (d, kk, te, sp, _) in enumerate(entries)
           if kk > starts[i] and (biased_exponent(at_start[i]) != e_runs[i]
                                  or not 27 <= biased_exponent(at_start[i]) <= 227
                                  or biased_exponent(at_end[i]) != e_runs[i])]
    if not bad:
        if more:
            return sv, entries[-1][1] + 1, False
        return sv, n, True
    i = bad[0]
    sb, st, kend = at_start[i], starts[i], entries[i][1]
    eb = int(biased_exponent(sb))
    if eb != e_runs[i] or not 27 <= eb <= 227:
        return sb, st, False
    S = int(np.ldexp(sb, 150 - eb))
    for kk in range(st, kend):
        if S + P[kk] >= 1 << 24:
            before = int(P[kk - 1]) if kk > st else 0
            return f32(f32(np.ldexp(f32(S + before), eb - 150)) + t[kk]), kk + 1, False
    raise AssertionError("a run that fails its end check has a crossing step")


def exact_sum(t, spec, s=0.0, stats=None, J=8, rule="thread", softmax=False):
    t = np.asarray(t, np.float32)
    spec = np.asarray(spec, bool)
    s, k0 = f32(s), 0
    passes = 0
    while True:
        passes += 1
        s2, k1, done = one_pass(t, spec, s, k0, J, rule, softmax)
        assert done or k1 > k0, "a pass that neither finishes nor moves forward"
        s, k0 = s2, k1
        if done:
            break
    if stats is not None:
        stats.append(passes)
    return s


def same(a, b):
    return (np.isnan(a) and np.isnan(b)) or a == b


def softmax_terms(x):
    """Terms and new-maximum flags of the reference's running sum (v_0 is the
    starting maximum, a zero term here)."""
    m = x[0]
    t = np.zeros(len(x), np.float32)
    spec = np.zeros(len(x), bool)
    for i in range(1, len(x)):
        if x[i] > m:
            spec[i] = True
            t[i] = np.exp(f32(m - x[i]))
            m = x[i]
        else:
            t[i] = np.exp(f32(x[i] - m))
    return t, spec


def test_sum_of_squares_rows():
    g = np.random.default_rng(11)
    for trial in range(24):
        x = (g.standard_normal(1536) * f32(10.0 ** g.uniform(-8, 8))).astype(np.float32)
        if trial % 3 == 0:
            x[g.integers(0, 1536, 5)] *= 1000
        if trial % 4 == 1:
            x[:40] *= f32(1e-6)
        t = f32(x * x)
        assert same(exact_sum(t, np.zeros(1536, bool)), sequential(t, np.zeros(1536, bool))), trial


def test_adversarial_sums():
    g = np.random.default_rng(12)
    n = 1536
    cases = [
        np.where(np.arange(n) % 3 == 0, f32(0.5), f32(1.0)).astype(np.float32),  # ties
        (2.0 ** g.integers(-10, 10, n)).astype(np.float32),                       # powers of two
        np.zeros(n, np.float32),                                                  # all zero
        (g.integers(0, 8, n) * 0.25 + 2 ** 20).astype(np.float32),                 # ties at a large sum
        (g.integers(1, 1 << 12, n) * 2.0 ** g.integers(-30, 30)).astype(np.float32),
        np.full(n, f32(3e38)),                                                    # overflow to inf
        np.concatenate([np.full(8, f32(1e-30)), np.ones(n - 8, np.float32)]),
    ]
    z = np.zeros(n, np.float32)
    z[g.integers(0, n, 10)] = 3
    cases.append(z)
    stats = []
    for i, t in enumerate(cases):
        spec = np.zeros(n, bool)
        assert same(exact_sum(t, spec, stats=stats), sequential(t, spec)), i
    assert max(stats) > 1  # some case needs more than one pass


def test_softmax_running_sums():
    g = np.random.default_rng(13)
    for trial in range(18):
        n = 512 * (1 + trial % 3)
        x = (g.standard_normal(n) * g.uniform(0.1, 20)).astype(np.float32)
        if trial % 3 == 0:
            x = np.sort(x)  # a new maximum at every step: hundreds of events
        t, spec = softmax_terms(x)
        assert same(exact_sum(t, spec, 1.0, softmax=True), sequential(t, spec, 1.0)), trial


def test_planted_mistake_is_caught():
    """A wrong run rule (ties not treated as events: R = rint(t / u) rounds
    half to even on t alone, not on the sum) must break exactness, so the
    comparisons above are not vacuous.  From s = 2^24 (grid u = 2) a term 2
    makes s / u odd and the term 1 after it is an exact half of the grid."""
    t = np.where(np.arange(1000) % 2 == 0, f32(2.0), f32(1.0)).astype(np.float32)
    spec = np.zeros(1000, bool)
    start = f32(2.0 ** 24)
    exact = sequential(t, spec, start)
    assert same(exact_sum(t, spec, start), exact)
    s = start
    for x in t:
        e = int(biased_exponent(s))
        if 27 <= e <= 227 and biased_exponent(f32(s + x)) == e:
            u = 2.0 ** (e - 150)
            s = f32(s + f32(np.rint(x / u) * u))
        else:
            s = f32(s + x)
    assert s != exact


def crawl(g, n, boundary, cross, lo, hi, start=0.0):
    """Terms whose sequential sum (from `start`) is brought to boundary - m u
    by its first term and then gains R = rint(r) ulps a term (r uniform in
    [lo, hi], u the ulp below boundary), passing boundary near term `cross`."""
    u = boundary * 2.0 ** -24
    R = round((lo + hi) / 2)
    t = (g.uniform(lo, hi, n) * u).astype(np.float32)
    t[0] = f32(boundary - R * (cross - 1) * u - start)
    return t


def crawl_rows(seed, n, count):
    g = np.random.default_rng(seed)
    rows = []
    for i in range(count):
        boundary = (2.0, 4.0, 1024.0, 2.0 ** -10)[i % 4]
        lo, hi = ((2.05, 2.45), (1.55, 2.45), (0.55, 0.95))[(i // 4) % 3]
        rows.append(crawl(g, n, boundary, int(g.integers(n // 10, n * 9 // 10)), lo, hi))
    return rows


def test_sums_crawling_past_a_power_of_two():
    """Sums of squares and softmax sums that pass a power of two a few ulps a
    term (each term rounds to R ulps below it and to another count above it),
    over the block shapes of the kernels (4 waves x 6 and x 8 terms a thread,
    8 x 3 and 6 x 4 (the one-token products' row tails), 16 x 4 and x 8,
    8 x 1)."""
    for J, n in ((6, 1536), (3, 1536), (4, 1536), (8, 2048), (4, 4096), (8, 8192), (1, 512)):
        for i, t in enumerate(crawl_rows(100 + J, n, 12)):
            spec = np.zeros(n, bool)
            assert same(exact_sum(t, spec, J=J), sequential(t, spec)), (J, n, i)
    g = np.random.default_rng(15)
    for J, n in ((8, 2048), (8, 8192), (1, 512)):
        for i in range(9):
            boundary = (2.0, 4.0, 8.0)[i % 3]
            lo, hi = ((2.05, 2.45), (1.55, 2.45), (0.55, 0.95))[(i // 3) % 3]
            t = crawl(g, n, boundary, int(g.integers(n // 10, n * 9 // 10)), lo, hi, start=1.0)
            spec = np.zeros(n, bool)
            assert same(exact_sum(t, spec, 1.0, J=J, softmax=True), sequential(t, spec, 1.0)), (J, n, i)


def test_first_step_rule_is_needed():
    """Without the thread-boundary rule (each thread's first step on the grid
    of its own start's binade) the same crawling sums come out wrong: a run
    then mixes two grids where the scanned start of a thread and the end of
    the previous thread's prediction lie on two sides of a power of two."""
    wrong = 0
    for J, n in ((6, 1536), (8, 2048), (4, 4096)):
        for t in crawl_rows(100 + J, n, 12):
            spec = np.zeros(n, bool)
            wrong += not same(exact_sum(t, spec, J=J, rule="start"), sequential(t, spec))
    assert wrong > 0
