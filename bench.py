"""Benchmark of the MI355X W8A8 forward path on the synthetic Gemma-4-E2B model.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--order reference|parallel]

Prints one JSON line.  A step is one 512-token prefill (g4_forward over 512
uniform-random token ids at position 0) followed by the logits of its last row,
the unit gemma4.c's --bench prefill times (gemma4.c:627-634); `value` is
prefill tokens per second over K such steps, with the model already resident
in HBM.  Also reported: prefill of 8192 tokens in 512-token chunks, 128 greedy
decode steps at 16384 tokens of context (forward + logits each, gemma4.c:636-643),
the int8-MFMA roofline of the prefill GEMM (X[512x1536] x W[6144x1536]) and the
HBM roofline of the decode GEMV sweep (every E2B linear shape at one token,
weighted by bytes), each timed with HIP events on the stream they run on, and
the oracle (the CPU restatement of the same path) timed on this host's cores.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

MODEL_SEED = 20261201
HBM_PEAK_GBS = 8000.0           # MI355X HBM3E
INT8_MFMA_PEAK_TOPS = 5000.0    # MI355X dense int8 MFMA

# (N, K, count per decoded token) for every linear of a Gemma-4-E2B step.
GEMV_SWEEP = [
    (2048, 1536, 28), (4096, 1536, 7), (256, 1536, 24), (512, 1536, 6),
    (1536, 2048, 28), (1536, 4096, 7), (6144, 1536, 30), (1536, 6144, 15),
    (12288, 1536, 40), (1536, 12288, 20), (256, 1536, 35), (1536, 256, 35),
    (8960, 1536, 1), (262144, 1536, 1),
]


# Algorithmic HBM bytes of one decode step at 16384 positions of context: the
# weights of every product (int8 + fp16 scales), the keys and values each of
# the 7 global layers reads (16384 rows of 512 floats each), and those each of
# the 28 window layers reads (512 rows of 256 floats each).
DECODE16K_STEP_BYTES = (sum(count * (n * k + n * k // 32) for n, k, count in GEMV_SWEEP)
                        + 7 * 16384 * 512 * 2 * 4 + 28 * 512 * 256 * 2 * 4)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gemv_bytes(n: int, k: int) -> int:
    """Algorithmic bytes of one W8A8 product at one token: int8 weights, fp16
    scales per 64, int8 activations + fp32 scales per 64, fp32 outputs."""
    return n * k + n * k // 32 + k + k // 16 + 4 * n


def pmc_traffic(name: str):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary
    (FETCH_SIZE and WRITE_SIZE passes scaled by a copy-kernel calibration,
    written by the commands listed in the file), or None if it is absent."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("hbm_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def random_weight(torch, n: int, k: int, gen):
    """int8 U[-127, 127] packed weights, fp16 scales log-uniform in [1e-3, 1e-2]."""
    w = torch.randint(-127, 128, (n * k,), dtype=torch.int8, device="cuda", generator=gen)
    u = torch.rand((n * k // 64,), device="cuda", generator=gen)
    s = torch.exp(math.log(1e-3) + u * (math.log(1e-2) - math.log(1e-3)))
    return w, s.to(torch.float16)


def graph_timed(torch, fn, count: int, replays: int, warmup: int = 20) -> float:
    """Average milliseconds per launch: `count` launches (fn(0) .. fn(count-1),
    each on torch's current stream) captured once as a HIP graph, replayed
    `warmup` times untimed (clocks and caches reach their steady state), then
    `replays` times between HIP events on the replay stream.  The host's launch
    rate drops out; what remains is each kernel's duration plus the device's
    gap between dependent kernels."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(count):
            fn(i)
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    stop.record()
    stop.synchronize()
    ms = start.elapsed_time(stop) / (replays * count)
    del graph
    return ms


def gemm_roofline(pkg, lib, torch) -> dict:
    """The prefill GEMM: X [512 x 1536] N(0,1) quantized per 64, W [6144 x 1536]
    U[-127,127] with log-uniform fp16 scales; 2*512*6144*1536 int8 ops."""
    gen = torch.Generator(device="cuda").manual_seed(1)
    m, n, k = 512, 6144, 1536
    x = torch.randn((m, k), device="cuda", generator=gen)
    xq = torch.empty((m, k), dtype=torch.int8, device="cuda")
    xs = torch.empty((m, k // 64), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    pkg.check(lib.g4_quantize(stream, xq.data_ptr(), xs.data_ptr(), x.data_ptr(), m, k))
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ops = 2.0 * m * n * k
    moved = n * k + n * k // 32 + m * k + m * k // 16 + 4 * m * n

    def timed(copies: int) -> float:
        ws = [random_weight(torch, n, k, gen) for _ in range(copies)]
        recs = []
        for w, s in ws:
            rec = pkg.Tensor()
            rec.data, rec.scales = w.data_ptr(), s.data_ptr()
            rec.shape[0], rec.shape[1] = n, k
            recs.append(rec)

        def launch(i):
            pkg.check(lib.g4_matmul_int8(torch.cuda.current_stream().cuda_stream, out.data_ptr(),
                                         xq.data_ptr(), xs.data_ptr(), recs[i % copies], m))

        ms = graph_timed(torch, launch, max(32, 4 * copies), 10)
        del ws, recs
        torch.cuda.empty_cache()
        return ms

    # 8 x 9.7 MB of weights (the headline): repeats are not served from one L2
    # alone; 1 copy: warm (cache-resident); 40 copies (388 MB): cold, beyond
    # the 256 MB Infinity Cache
    ms = timed(8)
    warm, cold = timed(1), timed(40)
    tops = ops / (ms * 1e-3) / 1e12
    return {"kernel": "k_gemm", "ms_per_launch": ms, "tops": tops, "bytes": moved, "ops": ops,
            "warm_ms": warm, "cold_ms": cold}


def vendor_int8_gemm(torch, m: int = 512, n: int = 6144, k: int = 1536) -> dict:
    """The vendor library's plain int8 GEMM on the same shape (hipBLASLt through
    torch._int_mm: int32 output, no scales, no fold), timed the same way: a
    reference point for what a 512-row GEMM reaches on this chip."""
    copies = 8
    try:
        gen = torch.Generator(device="cuda").manual_seed(3)
        a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device="cuda", generator=gen)
        bs = [torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda", generator=gen)
              for _ in range(copies)]

        def launch(i):
            torch._int_mm(a, bs[i % copies].t())

        ms = graph_timed(torch, launch, 4 * copies, 10)
    except Exception as ex:  # the comparison is optional
        return {"error": str(ex)[:160]}
    tops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    return {"library": "hipBLASLt via torch._int_mm (int32 out, no scales)", "us": round(ms * 1e3, 2),
            "tops": round(tops, 1), "frac": round(tops / INT8_MFMA_PEAK_TOPS, 4)}


def probe(pkg, lib, torch, what: str, launches: int = 20) -> None:
    """Launch one kernel alone, for hardware-counter runs under rocprofv3 --pmc:
    `gemm` = the prefill GEMM above, `gemv` = the lm_head GEMV (262144 x 1536,
    one token), `kv` = one global layer's decode attention at 16384 keys
    (scores, softmax, P.V), `copy` = a 256 MiB device-to-device copy (the
    calibration kernel: it reads and writes exactly 268,435,456 bytes)."""
    gen = torch.Generator(device="cuda").manual_seed(4)
    stream = torch.cuda.current_stream().cuda_stream
    if what == "kv":
        q, out, caches = kv_inputs(torch, 6)
        for i in range(launches):
            attend_global(pkg, lib, stream, q, out, caches[i % 6])
        torch.cuda.synchronize()
        return
    if what == "copy":
        a = torch.empty(64 << 20, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(launches):
            b.copy_(a)
        torch.cuda.synchronize()
        return
    m, n, k = (512, 6144, 1536) if what == "gemm" else (1, 262144, 1536)
    x = torch.randn((m, k), device="cuda", generator=gen)
    xq = torch.empty((m, k), dtype=torch.int8, device="cuda")
    xs = torch.empty((m, k // 64), dtype=torch.float32, device="cuda")
    pkg.check(lib.g4_quantize(stream, xq.data_ptr(), xs.data_ptr(), x.data_ptr(), m, k))
    copies = 8 if what == "gemm" else 2
    ws = [random_weight(torch, n, k, gen) for _ in range(copies)]
    recs = []
    for w, s in ws:
        rec = pkg.Tensor()
        rec.data, rec.scales = w.data_ptr(), s.data_ptr()
        rec.shape[0], rec.shape[1] = n, k
        recs.append(rec)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    for i in range(launches):
        pkg.check(lib.g4_matmul_int8(stream, out.data_ptr(), xq.data_ptr(), xs.data_ptr(), recs[i % copies], m))
    torch.cuda.synchronize()


def gemv_sweep(pkg, lib, torch) -> dict:
    """Every decode GEMV shape at one token, rotated over >= 512 MB of weight
    copies per shape so repeats come from HBM, not the 256 MB Infinity Cache."""
    gen = torch.Generator(device="cuda").manual_seed(2)
    stream = torch.cuda.current_stream().cuda_stream
    per_shape = {}
    total_bytes = total_time = 0.0
    for n, k, count in GEMV_SWEEP:
        key = f"{n}x{k}"
        if key in per_shape:
            rec = per_shape[key]
        else:
            copies = max(2, (512 << 20) // (n * k))
            pool_w = torch.randint(-127, 128, (copies, n * k), dtype=torch.int8, device="cuda", generator=gen)
            pool_s = (torch.rand((copies, n * k // 64), device="cuda", generator=gen) * 9e-3 + 1e-3).to(torch.float16)
            x = torch.randn((1, k), device="cuda", generator=gen)
            xq = torch.empty((1, k), dtype=torch.int8, device="cuda")
            xs = torch.empty((1, k // 64), dtype=torch.float32, device="cuda")
            pkg.check(lib.g4_quantize(stream, xq.data_ptr(), xs.data_ptr(), x.data_ptr(), 1, k))
            out = torch.empty((1, n), dtype=torch.float32, device="cuda")
            recs = []
            for c in range(copies):
                r = pkg.Tensor()
                r.data, r.scales = pool_w[c].data_ptr(), pool_s[c].data_ptr()
                r.shape[0], r.shape[1] = n, k
                recs.append(r)

            def launch(i, recs=recs, out=out, xq=xq, xs=xs):
                pkg.check(lib.g4_matmul_int8(torch.cuda.current_stream().cuda_stream, out.data_ptr(),
                                             xq.data_ptr(), xs.data_ptr(), recs[i % len(recs)], 1))

            captured = min(copies, 256)  # one pass over >= 512 MB of copies (or 256 launches)
            ms = graph_timed(torch, launch, captured, max(2, 1024 // captured))
            b = gemv_bytes(n, k)
            rec = {"ms": ms, "gbs": b / (ms * 1e-3) / 1e9, "bytes": b}
            per_shape[key] = rec
            del pool_w, pool_s
            torch.cuda.empty_cache()
        total_bytes += count * rec["bytes"]
        total_time += count * rec["ms"]
    return {
        "byte_weighted_gbs": total_bytes / (total_time * 1e-3) / 1e9,
        "bytes_per_token": total_bytes,
        "gemv_ms_per_token": total_time,
        "per_shape": {k: round(v["gbs"], 1) for k, v in per_shape.items()},
        "per_shape_us": {k: round(v["ms"] * 1e3, 2) for k, v in per_shape.items()},
    }


KV_KEYS, KV_HEAD_DIM, KV_HEADS = 16384, 512, 8  # a global layer's decode attention at 16K context


def kv_inputs(torch, copies: int):
    """Query rows and `copies` key/value caches of a global layer at 16384
    positions (N(0,1) rows, the scale of the model's normalized K/V rows)."""
    gen = torch.Generator(device="cuda").manual_seed(6)
    q = torch.randn((1, KV_HEADS * KV_HEAD_DIM), device="cuda", generator=gen) * 0.25
    out = torch.empty_like(q)
    caches = [torch.randn((2, KV_KEYS, KV_HEAD_DIM), device="cuda", generator=gen) for _ in range(copies)]
    return q, out, caches


def attend_global(pkg, lib, stream, q, out, cache) -> None:
    """gemma4.c:443-456 for one token at position 16383 of a global layer:
    scores over keys 0..16383, softmax, P.V (reference order, as in the model's
    decode step)."""
    pkg.check(lib.g4_attend(stream, out.data_ptr(), q.data_ptr(), cache[0].data_ptr(), cache[1].data_ptr(),
                            KV_KEYS, KV_HEAD_DIM, KV_HEADS, 1, KV_KEYS - 1, 1))


def profile_figures(name: str) -> dict:
    """`key: value` lines of a committed rocprofv3 summary under profiles/."""
    figures = {}
    try:
        with open(os.path.join(ROOT, "profiles", name)) as f:
            for line in f:
                key, sep, value = line.partition(":")
                if sep and key.strip().endswith("_us"):
                    try:
                        figures[key.strip()] = float(value.split()[0])
                    except (ValueError, IndexError):
                        pass
    except OSError:
        pass
    return figures


def kv_roofline(pkg, lib, torch) -> dict:
    """The KV-cache reads of one global layer's decode attention at 16384 keys
    (head_dim 512, 8 query heads on the one KV head): K and V, 33.5 MB each,
    read once per layer.  Six caches (403 MB) are rotated so that repeats come
    from HBM, not the 256 MB Infinity Cache; timed by graph replay like the
    GEMV sweep.  The split by kernel (scores read K, P.V reads V) comes from
    the committed kernel trace of `bench.py --probe kv`."""
    copies = 6
    q, out, caches = kv_inputs(torch, copies)

    def launch(i):
        attend_global(pkg, lib, torch.cuda.current_stream().cuda_stream, q, out, caches[i % copies])

    ms = graph_timed(torch, launch, 4 * copies, 10)
    kv_bytes = 2 * KV_KEYS * KV_HEAD_DIM * 4
    moved = kv_bytes + 2 * q.numel() * 4
    res = {"ms": ms, "bytes": moved, "gbs": moved / (ms * 1e-3) / 1e9}
    split = profile_figures("attend_global_16k_kernel_stats.txt")
    if {"scores_us", "values_us"} <= split.keys():
        half = kv_bytes / 2
        res["k_read_gbs_scores"] = half / (split["scores_us"] * 1e-6) / 1e9
        res["v_read_gbs_values"] = half / (split["values_us"] * 1e-6) / 1e9
        res["split_us"] = split
    del caches
    torch.cuda.empty_cache()
    return res


def decode_probe(pkg, lib, np, context: int = 16384, steps: int = 32) -> None:
    """Fill `context` positions in 512-token chunks, then `steps` decode steps
    (forward + logits each), as the decode figure of model_benchmarks."""
    rng = np.random.default_rng(3)
    out = np.empty(pkg.VOCAB, np.float32)
    tokens = rng.integers(0, pkg.VOCAB, context).astype(np.int32)
    for pos in range(0, context, 512):
        chunk = tokens[pos:pos + 512]
        pkg.check(lib.g4_forward(chunk.ctypes.data, chunk.size, pos))
    pkg.check(lib.g4_logits(0, out.ctypes.data))  # (waits for the fill)
    time.sleep(0.5)  # an idle gap that separates the decode steps in a trace
    token = np.array([2], np.int32)
    s = time.perf_counter()
    for i in range(steps):
        pkg.check(lib.g4_forward(token.ctypes.data, 1, context + i))
        pkg.check(lib.g4_logits(0, out.ctypes.data))
    log(f"decode @{context}: {steps / (time.perf_counter() - s):.1f} tok/s")


def prefill_8192_rate(prefill, rng, pkg, np) -> float:
    """8192 tokens in 512-token chunks + the last row's logits (gemma4.c:563-573
    with --bench 8192): 1 warmup + the mean of 3."""
    t8k = rng.integers(0, pkg.VOCAB, 8192).astype(np.int32)
    prefill(t8k)
    times = []
    for _ in range(3):
        s = time.perf_counter()
        prefill(t8k)
        times.append(time.perf_counter() - s)
    return 8192 / (sum(times) / len(times))


def decode_16k_rate(prefill, forward, logits, rng, pkg, np) -> float:
    """Decode at 16384 tokens of context (gemma4.c:636-643): fill, then 128 steps
    of forward + logits at positions 16384.., after one untimed step at 16384
    that captures the decode graph (the first timed step rewrites that
    position's K/V rows with the same values)."""
    t16k = rng.integers(0, pkg.VOCAB, 16384).astype(np.int32)
    prefill(t16k)
    token = np.array([2], np.int32)  # gemma4.c:637 decodes token 2
    forward(token, 16384)
    logits()
    s = time.perf_counter()
    for i in range(128):
        forward(token, 16384 + i)
        logits()
    return 128 / (time.perf_counter() - s)


def parallel_order_figures(pkg, lib, np) -> dict:
    """The other summation order (G4_ORDER_PARALLEL: tree sums, split-KV flash
    decoding) measured the same way in the same session, and how far it moves
    the logits: one 512-token prefill's last row in both orders."""
    rng = np.random.default_rng(5)
    out = np.empty(pkg.VOCAB, np.float32)
    rows = {}

    def forward(tokens, pos):
        pkg.check(lib.g4_forward(tokens.ctypes.data, tokens.size, pos))

    def prefill(tokens):
        for pos in range(0, tokens.size, 512):
            forward(tokens[pos:pos + 512], pos)
        pkg.check(lib.g4_logits((tokens.size - 1) % 512, out.ctypes.data))

    t512 = rng.integers(0, pkg.VOCAB, 512).astype(np.int32)
    for name, order in (("reference", pkg.ORDER_REFERENCE), ("parallel", pkg.ORDER_PARALLEL)):
        lib.g4_set_order(order)
        prefill(t512)
        rows[name] = out.copy()
    res = {
        "max_abs_logit_delta_vs_reference_order": float(np.abs(rows["reference"] - rows["parallel"]).max()),
        "argmax_agrees": bool(np.argmax(rows["reference"]) == np.argmax(rows["parallel"])),
    }
    try:
        res["prefill8192_tok_s"] = round(prefill_8192_rate(prefill, rng, pkg, np), 1)
        res["decode16k_tok_s"] = round(decode_16k_rate(prefill, forward,
                                                       lambda: pkg.check(lib.g4_logits(0, out.ctypes.data)),
                                                       rng, pkg, np), 2)
    finally:
        lib.g4_set_order(pkg.ORDER_REFERENCE)
    log(f"parallel order: {res}")
    return res


def model_benchmarks(pkg, lib, np, steps: int, warmup: int, prefill_only: bool = False) -> dict:
    rng = np.random.default_rng(3)
    out = np.empty(pkg.VOCAB, np.float32)

    def forward(tokens, pos):
        pkg.check(lib.g4_forward(tokens.ctypes.data, tokens.size, pos))

    def prefill(tokens):
        for pos in range(0, tokens.size, 512):
            forward(tokens[pos:pos + 512], pos)
        pkg.check(lib.g4_logits((tokens.size - 1) % 512, out.ctypes.data))

    # headline: K timed 512-token prefill steps
    t512 = rng.integers(0, pkg.VOCAB, 512).astype(np.int32)
    for _ in range(warmup):
        prefill(t512)
    start = time.perf_counter()
    for _ in range(steps):
        prefill(t512)
    elapsed = time.perf_counter() - start
    res = {"prefill512_s": elapsed, "prefill512_tok_s": 512 * steps / elapsed}
    log(f"prefill 512: {res['prefill512_tok_s']:.0f} tok/s ({elapsed / steps * 1e3:.2f} ms/step)")
    if prefill_only:
        return res

    res["prefill8192_tok_s"] = prefill_8192_rate(prefill, rng, pkg, np)
    log(f"prefill 8192: {res['prefill8192_tok_s']:.0f} tok/s")
    res["decode16k_tok_s"] = decode_16k_rate(prefill, forward, lambda: pkg.check(lib.g4_logits(0, out.ctypes.data)),
                                             rng, pkg, np)
    log(f"decode @16K: {res['decode16k_tok_s']:.1f} tok/s")

    # teacher-forced logit dump (gemma4.c:563-573 with dump on): 2388 ids in
    # 512-token chunks, every position's logits to host memory (one batched
    # lm_head per chunk)
    t_dump = rng.integers(0, pkg.VOCAB, 2388).astype(np.int32)
    dump = np.empty((512, pkg.VOCAB), np.float32)
    s = time.perf_counter()
    for pos in range(0, t_dump.size, 512):
        chunk = t_dump[pos:pos + 512]
        forward(chunk, pos)
        pkg.check(lib.g4_logits_all(dump.ctypes.data))
    res["dump2388_rows_s"] = t_dump.size / (time.perf_counter() - s)
    log(f"teacher-forced dump of 2388 positions: {res['dump2388_rows_s']:.0f} rows/s")
    return res


def cpu_baseline(pkg, image, np) -> dict:
    """gemma4.c's own forward()/logits() on this host's cores, on the same
    synthetic model: oracle/_ref/libgemma4ref.so, the reference's source built
    by oracle/Makefile for AVX-512 VNNI hosts (its VNNI matmul path).  Where
    that library is absent, the oracle (the CPU restatement, equal speed on
    the same cores) stands in, with kind "port".  Bounded samples of the
    reference's own measurements (gemma4.c:627-645), about a minute of CPU:
      - prefill 512 + logits of the last row: 1 discarded warmup + the mean of
        3 (the reference README's protocol), at the host's thread count (one
        per physical core, gemma4.c:182-188, or OMP_NUM_THREADS; at most 16)
        and at 8 threads (the README's published setup);
      - prefill 8192 in 512-token chunks + logits: one run after the warmups
        (about 16 s on 16 Zen 5 cores);
      - decode at 16384 positions of context: forward + logits per step, 1
        untimed and 16 timed steps, the rate from the median step, with KV
        rows 0..16383 filled with N(0,1) values in place of a 16384-token
        prefill (a synthetic-KV approximation: the step's work does not depend
        on the values; the rows the model writes are RMS-normalized, so of
        that scale)."""
    import ctypes

    import psutil

    from oracle import binding
    use_ref = binding.ref_available()
    lib = binding.ref() if use_ref else binding.oracle()
    threads = min(lib.ref_thread_count() if use_ref else lib.orc_threads(), 16)
    gomp = ctypes.CDLL(lib._name)  # omp_set_num_threads from the library's libgomp

    def set_threads(n: int) -> None:
        # the reference reads OMP_NUM_THREADS per call (gemma4.c:187): with it
        # set, the team size is omp_get_max_threads()
        os.environ["OMP_NUM_THREADS"] = str(n)
        gomp.omp_set_num_threads(n)
        if not use_ref:
            lib.orc_set_threads(n)

    model = binding.Model(image, use_ref=use_ref)
    rng = np.random.default_rng(3)
    t512 = rng.integers(0, pkg.VOCAB, 512).astype(np.int32)
    t8k = rng.integers(0, pkg.VOCAB, 8192).astype(np.int32)
    token = np.array([2], np.int32)  # gemma4.c:637

    def timed(fn) -> float:
        s = time.perf_counter()
        fn()
        return time.perf_counter() - s

    def prefill512_rate(n_threads: int) -> float:
        set_threads(n_threads)
        model.forward(t512, 0)
        model.logits(511)
        times = [timed(lambda: (model.forward(t512, 0), model.logits(511))) for _ in range(3)]
        return 512 / (sum(times) / len(times))

    def prefill(tokens) -> None:
        for pos in range(0, tokens.size, 512):
            model.forward(tokens[pos:pos + 512], pos)
        model.logits((tokens.size - 1) % 512)

    old_env = os.environ.get("OMP_NUM_THREADS")
    decode = None
    try:
        prefill8 = prefill512_rate(8)
        rate = prefill512_rate(threads)
        prefill8k = 8192 / timed(lambda: prefill(t8k))
        if use_ref:
            model.fill_kv_random(16384, seed=5)
            model.forward(token, 16384)
            model.logits(0)
            steps = [timed(lambda i=i: (model.forward(token, 16384 + i), model.logits(0))) for i in range(16)]
            decode = 1.0 / float(np.median(steps))
    finally:
        model.close()
        if old_env is None:
            os.environ.pop("OMP_NUM_THREADS", None)
        else:
            os.environ["OMP_NUM_THREADS"] = old_env
    nproc, physical = os.cpu_count(), psutil.cpu_count(logical=False)
    kind = "reference" if use_ref else "port"
    log(f"cpu {kind} ({threads} threads; nproc {nproc}, {physical} physical cores): prefill 512 "
        f"{rate:.1f} tok/s ({prefill8:.1f} at 8 threads); prefill 8192 {prefill8k:.1f} tok/s; "
        f"decode@16K {decode} tok/s")
    return {"value": rate, "unit": "tok/s", "cores": threads, "kind": kind,
            "sample": "gemma4.c forward()+logits() on the same synthetic model: 512-token prefill + "
                      "logits, 1 discarded warmup + mean of 3; prefill 8192 in 512-token chunks + logits, "
                      "1 run; decode at 16384 positions (synthetic KV: rows filled with N(0,1) in place "
                      "of the prefill), 1 untimed + 16 timed steps of forward + logits, median step",
            "prefill512_tok_s_8_threads": prefill8, "prefill8192_tok_s": prefill8k,
            "decode16k_tok_s": decode,
            "host": {"nproc": nproc, "physical_cores": physical, "threads": threads}}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--order", choices=["reference", "parallel"], default="reference")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--probe", choices=["gemm", "gemv", "kv", "copy", "prefill", "decode"],
                    help="only launch one kernel 20 times (for rocprofv3 --pmc runs), or run "
                         "3 + 10 prefill-512 steps of the model (prefill), or fill 16384 "
                         "positions and run 32 decode steps (decode); no JSON")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(this build runs the forward path on a single GPU)", file=sys.stderr)
        return 2

    import numpy as np
    import torch  # before libg4.so: one HIP runtime in the process

    import __graft_entry__
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    pkg = __graft_entry__.load_package()
    lib = pkg.lib()
    lib.g4_set_order(pkg.ORDER_REFERENCE if args.order == "reference" else pkg.ORDER_PARALLEL)
    if args.probe in ("prefill", "decode"):
        # one step kind alone, for kernel traces: the headline 512-token
        # prefill, or decode steps at 16384 positions of context
        image = pkg.Image.synthetic(seed=MODEL_SEED)
        pkg.check(lib.g4_init(image.records, 0))
        try:
            if args.probe == "prefill":
                model_benchmarks(pkg, lib, np, 10, 3, prefill_only=True)
            else:
                decode_probe(pkg, lib, np)
        finally:
            lib.g4_shutdown()
        return 0
    if args.probe:
        probe(pkg, lib, torch, args.probe)
        return 0

    t = time.perf_counter()
    image = pkg.Image.synthetic(seed=MODEL_SEED)
    log(f"synthetic E2B image {image.size / 1e9:.2f} GB in {time.perf_counter() - t:.1f} s")

    gemm = gemm_roofline(pkg, lib, torch)
    log(f"prefill GEMM 512x6144x1536: {gemm['ms_per_launch'] * 1e3:.1f} us, {gemm['tops']:.0f} TOPS")
    vendor = vendor_int8_gemm(torch)
    log(f"vendor int8 GEMM, same shape: {vendor}")
    sweep = gemv_sweep(pkg, lib, torch)
    log(f"decode GEMV sweep: {sweep['byte_weighted_gbs']:.0f} GB/s byte-weighted; {sweep['per_shape']}")
    kv = kv_roofline(pkg, lib, torch)
    log(f"global-layer decode attention at 16K keys: {kv['ms'] * 1e3:.1f} us, {kv['gbs']:.0f} GB/s of K+V")
    torch.cuda.empty_cache()

    t = time.perf_counter()
    pkg.check(lib.g4_init(image.records, 0))
    log(f"g4_init (upload + KV allocation) {time.perf_counter() - t:.1f} s")
    try:
        res = model_benchmarks(pkg, lib, np, args.steps, args.warmup)
        parallel = parallel_order_figures(pkg, lib, np) if args.order == "reference" else None
    finally:
        lib.g4_shutdown()

    cpu = None if args.no_cpu else cpu_baseline(pkg, image, np)
    steps_ms = res["prefill512_s"] / args.steps * 1e3
    line = {
        "metric": "prefill tok/s @512 & 8192 tok; decode tok/s @16K ctx; %HBM/%MFMA peak, 1 GPU",
        "value": round(res["prefill512_tok_s"], 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(steps_ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": "Gemma-4-E2B-shaped random-init model in the exporter .bin layout "
                        "(N(0,0.02) int8 matrices, seed 20261201); step = 512-token prefill + logits",
            "prefill_tokens": 512,
            "summation_order": args.order,
        },
        "prefill8192_tok_s": round(res["prefill8192_tok_s"], 1),
        "decode16k_tok_s": round(res["decode16k_tok_s"], 2),
        "dump2388_rows_s": round(res["dump2388_rows_s"], 1),
        # the same figures in the parallel summation order, which is not
        # bit-identical: the logits of one 512-token prefill move by the delta
        "prefill8192_tok_s_parallel": parallel and parallel["prefill8192_tok_s"],
        "decode16k_tok_s_parallel": parallel and parallel["decode16k_tok_s"],
        "parallel_order_logit_delta": parallel and round(parallel["max_abs_logit_delta_vs_reference_order"], 4),
        "roofline": {
            "bound": "mfma",
            "kernel": "k_gemm (prefill W8A8 GEMM, X[512x1536] x W[6144x1536])",
            "achieved": round(gemm["tops"], 1),
            "peak": INT8_MFMA_PEAK_TOPS,
            "unit": "TOPS",
            "frac": round(gemm["tops"] / INT8_MFMA_PEAK_TOPS, 4),
            "traffic": pmc_traffic("k_gemm_512x6144x1536_pmc.txt"),
            "algorithmic_bytes": gemm["bytes"],
            "traffic_source": "profiles/k_gemm_512x6144x1536_pmc.txt (HBM bytes per launch)",
            "us_per_launch": round(gemm["ms_per_launch"] * 1e3, 2),
            "hbm_frac": round(gemm["bytes"] / (gemm["ms_per_launch"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "warm": {"us": round(gemm["warm_ms"] * 1e3, 2),
                     "frac": round(gemm["ops"] / (gemm["warm_ms"] * 1e-3) / 1e12 / INT8_MFMA_PEAK_TOPS, 4)},
            "cold": {"us": round(gemm["cold_ms"] * 1e3, 2),
                     "frac": round(gemm["ops"] / (gemm["cold_ms"] * 1e-3) / 1e12 / INT8_MFMA_PEAK_TOPS, 4),
                     "hbm_frac": round(gemm["bytes"] / (gemm["cold_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
            "vendor_int8_gemm_same_shape": vendor,
        },
        "roofline_decode": {
            "bound": "hbm",
            "kernel": "k_gemv (decode W8A8 GEMV sweep, byte-weighted over one token's linears)",
            "achieved": round(sweep["byte_weighted_gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(sweep["byte_weighted_gbs"] / HBM_PEAK_GBS, 4),
            "bytes_per_token": sweep["bytes_per_token"],
            "per_shape_gbs": sweep["per_shape"],
            "traffic": pmc_traffic("k_gemv_262144x1536_pmc.txt"),
            "traffic_source": "profiles/k_gemv_262144x1536_pmc.txt (HBM bytes per lm_head launch)",
        },
        "roofline_kv": {
            "bound": "hbm",
            "kernel": "global-layer decode attention over 16384 keys (scores read K, P.V reads V; hd 512, "
                      "8 query heads, reference order)",
            "achieved": round(kv["gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(kv["gbs"] / HBM_PEAK_GBS, 4),
            "bytes_per_layer": kv["bytes"],
            "us_per_layer": round(kv["ms"] * 1e3, 2),
            "k_read_gbs_scores": kv.get("k_read_gbs_scores") and round(kv["k_read_gbs_scores"], 1),
            "v_read_gbs_values": kv.get("v_read_gbs_values") and round(kv["v_read_gbs_values"], 1),
            "split_source": "profiles/attend_global_16k_kernel_stats.txt (kernel trace of bench.py --probe kv)",
            "decode_step_traffic": pmc_traffic("decode16k_step_pmc.txt"),
            "decode_step_algorithmic_bytes": DECODE16K_STEP_BYTES,
            "decode_step_traffic_source": "profiles/decode16k_step_pmc.txt (HBM bytes per decode step at 16K)",
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
