"""Write the golden vectors in tests/golden/ by running the reference's own
compiled gemma4.c (oracle/_ref/libgemma4ref.so, built from the reference
sources by oracle/Makefile) on seeded inputs.

    python tests/golden/make_golden.py

    python tests/golden/make_golden.py sample   # sample.npz only

sample.npz the sampler (gemma4.c:527-561): logits rows, temperatures, the
           generator state before each call, and the token and state after
ops.npz    per-kernel inputs and outputs (quantize, matmul_int8,
           attention_scores, softmax, weighted_value_sum, geglu, embedding,
           rmsnorm, add_and_scale, apply_rope)
model.npz  forward()/logits() of the synthetic E2B image (seed 20261201):
           SHA-256 and sampled values of whole logits rows, greedy tokens,
           and a digest of the image itself

The fixtures hold data only (inputs and the reference's outputs).
"""

from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

import __graft_entry__  # noqa: E402
from helpers import HostF32, HostWeight, gelu_table_exporter, image_digest  # noqa: E402
from oracle import binding  # noqa: E402

MODEL_SEED = 20261201
MODEL_TOKENS = np.array([2, 818, 5000, 262143, 17, 9, 100000, 31337], dtype=np.int32)
SAMPLE_IDX = np.random.default_rng(7).choice(262144, size=512, replace=False).astype(np.int64)


def sha(a: np.ndarray) -> np.ndarray:
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), dtype=np.uint8)


def make_ops(pkg, k: binding.Kernels) -> dict[str, np.ndarray]:
    g = np.random.default_rng(1234)
    out: dict[str, np.ndarray] = {}

    # quantize: a normal block plus a zero group, a single spike and a tiny row
    x = g.standard_normal((8, 1536)).astype(np.float32)
    x[3, :] = 0.0
    x[4, 70] = 1.0e4
    x[5, :] *= 1e-30
    x[6, :64] = np.linspace(-1, 1, 64, dtype=np.float32)
    q, s = k.quantize(x)
    out.update(quant_x=x, quant_q=q, quant_s=s)

    # matmul: two shapes, row counts that exercise partial row groups
    for name, (n, kk, rows) in {"mm_a": (64, 256, 5), "mm_b": (48, 1536, 9)}.items():
        w = g.integers(-127, 128, size=(n, kk), dtype=np.int8)
        ws = np.exp(g.uniform(np.log(1e-3), np.log(1e-2), size=(n, kk // 64))).astype(np.float16)
        hw = HostWeight(pkg, w, ws)
        xin = g.standard_normal((rows, kk)).astype(np.float32)
        xq, xs = k.quantize(xin)
        y = k.matmul(xq, xs, hw.record, n)
        out.update({f"{name}_w": w, f"{name}_ws": ws, f"{name}_xq": xq, f"{name}_xs": xs, f"{name}_y": y})

    # attention primitives over a wrapping ring of 256 rows
    hd, ring = 256, 256
    qv = g.standard_normal(hd).astype(np.float32)
    kc = g.standard_normal((ring, hd)).astype(np.float32)
    vc = g.standard_normal((ring, hd)).astype(np.float32)
    first, num = 200, 150
    sc = k.scores(qv, kc, first, num, ring - 1, hd)
    p = k.softmax(sc)
    o = k.value_sum(p, vc, first, num, ring - 1, hd)
    out.update(att_q=qv, att_k=kc, att_v=vc, att_first=np.int32(first), att_num=np.int32(num),
               att_scores=sc, att_p=p, att_o=o)

    # geglu with the exporter's table, values beyond both ends
    table = gelu_table_exporter()
    tab = HostF32(pkg, table, shape=(4096, -8, 8))
    gate = (g.standard_normal((4, 300)) * 4).astype(np.float32)
    gate[0, :4] = [-8.0, 8.0, -100.0, 100.0]
    up = g.standard_normal((4, 320)).astype(np.float32)
    gg = k.geglu(gate, up, 320, tab.record)
    out.update(geglu_table=table, geglu_gate=gate, geglu_up=up, geglu_out=gg)

    # embedding gather from a small packed table
    w = g.integers(-127, 128, size=(32, 128), dtype=np.int8)
    ws = np.exp(g.uniform(np.log(1e-3), np.log(1e-2), size=(32, 2))).astype(np.float16)
    hw = HostWeight(pkg, w, ws)
    toks = np.array([0, 31, 16, 5, 17, 5], dtype=np.int32)
    emb = k.embedding(hw.record, toks, np.float32(np.sqrt(np.float32(1536))))
    out.update(emb_w=w, emb_ws=ws, emb_tokens=toks, emb_out=emb)

    # rmsnorm with and without weight
    xr = (g.standard_normal((6, 1536)) * 3).astype(np.float32)
    wr = g.uniform(0.5, 1.5, 1536).astype(np.float32)
    rw = k.rmsnorm(xr, HostF32(pkg, wr).record, 1536, np.float32(1e-6))
    xh = g.standard_normal((16, 256)).astype(np.float32)
    rn = k.rmsnorm(xh, None, 256, np.float32(1e-6))
    out.update(rms_x=xr, rms_w=wr, rms_out=rw, rms_xh=xh, rms_outh=rn)

    # add_and_scale
    a = g.standard_normal(1000).astype(np.float32)
    b = g.standard_normal(1000).astype(np.float32)
    out.update(add_a=a, add_b=b, add_out=k.add_and_scale(a, b, np.float32(0.7071067)))

    # rope: 3 tokens x 2 heads x 256, 128 pairs, start 5; and 64 partial pairs of 512
    for name, (hdr, pairs) in {"rope_s": (256, 128), "rope_g": (512, 64)}.items():
        cosv = g.uniform(-1, 1, (16, pairs)).astype(np.float32)
        sinv = g.uniform(-1, 1, (16, pairs)).astype(np.float32)
        v = g.standard_normal((3, 2, hdr)).astype(np.float32)
        r = k.rope(HostF32(pkg, cosv).record, HostF32(pkg, sinv).record, v, 2, hdr, 5)
        out.update({f"{name}_cos": cosv, f"{name}_sin": sinv, f"{name}_v": v, f"{name}_out": r})
    return out


def make_model(pkg, image) -> dict[str, np.ndarray]:
    m = binding.Model(image, use_ref=True)
    m.forward(MODEL_TOKENS, 0)
    rows = {}
    for r in (0, 7):
        lg = m.logits(r)
        rows[r] = lg
    decoded = []
    lg = rows[7]
    pos = MODEL_TOKENS.size
    decode_sha = []
    for _ in range(4):
        nxt = int(np.argmax(lg))
        decoded.append(nxt)
        m.forward(np.array([nxt], np.int32), pos)
        pos += 1
        lg = m.logits(0)
        decode_sha.append(sha(lg))
    return dict(
        tokens=MODEL_TOKENS, sample_idx=SAMPLE_IDX,
        row0_sha=sha(rows[0]), row7_sha=sha(rows[7]),
        row0_sample=rows[0][SAMPLE_IDX], row7_sample=rows[7][SAMPLE_IDX],
        row7_argmax=np.int64(np.argmax(rows[7])),
        decode_tokens=np.array(decoded, np.int32), decode_sha=np.stack(decode_sha),
        decode_last_sample=lg[SAMPLE_IDX],
        image_digest=image_digest(image),
    )


def make_sample() -> dict[str, np.ndarray]:
    """The reference's sample() over SAMPLE_CASES (tests/helpers.py): for each
    logits row and temperature, DRAWS consecutive calls from a recorded
    generator state."""
    import ctypes

    from helpers import sample_cases

    lib = binding.ref()
    state = ctypes.c_ulonglong.in_dll(lib, "rng_state")
    rows, temps, states = sample_cases()
    tokens = np.zeros((len(rows), len(temps), len(states), SAMPLE_DRAWS), np.int32)
    after = np.zeros(tokens.shape, np.uint64)
    for r, row in enumerate(rows):
        for t, temp in enumerate(temps):
            for s0, start in enumerate(states):
                state.value = int(start)
                for d in range(SAMPLE_DRAWS):
                    tokens[r, t, s0, d] = lib.sample(row.ctypes.data, row.size, float(temp))
                    after[r, t, s0, d] = state.value
    return dict(rows=np.stack(rows), temps=np.array(temps, np.float32),
                states=np.array(states, np.uint64), tokens=tokens, states_after=after)


SAMPLE_DRAWS = 6


def main() -> None:
    if not binding.ref_available():
        sys.exit("oracle/_ref/libgemma4ref.so is not built (needs the reference checkout)")
    if sys.argv[1:] == ["sample"]:
        np.savez_compressed(os.path.join(HERE, "sample.npz"), **make_sample())
        print("sample.npz", os.path.getsize(os.path.join(HERE, "sample.npz")), "bytes")
        return
    pkg = __graft_entry__.load_package()
    ops = make_ops(pkg, binding.Kernels(use_ref=True))
    np.savez_compressed(os.path.join(HERE, "ops.npz"), **ops)
    image = pkg.Image.synthetic(seed=MODEL_SEED)
    digest_before = image_digest(image)
    model = make_model(pkg, image)
    model["image_digest"] = digest_before
    np.savez_compressed(os.path.join(HERE, "model.npz"), **model)
    for name in ("ops.npz", "model.npz"):
        print(name, os.path.getsize(os.path.join(HERE, name)), "bytes")


if __name__ == "__main__":
    main()
