"""Writes tests/golden/*.npz: outputs of the reference's own x86_avx2 silicon family (oracle/_ref, built from
/root/reference's sources by oracle/Makefile) on the BASELINE configurations' seeded inputs.

The reference ships no known-answer vectors for attention, so these are made here, by running the
reference's code as its engine runs it: the family's nn doors called through its door table. Each file
holds the fp16 output bits (uint16), the rows they are for, and the SHA-256 of the seeded inputs, so a
change in the input generator is caught before any comparison. Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle.oracle import RefFamily  # noqa: E402
from silvann_amd import workloads as W  # noqa: E402

OUT = Path(__file__).resolve().parent


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def decode_rows(R, w, rows, route):
    fn = R.decode if route == "scores_mix" else R.decode_tiered
    qs = w.q.reshape(w.rows, -1)
    out = []
    for u in rows:
        k, v = w.gathered(u)
        o, over = fn(qs[u], k, v, w.q_heads, w.kv_heads, w.head_dim, int(w.lens[u]))
        assert over == 0
        out.append(o.view(np.uint16))
    return np.stack(out)


def causal_rows(R, c, rows):
    """Row r of the chunk is the reference's decode at position first + r over positions 0..first+r (the rows
    verb's causal doors compute exactly that row, attention__abi.cuh:336-342)."""
    k, v = c.gathered()
    row = c.kv_heads * c.head_dim
    qs = c.q.reshape(c.rows, -1)
    out = []
    for r in rows:
        n = c.first + r + 1
        o, over = R.decode(qs[r], k[: n * row], v[: n * row], c.q_heads, c.kv_heads, c.head_dim, n)
        assert over == 0
        out.append(o.view(np.uint16))
    return np.stack(out)


def main():
    R = RefFamily()
    # C1: both decode routes, the whole output
    w = W.config1()
    np.savez_compressed(OUT / "decode_c1.npz", scores_mix=decode_rows(R, w, [0], "scores_mix"),
                        tiered=decode_rows(R, w, [0], "tiered"), inputs=digest(w.q, w.k, w.v))
    print("decode_c1")
    # C2: every sequence through the tiered route, four through scores+mix
    w = W.config2()
    np.savez_compressed(OUT / "decode_c2.npz", tiered=decode_rows(R, w, range(w.rows), "tiered"),
                        scores_mix=decode_rows(R, w, [0, 1, 2, 3], "scores_mix"), lens=w.lens,
                        inputs=digest(w.lens, w.pages, w.q, w.k, w.v))
    print("decode_c2")
    # C5
    w = W.config5()
    np.savez_compressed(OUT / "decode_c5.npz", tiered=decode_rows(R, w, [0], "tiered"),
                        inputs=digest(w.pages, w.q, w.k, w.v))
    print("decode_c5")
    # C3 / C4: chosen rows
    c = W.config3()
    rows3 = np.array([0, 1, 31, 32, 63, 64, 255, 1000, 2047, 4095], np.uint32)
    np.savez_compressed(OUT / "causal_c3.npz", rows=rows3, out=causal_rows(R, c, rows3), inputs=digest(c.q, c.k, c.v))
    print("causal_c3")
    c = W.config4()
    rows4 = np.array([0, 1, 1000, 2047], np.uint32)
    np.savez_compressed(OUT / "causal_c4.npz", rows=rows4, out=causal_rows(R, c, rows4),
                        inputs=digest(c.pages, c.q, c.k, c.v))
    print("causal_c4")
    # a small causal chunk through the rows verb's three doors, whole (causal_scores_grouped, causal_softmax,
    # causal_mix), fp32 weights included
    c = W.causal("small", 16, 2, 128, 40, 64, seed=77)
    k, v = c.gathered()
    p = R.causal_scores_grouped(c.q, k, 16, 2, 128, 40, 64)
    p = R.causal_softmax(p, 16, 40, 64)
    o, over = R.causal_mix(p, v, 16, 2, 128, 40, 64)
    assert over == 0
    np.savez_compressed(OUT / "causal_small.npz", p=p, out=o.view(np.uint16), inputs=digest(c.q, c.k, c.v))
    print("causal_small")


if __name__ == "__main__":
    main()
