"""The C oracle against the golden vectors the reference's own x86_avx2 family produced (tests/golden/).

The family runs attention_mix through its own AVX loop (x86_avx2/overrides/nn.cuh:1973-2071), a different
fp32 summation order from the generic body the oracle restates, so outputs are compared to within two fp16
ulps of the larger magnitude (plus the north star's max-abs / cosine bar); the input digests are exact.
"""
import hashlib
from pathlib import Path

import numpy as np
import pytest

from silvann_amd import workloads as W
from tests.conftest import parity

GOLD = Path(__file__).resolve().parent / "golden"


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def load(name):
    return np.load(GOLD / name, allow_pickle=False)


def within_ulp(got, want_bits):
    g = np.asarray(got, np.float16).astype(np.float32).ravel()
    w = want_bits.view(np.float16).astype(np.float32).ravel()
    ulp = np.spacing(np.maximum(np.abs(g), np.abs(w)).astype(np.float16)).astype(np.float32)
    tol = 2 * ulp + 1e-6   # the floor covers fp16 subnormals, whose spacing is 6e-8
    assert np.all(np.abs(g - w) <= tol), float(np.max(np.abs(g - w) - tol))
    parity(g, w)


def oracle_decode_rows(oracle, w, rows):
    qs = w.q.reshape(w.rows, -1)
    out = []
    for u in rows:
        k, v = w.gathered(u)
        p = oracle.scores(qs[u], k, w.q_heads, w.kv_heads, w.head_dim, int(w.lens[u]))
        o, over = oracle.mix(p, v, w.q_heads, w.kv_heads, w.head_dim, int(w.lens[u]))
        assert over == 0
        out.append(o)
    return np.stack(out)


def test_config1(oracle):
    g = load("decode_c1.npz")
    w = W.config1()
    assert digest(w.q, w.k, w.v) == str(g["inputs"])
    o = oracle_decode_rows(oracle, w, [0])
    within_ulp(o, g["scores_mix"])
    within_ulp(o, g["tiered"])


def test_config2_rows(oracle):
    g = load("decode_c2.npz")
    w = W.config2()
    assert digest(w.lens, w.pages, w.q, w.k, w.v) == str(g["inputs"])
    assert np.array_equal(w.lens, g["lens"])
    o = oracle_decode_rows(oracle, w, [0, 1, 2, 3])
    within_ulp(o, g["scores_mix"])
    within_ulp(o, g["tiered"][:4])


def test_config5(oracle):
    g = load("decode_c5.npz")
    w = W.config5()
    assert digest(w.pages, w.q, w.k, w.v) == str(g["inputs"])
    o, over = oracle.decode_paged(w.q, w.k, w.v, w.pages, w.pages_row, w.page_size, 0, w.lens, 16, 2, 256, 1)
    within_ulp(o, g["tiered"])


@pytest.mark.parametrize("name,make", [("causal_c3.npz", W.config3), ("causal_c4.npz", W.config4)])
def test_causal_rows(oracle, name, make):
    g = load(name)
    c = make()
    ins = (c.q, c.k, c.v) if c.pages is None else (c.pages, c.q, c.k, c.v)
    assert digest(*ins) == str(g["inputs"])
    rows = g["rows"] if c.pages is None else g["rows"][:2]   # two rows over the 100k prefix keep this quick
    o, over = oracle.causal_rows(c.q, c.k, c.v, c.pages, c.page_size, c.q_heads, c.kv_heads, c.head_dim, c.first, rows)
    assert over == 0
    within_ulp(o.reshape(len(rows), -1), g["out"][: len(rows)])


def test_causal_small_three_doors(oracle):
    g = load("causal_small.npz")
    c = W.causal("small", 16, 2, 128, 40, 64, seed=77)
    assert digest(c.q, c.k, c.v) == str(g["inputs"])
    p = oracle.causal_scores_grouped(c.q, c.k, 16, 2, 128, 40, 64)
    p = oracle.causal_softmax(p, 16, 40, 64)
    np.testing.assert_allclose(p, g["p"], rtol=2e-5, atol=1e-7)
    o, _ = oracle.causal_mix(p, c.v, 16, 2, 128, 40, 64)
    within_ulp(o, g["out"])
