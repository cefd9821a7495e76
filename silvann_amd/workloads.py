"""The benchmark configurations' synthetic inputs, made the same way everywhere (tests, bench, smoke).

Every array comes from one `numpy.random.default_rng(seed)` in a fixed order: the lengths (batched decode),
the page permutation, then q, k, v as standard normals in float32 narrowed to float16. A cache is a pool of
pages, `page_size` positions × kv_heads × head_dim halves a page; row u's logical page j is physical page
`pages[u·pages_row + j]`. `page_size` 0 means a contiguous cache, as the reference keeps it.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class Decode:
    name: str
    q_heads: int
    kv_heads: int
    head_dim: int
    lens: np.ndarray          # uint32 [rows]
    page_size: int            # 0: contiguous, row u's cache at u·k_row halves
    pages: np.ndarray | None  # uint32 [rows · pages_row]
    pages_row: int
    k_row: int
    q: np.ndarray             # f16 [rows][q_heads][head_dim]
    k: np.ndarray             # f16 pool
    v: np.ndarray
    seed: int = 0

    @property
    def rows(self) -> int:
        return len(self.lens)

    @property
    def most(self) -> int:
        return int(self.lens.max())

    def kv_bytes(self) -> int:
        """The algorithmic bytes: every cached position's K and V row of every kv head, once."""
        return int(self.lens.astype(np.int64).sum()) * self.kv_heads * self.head_dim * 2 * 2

    def io_bytes(self) -> int:
        """Plus q and o (fp16) and the page-table entries read."""
        qo = 2 * self.rows * self.q_heads * self.head_dim * 2
        pt = 0 if self.pages is None else 4 * int(sum((int(l) + self.page_size - 1) // self.page_size for l in self.lens))
        return self.kv_bytes() + qo + pt

    def gathered(self, u: int):
        """Row u's K and V as the reference keeps them: contiguous [position][kv_head][head_dim]."""
        row = self.kv_heads * self.head_dim
        n = int(self.lens[u])
        if self.pages is None:
            base = u * self.k_row
            return self.k[base: base + n * row], self.v[base: base + n * row]
        pos = np.arange(n)
        phys = self.pages[u * self.pages_row + pos // self.page_size].astype(np.int64) * self.page_size + pos % self.page_size
        idx = (phys[:, None] * row + np.arange(row)[None, :]).ravel()
        return self.k[idx], self.v[idx]


@dataclass
class Causal:
    name: str
    q_heads: int
    kv_heads: int
    head_dim: int
    first: int
    rows: int
    page_size: int
    pages: np.ndarray | None
    q: np.ndarray
    k: np.ndarray
    v: np.ndarray
    seed: int = 0

    def pairs(self) -> int:
        """Unmasked (query, key) pairs: every row sees `first` prefix keys plus itself and the rows before."""
        return self.rows * self.first + self.rows * (self.rows + 1) // 2

    def flops(self) -> int:
        """4·q_heads·head_dim a pair: QK^T and PV, a multiply and an add each."""
        return 4 * self.q_heads * self.head_dim * self.pairs()

    def kv_bytes(self) -> int:
        return (self.first + self.rows) * self.kv_heads * self.head_dim * 2 * 2

    def gathered(self):
        row = self.kv_heads * self.head_dim
        n = self.first + self.rows
        if self.pages is None:
            return self.k[: n * row], self.v[: n * row]
        pos = np.arange(n)
        phys = self.pages[pos // self.page_size].astype(np.int64) * self.page_size + pos % self.page_size
        idx = (phys[:, None] * row + np.arange(row)[None, :]).ravel()
        return self.k[idx], self.v[idx]


def _normal(rng, n):
    return rng.standard_normal(n, dtype=np.float32).astype(np.float16)


def device_normal(n, seed, dev):
    """N(0,1) halves made on the GPU from a seeded torch generator — the benchmark's fast path for large
    pools (a different stream of numbers from the numpy one; both sides of a check use the same arrays)."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return torch.randn(n, generator=g, dtype=torch.float32, device=dev).half()


def _qkv(rng, seed, dev, nq, nkv):
    if dev is None:
        return _normal(rng, nq), _normal(rng, nkv), _normal(rng, nkv)
    return (device_normal(nq, 3 * seed + 1, dev), device_normal(nkv, 3 * seed + 2, dev),
            device_normal(nkv, 3 * seed + 3, dev))


def decode(name, q_heads, kv_heads, head_dim, lens, page_size=0, seed=0, permute=True, rng=None, dev=None) -> Decode:
    rng = rng or np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.uint32)
    rows, row = len(lens), kv_heads * head_dim
    if page_size:
        per = [(int(l) + page_size - 1) // page_size for l in lens]
        pool = sum(per)
        perm = rng.permutation(pool).astype(np.uint32) if permute else np.arange(pool, dtype=np.uint32)
        pages_row = max(per)
        pages = np.zeros(rows * pages_row, np.uint32)
        at = 0
        for u, n in enumerate(per):
            pages[u * pages_row: u * pages_row + n] = perm[at: at + n]
            at += n
        slots, k_row = pool * page_size, 0
    else:
        pages, pages_row = None, 0
        k_row = int(lens.max()) * row
        slots = rows * int(lens.max())
    q, k, v = _qkv(rng, seed, dev, rows * q_heads * head_dim, slots * row)
    return Decode(name, q_heads, kv_heads, head_dim, lens, page_size, pages, pages_row, k_row, q, k, v, seed)


def causal(name, q_heads, kv_heads, head_dim, first, rows, page_size=0, seed=0, permute=True, dev=None) -> Causal:
    rng = np.random.default_rng(seed)
    n, row = first + rows, kv_heads * head_dim
    if page_size:
        npages = (n + page_size - 1) // page_size
        pages = rng.permutation(npages).astype(np.uint32) if permute else np.arange(npages, dtype=np.uint32)
        slots = npages * page_size
    else:
        pages, slots = None, n
    q, k, v = _qkv(rng, seed, dev, rows * q_heads * head_dim, slots * row)
    return Causal(name, q_heads, kv_heads, head_dim, first, rows, page_size, pages, q, k, v, seed)


# ── the BASELINE configurations ─────────────────────────────────────────────────────────────────────

def config1(seed=1, dev=None) -> Decode:
    """C1: single-sequence decode, 16 q / 2 kv heads, head_dim 256, 2,048 cached positions (contiguous)."""
    return decode("decode_c1_16q2kv_hd256_len2048", 16, 2, 256, [2048], page_size=0, seed=seed, dev=dev)


def config2(seed=2, dev=None) -> Decode:
    """C2: 32 sequences, lengths U[1024, 32768] from the seed, 32 q / 4 kv, head_dim 128, 256-position pages,
    each sequence's page table a slice of a seeded permutation of the pool."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(1024, 32769, 32)
    return decode("decode_c2_32seq_32q4kv_hd128_paged256", 32, 4, 128, lens, page_size=256, rng=rng, seed=seed, dev=dev)


def config3(seed=3, dev=None) -> Causal:
    """C3: causal prefill of 4,096 positions, no prefix, 16 q / 2 kv heads, head_dim 256."""
    return causal("causal_c3_4096_16q2kv_hd256", 16, 2, 256, 0, 4096, page_size=0, seed=seed, dev=dev)


def config4(seed=4, dev=None) -> Causal:
    """C4: 2,048 new positions over a 100,000-position paged prefix (256-position pages, permuted)."""
    return causal("causal_c4_2048_over_100000_16q2kv_hd256_paged256", 16, 2, 256, 100000, 2048, page_size=256, seed=seed, dev=dev)


def config5(seed=5, dev=None) -> Decode:
    """C5: one query over 262,144 cached positions in 1,024 permuted 256-position pages, 16 q / 2 kv, hd 256."""
    return decode("decode_c5_16q2kv_hd256_len262144_paged256", 16, 2, 256, [262144], page_size=256, seed=seed, dev=dev)


CONFIGS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}


@dataclass
class Tier:
    """A TurboQuant tier of one layer's cache (the tiers' verbs, mixer__abi.cuh:395-410): `length` key and value
    rows of width d (8 warm, 4 cold), kv head g of position t at row t·kv_heads + g, and `rows` rotated queries."""
    name: str
    q_heads: int
    kv_heads: int
    head_dim: int
    length: int
    d: int
    rows: int
    q: object
    k_codes: object
    k_scales: object
    v_codes: object
    v_scales: object
    seed: int = 0

    def row_bytes(self) -> int:
        per = 16 // self.d
        return (self.head_dim + per - 1) // per * 2

    def io_bytes(self) -> int:
        """What one pass reads and writes: every key and value row (codes and scale) once, the queries and the
        residuals."""
        cache = self.length * self.kv_heads * 2 * (self.row_bytes() + 2)
        return cache + self.rows * self.q_heads * (self.head_dim * 2 + (self.head_dim + 2) * 4)


def tier(name, q_heads, kv_heads, head_dim, length, d, rows=1, seed=0, dev=None) -> Tier:
    """Codes uniform over every code, scales the codec's for unit-rms rows (fp16(clip_d), kernels.cuh:2905-2925),
    q N(0,1) — the rows a rotated Gaussian cache encodes to, without running the encoder."""
    clip = {4: 2.7325895709952577, 8: 4.6036453045214065}[d]
    per = 16 // d
    rb = (head_dim + per - 1) // per * 2
    n = length * kv_heads
    if dev is None:
        rng = np.random.default_rng(seed)
        q = _normal(rng, rows * q_heads * head_dim)
        kc = rng.integers(0, 256, n * rb, dtype=np.uint8)
        vc = rng.integers(0, 256, n * rb, dtype=np.uint8)
        sc = np.full(n, clip, np.float16).view(np.uint16)
        return Tier(name, q_heads, kv_heads, head_dim, length, d, rows, q, kc, sc.copy(), vc, sc.copy(), seed)
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q = device_normal(rows * q_heads * head_dim, 3 * seed + 1, dev)
    kc = torch.randint(0, 256, (n * rb,), generator=g, dtype=torch.uint8, device=dev)
    vc = torch.randint(0, 256, (n * rb,), generator=g, dtype=torch.uint8, device=dev)
    sc = torch.full((n,), clip, dtype=torch.float16, device=dev)
    return Tier(name, q_heads, kv_heads, head_dim, length, d, rows, q, kc, sc, vc, sc.clone(), seed)


def tier_cold(seed=6, dev=None) -> Tier:
    """A long cold tier at C5's shape: 262,144 positions of 4-bit rows, 16 q / 2 kv heads, head_dim 256."""
    return tier("tq4_16q2kv_hd256_len262144", 16, 2, 256, 262144, 4, seed=seed, dev=dev)


def tier_warm(seed=7, dev=None) -> Tier:
    """The same at the warm tier's 8 bits."""
    return tier("tq8_16q2kv_hd256_len262144", 16, 2, 256, 262144, 8, seed=seed, dev=dev)


TIERS = {6: tier_cold, 7: tier_warm}


@dataclass
class Write:
    """New rows for the cache writer (attention_cache_write_paged): `rows` key and value rows of one sequence at
    positions first .. first+rows-1, the keys turned over `rot` elements by their positions' angles, into
    permuted pages of a pool sized for first + rows positions."""
    name: str
    kv_heads: int
    head_dim: int
    first: int
    rows: int
    page_size: int
    rot: int
    pages: object
    positions: object
    k: object
    v: object
    cs: object
    k_cache: object
    v_cache: object
    seed: int = 0

    @property
    def capacity(self) -> int:
        return self.first + self.rows

    def io_bytes(self) -> int:
        """What one write moves: each new key and value row read and written once, and the angles read."""
        return self.rows * self.kv_heads * self.head_dim * 2 * 2 * 2 + self.rows * self.rot * 4


def write(name, kv_heads, head_dim, first, rows, page_size, rot=None, seed=0, dev=None) -> Write:
    import torch
    rot = head_dim if rot is None else rot
    rng = np.random.default_rng(seed)
    npages = (first + rows + page_size - 1) // page_size
    pages = rng.permutation(npages).astype(np.int32)
    i = np.arange(rot // 2, dtype=np.float64)
    ang = np.arange(first, first + rows, dtype=np.float64)[:, None] * 1e6 ** (-2.0 * i / rot)[None, :]
    cs = np.concatenate([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32).ravel()
    n = rows * kv_heads * head_dim
    k = device_normal(n, 5 * seed + 1, dev)
    v = device_normal(n, 5 * seed + 2, dev)
    slots = npages * page_size * kv_heads * head_dim
    kc = torch.zeros(slots, dtype=torch.float16, device=dev)
    vc = torch.zeros(slots, dtype=torch.float16, device=dev)
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    return Write(name, kv_heads, head_dim, first, rows, page_size, rot, t(pages), t(np.array([first], np.int32)), k, v,
                 t(cs), kc, vc, seed)


def write_c4(seed=8, dev=None) -> Write:
    """C4's chunk written before it is attended: 2,048 rows after a 100,000-position prefix, 2 kv heads, head_dim
    256, fully turned, into 256-position permuted pages."""
    return write("write_2kv_hd256_rows2048_at100000", 2, 256, 100000, 2048, 256, seed=seed, dev=dev)


WRITES = {8: write_c4}


def latent(name, heads, latent_dim, lens, seed=0, dev=None) -> Decode:
    """Latent attention as row 137 takes it: `heads` query heads, one kv head, contiguous per-row caches of latents
    (v is the same tensor as k: the latents are both)."""
    w = decode(name, heads, 1, latent_dim, lens, page_size=0, seed=seed, dev=dev)
    w.v = w.k
    return w


def latent_glm(seed=9, dev=None) -> Decode:
    """GLM 5.3's latent attention over a dense cache: one decode query, 64 heads, 512-wide latents, 131,072 of them."""
    return latent("latent_64h_lat512_len131072", 64, 512, [131072], seed=seed, dev=dev)


LATENTS = {9: latent_glm}
