"""Device copies of the workloads, the library's calls on them, and a plain torch fp32 attention (the
floating-point reference for full-size checks, beside the C oracle on subsets)."""
from __future__ import annotations

import math

import numpy as np
import torch

from silvann_amd import verbs


def t(a, dev, dtype=None):
    x = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return x if dtype is None else x.view(dtype)


class DecodeOnDevice:
    def __init__(self, w, dev):
        self.w = w
        self.q = t(w.q, dev)
        self.k = t(w.k, dev)
        self.v = t(w.v, dev)
        self.lens = t(w.lens, dev)
        self.pages = None if w.pages is None else t(w.pages, dev)
        self.out = torch.zeros(w.rows * w.q_heads * w.head_dim, dtype=torch.float16, device=dev)
        self.over = torch.zeros(1, dtype=torch.int32, device=dev)
        need = verbs.decode_paged_scratch_bytes(w.q_heads, w.kv_heads, w.head_dim, w.most, w.rows)
        self.scratch = torch.empty(max(need, 4), dtype=torch.uint8, device=dev)

    def run(self):
        w = self.w
        verbs.decode_paged(self.q, self.k, self.v, self.pages, self.lens, self.out, w.q_heads, w.kv_heads,
                           w.head_dim, w.most, page_size=w.page_size, pages_row=w.pages_row, k_row=w.k_row,
                           scratch=self.scratch, over=self.over)
        return self.out


class CausalOnDevice:
    def __init__(self, w, dev):
        self.w = w
        self.q = t(w.q, dev)
        self.k = t(w.k, dev)
        self.v = t(w.v, dev)
        self.pages = None if w.pages is None else t(w.pages, dev)
        self.out = torch.zeros(w.rows * w.q_heads * w.head_dim, dtype=torch.float16, device=dev)
        self.over = torch.zeros(1, dtype=torch.int32, device=dev)

    def run(self):
        w = self.w
        verbs.causal_paged(self.q, self.k, self.v, self.pages, self.out, w.q_heads, w.kv_heads, w.head_dim, w.first,
                           w.rows, page_size=w.page_size, over=self.over)
        return self.out


def torch_decode_row(q, k, v, q_heads, kv_heads, head_dim):
    """softmax(q·kᵀ/√d)·v in fp32 for one query over a gathered cache (torch tensors of halves)."""
    n = k.numel() // (kv_heads * head_dim)
    qf = q.float().view(q_heads, head_dim)
    kf = k.float().view(n, kv_heads, head_dim)
    vf = v.float().view(n, kv_heads, head_dim)
    g = q_heads // kv_heads
    kh = kf[:, torch.arange(q_heads, device=q.device) // g, :]   # [n][qh][hd]
    vh = vf[:, torch.arange(q_heads, device=q.device) // g, :]
    s = torch.einsum("hd,nhd->hn", qf, kh) * (1.0 / math.sqrt(head_dim))
    p = torch.softmax(s, dim=1)
    return torch.einsum("hn,nhd->hd", p, vh)


def torch_causal(q, k, v, q_heads, kv_heads, head_dim, first, rows, chunk=256):
    """Causal attention of rows first.. over a gathered cache, fp32, `chunk` rows at a time."""
    n = first + rows
    qf = q.float().view(rows, q_heads, head_dim)
    kf = k.float().view(n, kv_heads, head_dim)
    vf = v.float().view(n, kv_heads, head_dim)
    g = q_heads // kv_heads
    out = torch.empty(rows, q_heads, head_dim, dtype=torch.float32, device=q.device)
    scale = 1.0 / math.sqrt(head_dim)
    pos = torch.arange(n, device=q.device)
    for h in range(q_heads):
        kh, vh = kf[:, h // g, :], vf[:, h // g, :]
        for r0 in range(0, rows, chunk):
            r1 = min(rows, r0 + chunk)
            s = (qf[r0:r1, h, :] @ kh.T) * scale
            rowpos = first + torch.arange(r0, r1, device=q.device)
            s = s.masked_fill(pos[None, :] > rowpos[:, None], float("-inf"))
            out[r0:r1, h, :] = torch.softmax(s, dim=1) @ vh
    return out.view(-1)
