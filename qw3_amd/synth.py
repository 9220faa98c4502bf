"""Seeded synthetic inputs for the benchmark configurations.

Host-side generation uses numpy's PCG64 generator; each tensor gets its own
stream, seeded by SeedSequence([config, layer, tensor-id, seed]), so inputs are
reproducible and independent across layers. Large KV caches can instead be
filled on the device (Ctx.fill_normal_f16), which the benchmark uses.

Config shapes (head_dim 128 throughout):
  C0  decode, 32q/4kv, cap 32, 31 cached tokens, theta 1e6
  C1  decode, 32q/4kv, cap 8192, 8191 cached tokens, 48 layers, theta 1e6
  C2  prefill, 2048 tokens, 32q/4kv, empty cache of 2048, theta 1e6,
      q/k/v drawn as f16 values (carried in f32, exactly representable)
  C3  decode, 64q/4kv, cap 32768, 32767 cached tokens, 47 layers, theta 5e6
  C4  paged decode: 32 sequences, lengths U[512, 16384] (the appended token
      included), 16-token pages, each sequence's pages a seeded random draw
      without replacement from a shared pool of sum(ceil(L/16)) pages
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

TENSOR_IDS = {"q": 1, "k": 2, "v": 3, "q_norm": 4, "k_norm": 5, "k_cache": 6, "v_cache": 7, "lens": 8,
              "pages": 9}


def rng(config: int, layer: int, tensor: str, seed: int = 0) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence([config, layer, TENSOR_IDS[tensor], seed])))


def normal_f32(g: np.random.Generator, shape, mean=0.0, std=1.0) -> np.ndarray:
    return (g.standard_normal(shape, dtype=np.float32) * np.float32(std) + np.float32(mean)).astype(np.float32)


def f16_bits(x: np.ndarray) -> np.ndarray:
    """IEEE round-to-nearest-even f32 -> f16, as uint16 bit patterns."""
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def f16_values(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


@dataclass
class Shape:
    n_q_heads: int = 32
    n_kv_heads: int = 4
    head_dim: int = 128
    theta: float = 1.0e6
    eps: float = 1.0e-6

    @property
    def scale(self) -> float:
        return float(np.float32(1.0) / np.sqrt(np.float32(self.head_dim)))


CONFIGS = {
    0: dict(kind="decode", shape=Shape(), cap=32, pos=31, layers=1),
    1: dict(kind="decode", shape=Shape(), cap=8192, pos=8191, layers=48),
    2: dict(kind="prefill", shape=Shape(), cap=2048, pos=0, tokens=2048, layers=1),
    3: dict(kind="decode", shape=Shape(n_q_heads=64, theta=5.0e6), cap=32768, pos=32767, layers=47),
    4: dict(kind="paged", shape=Shape(), n_seqs=32, lo=512, hi=16384, page_size=16, layers=48),
}


def step_inputs(config: int, layer: int, n_tokens: int, s: Shape, f16_exact: bool = False, seed: int = 0):
    """q [T,Hq,d], k/v [T,Hkv,d] f32 N(0,1); q_norm/k_norm [d] f32 N(1, 0.02)."""
    d = s.head_dim
    q = normal_f32(rng(config, layer, "q", seed), (n_tokens, s.n_q_heads, d))
    k = normal_f32(rng(config, layer, "k", seed), (n_tokens, s.n_kv_heads, d))
    v = normal_f32(rng(config, layer, "v", seed), (n_tokens, s.n_kv_heads, d))
    if f16_exact:
        q, k, v = (f16_values(f16_bits(t)) for t in (q, k, v))
    qn = normal_f32(rng(config, layer, "q_norm", seed), (d,), 1.0, 0.02)
    kn = normal_f32(rng(config, layer, "k_norm", seed), (d,), 1.0, 0.02)
    return q, k, v, qn, kn


def cache_f16(config: int, layer: int, s: Shape, cap: int, n_filled: int, seed: int = 0):
    """K and V caches [Hkv, cap, d] as f16 bits; positions < n_filled hold N(0,1)."""
    out = []
    for name in ("k_cache", "v_cache"):
        c = np.zeros((s.n_kv_heads, cap, s.head_dim), np.uint16)
        if n_filled:
            c[:, :n_filled] = f16_bits(normal_f32(rng(config, layer, name, seed), (s.n_kv_heads, n_filled, s.head_dim)))
        out.append(c)
    return out[0], out[1]


@dataclass
class PagedLayout:
    seq_lens: np.ndarray     # i32 [n_seqs], includes the appended token
    page_table: np.ndarray   # i32 [n_seqs, max_pages], -1 past a sequence's pages
    n_pages: int
    page_size: int

    @property
    def max_pages(self) -> int:
        return self.page_table.shape[1]

    def slot(self, b: int, p: int) -> int:
        return int(self.page_table[b, p // self.page_size]) * self.page_size + p % self.page_size


def paged_layout(n_seqs: int, lo: int, hi: int, page_size: int, seed: int = 0, config: int = 4) -> PagedLayout:
    lens = rng(config, 0, "lens", seed).integers(lo, hi + 1, size=n_seqs, dtype=np.int64).astype(np.int32)
    pages_per = (lens.astype(np.int64) + page_size - 1) // page_size
    n_pages = int(pages_per.sum())
    perm = rng(config, 0, "pages", seed).permutation(n_pages).astype(np.int32)
    max_pages = int(pages_per.max())
    table = np.full((n_seqs, max_pages), -1, np.int32)
    off = 0
    for b in range(n_seqs):
        table[b, :pages_per[b]] = perm[off:off + pages_per[b]]
        off += pages_per[b]
    return PagedLayout(lens, table, n_pages, page_size)
