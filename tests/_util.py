"""Shared test helpers: seeded inputs and host<->device copies."""
from __future__ import annotations

import numpy as np


class Lcg:
    """The fixed LCG of the reference kernel tests (native/tests/kernel_ops.cpp:
    206-216): x = x*1664525 + 1013904223; uniform = lo + (hi-lo)*(x>>8)/2^24,
    rounded to bf16 (RNE)."""

    def __init__(self, seed: int):
        self.x = seed & 0xFFFFFFFF

    def next(self) -> int:
        self.x = (self.x * 1664525 + 1013904223) & 0xFFFFFFFF
        return self.x

    def uniform(self, lo: float, hi: float, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        for i in range(n):
            out[i] = np.float32(lo) + np.float32(hi - lo) * (
                np.float32(self.next() >> 8) * np.float32(1.0 / 16777216.0))
        return out

    def bf16(self, lo, hi, n):
        import oracle
        return oracle.f32_to_bf16(self.uniform(lo, hi, n))


def randn_bf16(rng: np.random.Generator, n: int, scale: float = 1.0) -> np.ndarray:
    import oracle
    return oracle.f32_to_bf16((rng.standard_normal(n) * scale).astype(np.float32))


def to_dev(a: np.ndarray, dev):
    import torch
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.uint32:
        a = a.view(np.int32)
    elif a.dtype == np.uint64:
        a = a.view(np.int64)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def from_dev(t, dtype=np.uint16) -> np.ndarray:
    return t.detach().cpu().numpy().view(dtype)


def fill_pool(pool, orc, P, maxp, layer, pt, seq, gen, kv_heads=(0, 1)):
    """Writes K/V of positions 0..seq-1 (all heads) from `gen(n)` bf16 values."""
    for j in range(seq):
        base = orc.kv_off(P, maxp, layer, int(pt[j // P]), j % P, 0, 0, 0)
        pool[base:base + 512] = gen(512)
