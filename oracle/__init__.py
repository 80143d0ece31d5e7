"""CPU oracle of the paged KV-cache hot path.

TEST INFRASTRUCTURE ONLY: this package is the checker for the HIP kernels. It
may be imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg only; the product library (libminicpm_native.so) never calls it.

The numeric functions live in kv_oracle.c (liboracle_kv.so, built by
`make -C oracle`); each cites the reference file:line it restates. The page
allocator model below is pure Python integer logic. cpu_baseline.c is the
speed-oriented CPU restatement bench.py times as its reported CPU baseline
(checked against the oracle in tests/test_cpu_oracle.py).
"""
from __future__ import annotations

import ctypes as C
import math
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

HQ, HKV, GROUP, HD, ROW, PSTRIDE, SPLIT2 = 16, 2, 8, 128, 2560, 130, 32


def build() -> str:
    """Compiles liboracle_kv.so in place (gcc) and returns its path."""
    import subprocess
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle_kv.so"], check=True)
    return os.path.join(_HERE, "liboracle_kv.so")


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle_kv.so")
        if not os.path.exists(path):
            build()
        L = C.CDLL(path)
        P = C.c_void_p
        u32, u64, dbl, i32 = C.c_uint32, C.c_uint64, C.c_double, C.c_int
        L.orc_kv_off.restype = u64
        L.orc_kv_off.argtypes = [u32] * 8
        L.orc_f2bf.restype = C.c_uint16
        L.orc_f2bf.argtypes = [C.c_float]
        L.orc_rope_sincos_batch.argtypes = [P, C.c_size_t, P, P]
        L.orc_inv_freq.argtypes = [dbl, P]
        L.orc_rope_append.argtypes = [P, u32, u32, u32, P, u32, u32, dbl, i32, P, P]
        L.orc_attn_ref.argtypes = [P, u32, u32, u32, P, P, u32, u32, P, i32]
        L.orc_decode_chunks.argtypes = [P, u32, u32, P, P, u32, u32, u32, u32, P, P]
        L.orc_decode_chunks_p.argtypes = [P, u32, u32, P, P, u32, u32, u32, u32, P, P, i32]
        L.orc_merge2.argtypes = [P, u32, u32, P, P]
        L.orc_decode_cpu_mt.argtypes = [P, P, P, P, u32, u32, u32, u32, P, i32]
        _LIB = L
    return _LIB


_CPB = {}


def cpu_baseline_lib(native: bool = False):
    """The CPU baseline library: the portable build (make -C oracle), or,
    with native=True, a -O3 -march=native build for this host compiled into a
    temporary directory (falls back to the portable build if gcc fails).
    Returns (ctypes library, description of the build)."""
    import subprocess
    import tempfile
    key = "native" if native else "portable"
    if key in _CPB:
        return _CPB[key]
    path, how = os.path.join(_HERE, "libcpu_baseline.so"), "gcc -O3 -march=x86-64-v2"
    if native:
        d = tempfile.mkdtemp(prefix="cpb_")
        cand = os.path.join(d, "libcpu_baseline_native.so")
        r = subprocess.run(["gcc", "-O3", "-march=native", "-fPIC", "-std=c11", "-shared",
                            os.path.join(_HERE, "cpu_baseline.c"), "-o", cand, "-lm",
                            "-lpthread"], capture_output=True)
        if r.returncode == 0:
            path, how = cand, "gcc -O3 -march=native"
    if not os.path.exists(path):
        subprocess.run(["make", "-s", "-C", _HERE, "libcpu_baseline.so"], check=True)
    L = C.CDLL(path)
    P, u32 = C.c_void_p, C.c_uint32
    L.cpb_decode_state_bytes.restype = C.c_size_t
    L.cpb_decode_state_bytes.argtypes = [u32, u32]
    L.cpb_decode.argtypes = [P, P, P, P, u32, u32, u32, u32, u32, P, P, C.c_int]
    L.cpb_rope_append.argtypes = [P, u32, u32, u32, P, u32, u32, P, P, C.c_int]
    _CPB[key] = (L, how)
    return _CPB[key]


def cpb_decode(q_rows, limits, page_tables, pool, layer, P, maxp, threads, nseg=None,
               native=False):
    """Speed-oriented fp32 CPU decode of B sessions (cpu_baseline.c)."""
    L, _ = cpu_baseline_lib(native)
    B = len(limits)
    if nseg is None:
        nseg = max(1, (4 * threads + 2 * B - 1) // (2 * B))
    lim = np.ascontiguousarray(limits, dtype=np.uint32)
    tabs = [np.ascontiguousarray(t, dtype=np.uint32) for t in page_tables]
    ptrs = (C.c_void_p * B)(*[t.ctypes.data for t in tabs])
    states = np.zeros(L.cpb_decode_state_bytes(B, nseg), dtype=np.uint8)
    out = np.zeros((B, 2048), dtype=np.uint16)
    L.cpb_decode(_p(np.ascontiguousarray(q_rows)), _p(lim), ptrs, _p(pool), layer, P, maxp, B,
                 nseg, _p(states), _p(out), threads)
    return out


def cpb_rope_append(qkv, tokens, base_pos, layer, pt, P, maxp, theta, pool, threads,
                    native=False):
    """Speed-oriented RoPE + append (cpu_baseline.c); q rotated in place."""
    L, _ = cpu_baseline_lib(native)
    inv = inv_freq(theta)
    pt = np.ascontiguousarray(pt, dtype=np.uint32)
    L.cpb_rope_append(_p(qkv), tokens, base_pos, layer, _p(pt), P, maxp, _p(inv), _p(pool),
                      threads)


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


# ---------------- bf16 helpers (numpy, RNE) ----------------

def f32_to_bf16(x) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bits (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------- layout ----------------

def kv_off(P, maxp, layer, page, slot, kv, head, d) -> int:
    """native/runtime/kv_cache.h:40-45 (P as a parameter)."""
    return int(lib().orc_kv_off(P, maxp, layer, page, slot, kv, head, d))


def chunk_pos(max_ctx: int, c512: bool = False) -> int:
    """native/kernels/sm120/kernels.h:292-304; c512: MC_ATTN_CHUNK512_ON set
    (and MC_ATTN_CHUNK512_OFF unset), which gives contexts above 114688
    positions 512-position chunks."""
    if max_ctx <= 16384:
        return 64
    if max_ctx <= 49152:
        return 128
    if max_ctx <= 114688 or not c512:
        return 256
    return 512


def prefill_split_kv(tokens: int) -> int:
    """native/kernels/sm120/kernels.h:517-521."""
    if tokens >= 2048:
        return 1
    return max(1, min(8, 4096 // tokens))


# ---------------- allocator model ----------------

class PagedKvAllocatorModel:
    """native/runtime/kv_cache.cpp:8-91 stated in Python: lowest free page,
    host shadow, sync only when the owned count grew, release_all."""

    def __init__(self, max_pages: int, tokens_per_page: int):
        self.max_pages, self.P = max_pages, tokens_per_page
        self.owned = [False] * max_pages
        self.shadow: list[int] = []
        self.synced = 0
        self.uploads = 0  # number of H2D copies the allocator would issue

    def ensure_pages_for(self, total_tokens: int) -> str:
        needed = -(-total_tokens // self.P)
        if needed > self.max_pages:
            return "OOM"
        while len(self.shadow) < needed:
            page = self.owned.index(False)
            self.owned[page] = True
            self.shadow.append(page)
        if len(self.shadow) > self.synced:
            self.synced = len(self.shadow)
            self.uploads += 1
        return "OK"

    def release_all(self):
        self.owned = [False] * self.max_pages
        self.shadow = []
        self.synced = 0


class SharedPoolModel:
    """Model of the shared multi-session pool (lowest free id, per-session
    free)."""

    def __init__(self, max_pages: int, P: int, sessions: int):
        self.max_pages, self.P = max_pages, P
        self.used = [False] * max_pages
        self.tables = [[] for _ in range(sessions)]

    def ensure(self, sid: int, total_tokens: int) -> str:
        t = self.tables[sid]
        needed = -(-total_tokens // self.P)
        if needed - len(t) > self.used.count(False):
            return "OOM"
        while len(t) < needed:
            page = self.used.index(False)
            self.used[page] = True
            t.append(page)
        return "OK"

    def release(self, sid: int):
        for p in self.tables[sid]:
            self.used[p] = False
        self.tables[sid] = []


# ---------------- numeric wrappers ----------------

def rope_sincos(angles: np.ndarray):
    a = np.ascontiguousarray(angles, dtype=np.float32)
    c = np.empty_like(a)
    s = np.empty_like(a)
    lib().orc_rope_sincos_batch(_p(a), a.size, _p(c), _p(s))
    return c, s


def inv_freq(theta: float) -> np.ndarray:
    out = np.empty(64, dtype=np.float32)
    lib().orc_inv_freq(float(theta), _p(out))
    return out


def rope_append(qkv: np.ndarray, tokens, base_pos, layer, pt, P, maxp, theta, mode,
                pool: np.ndarray, written: np.ndarray | None = None):
    """In-place on qkv (uint16 [T][2560]) and pool (uint16). mode 0 = the
    reference double oracle, mode 1 = the kernel-exact fp32 statement."""
    pt = np.ascontiguousarray(pt, dtype=np.uint32)
    lib().orc_rope_append(_p(qkv), tokens, base_pos, layer, _p(pt), P, maxp,
                          float(theta), mode, _p(pool),
                          None if written is None else _p(written))


def attn_ref(q_rows, tokens, base_pos, layer, pool, pt, P, maxp, threads=None):
    out = np.zeros((tokens, 2048), dtype=np.uint16)
    pt = np.ascontiguousarray(pt, dtype=np.uint32)
    lib().orc_attn_ref(_p(np.ascontiguousarray(q_rows)), tokens, base_pos, layer,
                       _p(pool), _p(pt), P, maxp, _p(out), threads or os.cpu_count() or 1)
    return out


def decode_chunks(q_row, limit, layer, pool, pt, P, maxp, C_, NC, fp32_p=False):
    """Per-chunk partials [16][NC][130] (and the direct output when
    limit < C_); fp32_p selects fp32 P in P.V instead of bf16-rounded P."""
    parts = np.full((16, NC, PSTRIDE), np.nan, dtype=np.float32)
    out = np.zeros(2048, dtype=np.uint16)
    pt = np.ascontiguousarray(pt, dtype=np.uint32)
    lib().orc_decode_chunks_p(_p(np.ascontiguousarray(q_row)), limit, layer, _p(pool),
                              _p(pt), P, maxp, C_, NC, _p(parts), _p(out),
                              1 if fp32_p else 0)
    return parts, out


def merge2(parts: np.ndarray, NC: int, n_valid: int):
    parts = np.ascontiguousarray(parts, dtype=np.float32)
    lvl2 = np.zeros((16, SPLIT2, PSTRIDE), dtype=np.float32)
    out = np.zeros(2048, dtype=np.uint16)
    lib().orc_merge2(_p(parts), NC, n_valid, _p(lvl2), _p(out))
    return lvl2, out


def decode_cpu_mt(q_rows, limits, page_tables, pool, layer, P, maxp, threads):
    """Multi-threaded fp32 CPU decode of B sessions (reported baseline)."""
    B = len(limits)
    lim = np.ascontiguousarray(limits, dtype=np.uint32)
    tabs = [np.ascontiguousarray(t, dtype=np.uint32) for t in page_tables]
    ptrs = (C.c_void_p * B)(*[t.ctypes.data for t in tabs])
    out = np.zeros((B, 2048), dtype=np.uint16)
    lib().orc_decode_cpu_mt(_p(np.ascontiguousarray(q_rows)), _p(lim), ptrs, _p(pool),
                            layer, P, maxp, B, _p(out), threads)
    return out


# ---------------- comparison statistics ----------------

def compare_bf16(got, ref):
    """relL2 / cosine / max-abs / mean-abs of two bf16 arrays (as float)."""
    a = bf16_to_f32(got).astype(np.float64).ravel()
    r = bf16_to_f32(ref).astype(np.float64).ravel()
    d = a - r
    rr = float((r * r).sum())
    aa = float((a * a).sum())
    return {
        "rel_l2": math.sqrt(float((d * d).sum()) / (rr if rr > 0 else 1.0)),
        "cos": float((a * r).sum() / math.sqrt(aa * rr)) if aa * rr > 0 else 1.0,
        "max_abs": float(np.abs(d).max()) if d.size else 0.0,
        "mean_abs": float(np.abs(d).mean()) if d.size else 0.0,
    }


def bf16_ulp(x):
    """Spacing of bf16 at |x| (for ulp tolerances)."""
    x = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(x, 2.0 ** -126)))
    return 2.0 ** (e - 7)
