"""Host-side mirror of the reference's KV-path launcher interface.

Names, argument meaning and error behaviour follow the reference launchers in
native/kernels/sm120/kernels.h (launch_rope_kv :214-225, launch_rope_inv_freq_init
:229-230, launch_attention_decode :369-388, launch_attention_decode_merge
:394-400, launch_attention_decode_batch :465-480, launch_attn_prefill_flash
:575-585, launch_decode_advance :632-635, launch_batch_advance :651-655) and the
PagedKvAllocator of native/runtime/kv_cache.h:68-104. Device buffers are torch
tensors (plumbing only); every call goes through the C ABI of
libminicpm_native.so and raises McError on a non-OK status, carrying the
library's mc_last_error() text.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._native import McError, check, lib, LayoutT

Q_HEADS, KV_HEADS, HEAD_DIM, QKV_ROW = 16, 2, 128, 2560
PARTIAL_STRIDE, MERGE_SPLIT2 = 130, 32


def _ptr(t):
    if t is None:
        return None
    return C.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is None:
        import torch
        return C.c_void_p(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, int):
        return C.c_void_p(stream)
    return C.c_void_p(stream.cuda_stream)


@dataclass(frozen=True)
class KvLayout:
    """Pool geometry (reference KvLayout, kv_cache.h:29-66, with P and L as
    runtime values)."""
    max_pages: int
    tokens_per_page: int = 32
    num_layers: int = 42

    def c(self) -> LayoutT:
        return LayoutT(self.max_pages, self.tokens_per_page, self.num_layers, 0)

    def elem_offset(self, layer, page, slot, kv, head, d) -> int:
        return int(lib().mc_kv_elem_offset(self.c(), layer, page, slot, kv, head, d))

    def total_elems(self) -> int:
        return int(lib().mc_kv_total_elems(self.c()))

    def page_index(self, pos: int) -> int:
        return pos // self.tokens_per_page

    def slot_index(self, pos: int) -> int:
        return pos % self.tokens_per_page


def attention_decode_chunk_pos(max_ctx: int) -> int:
    return int(lib().mc_kv_decode_chunk_pos(max_ctx))


def attention_decode_max_chunks(max_ctx: int, chunk: int = 64) -> int:
    return int(lib().mc_kv_decode_max_chunks(max_ctx, chunk))


def prefill_flash_split_kv(tokens: int) -> int:
    return int(lib().mc_kv_prefill_split_kv(tokens))


# ---------------- kernels ----------------

def launch_rope_inv_freq_init(d_table, rope_theta: float, stream=None) -> None:
    check(lib().mc_kv_rope_inv_freq_init(_ptr(d_table), float(rope_theta),
                                         _stream(stream)), "launch_rope_inv_freq_init")


def launch_rope_kv(d_qkv, tokens, d_base_pos, layer, d_page_table, d_kv_pool,
                   layout: KvLayout, rope_theta, stream=None, d_inv_freq=None) -> None:
    check(lib().mc_kv_rope_append(_ptr(d_qkv), tokens, _ptr(d_base_pos), layer,
                                  _ptr(d_page_table), _ptr(d_kv_pool), layout.c(),
                                  float(rope_theta), _ptr(d_inv_freq), _stream(stream)),
          "launch_rope_kv")


def launch_attention_decode(d_q_rows, d_pos, layer, d_page_table, d_kv_pool,
                            layout: KvLayout, d_partials, max_chunks, d_out, stream=None,
                            d_inv_freq=None, chunk_pos=64, d_partials2=None) -> None:
    check(lib().mc_kv_attention_decode(_ptr(d_q_rows), _ptr(d_pos), layer,
                                       _ptr(d_page_table), _ptr(d_kv_pool), layout.c(),
                                       _ptr(d_partials), max_chunks, _ptr(d_out),
                                       _stream(stream), _ptr(d_inv_freq), chunk_pos,
                                       _ptr(d_partials2)), "launch_attention_decode")


def launch_attention_decode_noalloc(d_q_rows, d_pos, layer, d_page_table, d_kv_pool,
                                    layout: KvLayout, max_chunks, d_out, stream=None,
                                    d_inv_freq=None, chunk_pos=64) -> None:
    """Decode without caller scratch (records in a library-owned device array;
    calls overlapping on one device race). No reference counterpart."""
    check(lib().mc_kv_attention_decode_noalloc(_ptr(d_q_rows), _ptr(d_pos), layer,
                                               _ptr(d_page_table), _ptr(d_kv_pool),
                                               layout.c(), max_chunks, _ptr(d_out),
                                               _stream(stream), _ptr(d_inv_freq), chunk_pos),
          "launch_attention_decode_noalloc")


def launch_attention_decode_chunks(d_q_rows, d_pos, layer, d_page_table, d_kv_pool,
                                   layout: KvLayout, d_partials, max_chunks, d_out,
                                   stream=None, d_inv_freq=None, chunk_pos=64) -> None:
    check(lib().mc_kv_attention_decode_chunks(_ptr(d_q_rows), _ptr(d_pos), layer,
                                              _ptr(d_page_table), _ptr(d_kv_pool),
                                              layout.c(), _ptr(d_partials), max_chunks,
                                              _ptr(d_out), _stream(stream),
                                              _ptr(d_inv_freq), chunk_pos),
          "launch_attention_decode_chunks")


def launch_attention_decode_merge(d_partials, d_pos, max_chunks, chunk_pos, d_partials2,
                                  d_out, stream=None) -> None:
    check(lib().mc_kv_attention_decode_merge(_ptr(d_partials), _ptr(d_pos), max_chunks,
                                             chunk_pos, _ptr(d_partials2), _ptr(d_out),
                                             _stream(stream)),
          "launch_attention_decode_merge")


def launch_attention_decode_batch(d_q_rows, d_slot_pos, B, layer, d_slot_pt, d_slot_kv,
                                  layout: KvLayout, d_partials, max_chunks, d_out,
                                  stream=None, d_inv_freq=None, chunk_pos=64,
                                  d_partials2=None) -> None:
    """d_slot_pos / d_slot_pt / d_slot_kv are device uint64 tensors of [B]
    pointers (the reference's per-slot device pointer tables)."""
    check(lib().mc_kv_attention_decode_batch(_ptr(d_q_rows), _ptr(d_slot_pos), B, layer,
                                             _ptr(d_slot_pt), _ptr(d_slot_kv),
                                             layout.c(), _ptr(d_partials), max_chunks,
                                             _ptr(d_out), _stream(stream),
                                             _ptr(d_inv_freq), chunk_pos,
                                             _ptr(d_partials2)),
          "launch_attention_decode_batch")


def launch_attn_prefill_flash(d_q_rows, tokens, d_base_pos, layer, d_page_table,
                              d_kv_pool, layout: KvLayout, d_out, d_partials, S_kv,
                              stream=None) -> None:
    check(lib().mc_kv_attention_prefill(_ptr(d_q_rows), tokens, _ptr(d_base_pos), layer,
                                        _ptr(d_page_table), _ptr(d_kv_pool), layout.c(),
                                        _ptr(d_out), _ptr(d_partials), S_kv,
                                        _stream(stream)), "launch_attn_prefill_flash")


PREFILL_SHAPE_AUTO = 0xFFFFFFFF


def debug_prefill_shape(shape: int) -> int:
    """Forces the prefill workgroup shape (0 = 32 rows, 1 = 16 rows on 4
    waves, 2 = 16 rows on two halves, PREFILL_SHAPE_AUTO = per launch) and
    returns the previous setting. Debug hook, no reference counterpart."""
    prev = C.c_uint32(0)
    check(lib().mc_kv_debug_prefill_shape(shape, C.byref(prev)), "debug_prefill_shape")
    return prev.value


def debug_prefill_packing(enable: bool) -> bool:
    """Turns the fixed prefill job packing on or off and returns the previous
    setting. Debug hook, no reference counterpart."""
    prev = C.c_uint32(0)
    check(lib().mc_kv_debug_prefill_packing(1 if enable else 0, C.byref(prev)),
          "debug_prefill_packing")
    return bool(prev.value)


def debug_prefill_status(reset: bool = False) -> int:
    """Number of two-half prefill barrier waits that ran out of their bound on
    the current device since the last reset (non-zero means a prefill output
    may be wrong); `reset` clears the count after reading. Synchronous.
    Debug hook, no reference counterpart."""
    n = C.c_uint32(0)
    check(lib().mc_kv_debug_prefill_status(C.byref(n), 1 if reset else 0),
          "debug_prefill_status")
    return n.value


def debug_prefill_force_timeouts(count: int) -> None:
    """Sets the device's half-barrier timeout count from the host (no kernel
    runs), so that a test can see the session prefill path report it."""
    check(lib().mc_kv_debug_prefill_force_timeouts(count), "debug_prefill_force_timeouts")


DECODE_FP32P_FROM_ENV = 0xFFFFFFFF


def debug_decode_fp32p(fp32_p: int) -> int:
    """Sets the decode P.V precision (0 = bf16 P, 1 = fp32 P,
    DECODE_FP32P_FROM_ENV = MC_ATTN_HMMA_OFF) and returns the previous
    setting. Debug hook (the reference selects fp32 P by environment only)."""
    prev = C.c_uint32(0)
    check(lib().mc_kv_debug_decode_fp32p(fp32_p, C.byref(prev)), "debug_decode_fp32p")
    return prev.value


def debug_decode_records_only(enable: bool) -> bool:
    """Measurement switch: decode launches run only the chunk kernel (no
    merge, no output). Returns the previous setting. Debug hook."""
    prev = C.c_uint32(0)
    check(lib().mc_kv_debug_decode_records_only(1 if enable else 0, C.byref(prev)),
          "debug_decode_records_only")
    return bool(prev.value)


TIMELINE_WORDS = 36864  # uint64 words per decode launch (MC_KV_TIMELINE_WORDS)
TIMELINE_CHUNK_WGS = 8192
TIMELINE_MERGE_WGS = 2048


def debug_decode_timeline(d_stamps, launches: int) -> None:
    """Attaches (or, with None / 0, detaches) the decode timeline buffer:
    `launches` regions of TIMELINE_WORDS int64 words, one per decode in a
    ring. The caller zeroes the buffer. Debug hook."""
    check(lib().mc_kv_debug_decode_timeline(_ptr(d_stamps) if d_stamps is not None else None,
                                            launches), "debug_decode_timeline")


def timeline_summary(stamps) -> dict:
    """Per-decode timeline from a filled timeline buffer (numpy int64 array of
    launches * TIMELINE_WORDS words): the written regions ordered by chunk
    entry, each giving the chunk span (first workgroup entry to last wave
    exit), the median and latest workgroup entry, the per-XCC median exit
    range, the medians over workgroups of entry -> first K/V tile in registers
    and first tile -> exit, the gap to the merge's first entry, the merge
    span, and the gap to the next decode's chunk entry. Clock counts are
    10 ns; results in us."""
    import numpy as np
    st = np.asarray(stamps, dtype=np.int64).reshape(-1, TIMELINE_WORDS)
    recs = []
    for r in st:
        ck = r[:4 * TIMELINE_CHUNK_WGS].reshape(-1, 4)
        ck = ck[ck[:, 0] > 0]
        if len(ck) == 0:
            continue
        mg = r[4 * TIMELINE_CHUNK_WGS:].reshape(-1, 2)
        mg = mg[mg[:, 0] > 0]
        recs.append((ck, mg))
    recs.sort(key=lambda x: x[0][:, 0].min())
    rows = []
    for i, (ck, mg) in enumerate(recs):
        a, b = ck[:, 0].min(), ck[:, 1].max()
        xcc = [np.median(ck[ck[:, 2] == x, 1]) - a for x in np.unique(ck[:, 2])]
        row = {"chunk_span": (b - a) / 100, "median_wg_end": (np.median(ck[:, 1]) - a) / 100,
               "last_wg_entry": (ck[:, 0].max() - a) / 100,
               "xcc_median_end": [min(xcc) / 100, max(xcc) / 100], "workgroups": len(ck)}
        fd = ck[ck[:, 3] > 0]
        if len(fd):  # workgroup entry -> its first K/V tile in registers -> its exit
            row["wg_entry_to_first_data"] = float(np.median(fd[:, 3] - fd[:, 0])) / 100
            row["wg_first_data_to_exit"] = float(np.median(fd[:, 1] - fd[:, 3])) / 100
        end = b
        if len(mg):
            row["gap_to_merge"] = (mg[:, 0].min() - b) / 100
            row["merge_span"] = (mg[:, 1].max() - mg[:, 0].min()) / 100
            end = mg[:, 1].max()
        if i + 1 < len(recs):
            row["gap_to_next"] = (recs[i + 1][0][:, 0].min() - end) / 100
            row["decode_period"] = (recs[i + 1][0][:, 0].min() - a) / 100
        rows.append(row)
    out = {"decodes": len(rows)}
    for k in ("chunk_span", "median_wg_end", "last_wg_entry", "wg_entry_to_first_data",
              "wg_first_data_to_exit", "gap_to_merge", "merge_span", "gap_to_next",
              "decode_period"):
        v = [r[k] for r in rows if k in r]
        if v:
            out[k] = round(float(np.median(v)), 3)
    if rows:
        out["xcc_median_end"] = [round(float(np.median([r["xcc_median_end"][j] for r in rows])), 3)
                                 for j in (0, 1)]
    return out


def launch_decode_advance(d_seq, d_next_token, d_seq_len, stream=None) -> None:
    check(lib().mc_kv_decode_advance(_ptr(d_seq), _ptr(d_next_token), _ptr(d_seq_len),
                                     _stream(stream)), "launch_decode_advance")


def launch_batch_advance(d_slot_seq, d_slot_tok, d_slot_pos, n, stream=None) -> None:
    check(lib().mc_kv_batch_advance(_ptr(d_slot_seq), _ptr(d_slot_tok), _ptr(d_slot_pos),
                                    n, _stream(stream)), "launch_batch_advance")


# ---------------- allocators ----------------

class PagedKvAllocator:
    """Per-session page allocator (reference kv_cache.h:68-104) over the C ABI."""

    def __init__(self, d_table, max_pages: int, tokens_per_page: int = 32):
        h = C.c_void_p()
        check(lib().mc_kv_allocator_create(_ptr(d_table), max_pages, tokens_per_page,
                                           C.byref(h)), "PagedKvAllocator.init")
        self._h = h
        self.max_pages, self.tokens_per_page = max_pages, tokens_per_page

    def ensure_pages_for(self, total_tokens: int, stream=None) -> None:
        check(lib().mc_kv_allocator_ensure_pages_for(self._h, total_tokens,
                                                     _stream(stream)),
              "PagedKvAllocator.ensure_pages_for")

    def release_all(self) -> None:
        lib().mc_kv_allocator_release_all(self._h)

    def pages_owned(self) -> int:
        return int(lib().mc_kv_allocator_pages_owned(self._h))

    def pages_synced(self) -> int:
        return int(lib().mc_kv_allocator_pages_synced(self._h))

    def host_table(self) -> list[int]:
        n = self.pages_owned()
        buf = np.zeros(max(n, 1), dtype=np.uint32)
        k = lib().mc_kv_allocator_host_table(self._h, buf.ctypes.data_as(C.c_void_p), n)
        return buf[:k].tolist()

    def tokens_capacity(self) -> int:
        return self.max_pages * self.tokens_per_page

    def close(self):
        if self._h:
            lib().mc_kv_allocator_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class SharedPagePool:
    """Several sessions in one KV pool, pages freed per session and reused."""

    def __init__(self, max_pages: int, tokens_per_page: int, max_sessions: int):
        h = C.c_void_p()
        check(lib().mc_kv_pool_create(max_pages, tokens_per_page, max_sessions,
                                      C.byref(h)), "SharedPagePool.init")
        self._h = h

    def ensure(self, sid: int, total_tokens: int, d_table=None, stream=None) -> None:
        check(lib().mc_kv_pool_ensure(self._h, sid, total_tokens, _ptr(d_table),
                                      _stream(stream) if d_table is not None else None),
              "SharedPagePool.ensure")

    def release(self, sid: int) -> None:
        check(lib().mc_kv_pool_release(self._h, sid), "SharedPagePool.release")

    def pages_free(self) -> int:
        return int(lib().mc_kv_pool_pages_free(self._h))

    def table(self, sid: int) -> list[int]:
        n = int(lib().mc_kv_pool_session_pages(self._h, sid))
        buf = np.zeros(max(n, 1), dtype=np.uint32)
        k = lib().mc_kv_pool_session_table(self._h, sid, buf.ctypes.data_as(C.c_void_p), n)
        return buf[:k].tolist()

    def close(self):
        if self._h:
            lib().mc_kv_pool_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


__all__ = [n for n in dir() if n.startswith(("launch_", "attention_", "prefill_"))] + [
    "KvLayout", "PagedKvAllocator", "SharedPagePool", "McError"]
