"""Python binding of the mc_* session ABI (include/minicpm_runtime.h).

Mirrors what the reference's Rust wrapper does over dlopen
(rust/minicpm-runtime/src/native.rs:42-94,386-525): POD option structs with
struct_size/abi_version, by-value opaque handles, mc_last_error() on failure.
"""
from __future__ import annotations

import ctypes as C

from ._native import McError, check, lib, LayoutT

MC_ABI_VERSION = 0x00020000
EOS_STREAM_ID = 130073
VOCAB = 130560


class ModelOptions(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_version", C.c_uint32),
                ("device_id", C.c_int32), ("max_sessions", C.c_uint32),
                ("max_context_tokens", C.c_uint32), ("precision", C.c_int),
                ("kv_precision", C.c_int), ("enable_cuda_graph", C.c_uint32),
                ("reserve_vram_bytes", C.c_uint64)]


class GenerationConfig(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("max_new_tokens", C.c_uint32),
                ("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_uint32),
                ("repetition_penalty", C.c_float), ("seed", C.c_uint64)]


class RuntimeStats(C.Structure):
    _fields_ = [("prompt_tokens", C.c_uint64), ("generated_tokens", C.c_uint64),
                ("prefill_us", C.c_uint64), ("decode_us", C.c_uint64),
                ("peak_vram_bytes", C.c_uint64), ("cuda_graph_launches", C.c_uint64)]


class BatchOptions(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_version", C.c_uint32),
                ("max_slots", C.c_uint32), ("max_context_tokens", C.c_uint32),
                ("reserved", C.c_uint32 * 4)]


class Handle(C.Structure):
    _fields_ = [("impl", C.c_void_p)]


assert C.sizeof(ModelOptions) == 40 and C.sizeof(GenerationConfig) == 32
assert C.sizeof(BatchOptions) == 32

_P = C.c_void_p
_bound = False


def _bind():
    global _bound
    if _bound:
        return lib()
    L = lib()
    sig = {
        "mc_model_load": (C.c_int, [C.c_char_p, C.POINTER(ModelOptions), C.POINTER(Handle)]),
        "mc_model_destroy": (None, [Handle]),
        "mc_session_create": (C.c_int, [Handle, C.POINTER(Handle)]),
        "mc_session_reset": (C.c_int, [Handle]),
        "mc_session_destroy": (None, [Handle]),
        "mc_prefill": (C.c_int, [Handle, C.POINTER(C.c_int32), C.c_uint32]),
        "mc_decode_one": (C.c_int, [Handle, C.POINTER(GenerationConfig),
                                    C.POINTER(C.c_int32)]),
        "mc_get_stats": (C.c_int, [Handle, C.POINTER(RuntimeStats)]),
        "mc_batch_group_create": (C.c_int, [Handle, C.POINTER(BatchOptions),
                                            C.POINTER(Handle)]),
        "mc_batch_group_add": (C.c_int, [Handle, Handle, C.POINTER(C.c_uint32)]),
        "mc_batch_group_remove": (C.c_int, [Handle, C.c_uint32]),
        "mc_batch_step": (C.c_int, [Handle, C.POINTER(C.c_uint32), C.c_uint32,
                                    C.POINTER(GenerationConfig), C.POINTER(C.c_int32)]),
        "mc_batch_group_destroy": (None, [Handle]),
        "mc_debug_session_info": (C.c_int, [Handle, C.POINTER(C.c_uint32),
                                            C.POINTER(C.c_uint32), C.POINTER(LayoutT),
                                            C.POINTER(_P), C.POINTER(_P)]),
        "mc_debug_session_seq": (C.c_int, [Handle, C.POINTER(C.c_int32), C.c_uint32]),
        "mc_debug_session_arena_bytes": (C.c_size_t, [Handle]),
        "mc_debug_session_attn_chunk": (C.c_uint32, [Handle]),
        "mc_debug_session_set_graph_enabled": (None, [Handle, C.c_int]),
        "mc_debug_session_graph_nodes": (C.c_size_t, [Handle]),
        "mc_debug_session_rope_intact": (C.c_int, [Handle]),
        "mc_debug_seed_residual": (C.c_int, [Handle, C.c_void_p, C.c_uint32]),
        "mc_debug_dump_set_steps": (None, [C.c_int]),
        "mc_debug_breakdown_raw_segments": (C.c_int, [Handle]),
        "mc_debug_breakdown_collect": (C.c_int, [Handle, C.POINTER(C.c_double), C.c_int]),
        "mc_debug_batch_group_stats": (C.c_int, [Handle, C.POINTER(C.c_uint64),
                                                 C.POINTER(C.c_uint64), C.POINTER(C.c_uint32)]),
        "mc_debug_batch_breakdown_collect": (C.c_int, [Handle, C.POINTER(C.c_double),
                                                       C.c_int]),
        "mc_debug_session_last_logits": (C.c_int, [Handle, C.POINTER(C.c_float)]),
        "mc_debug_batch_last_logits": (C.c_int, [Handle, C.c_uint32, C.POINTER(C.c_float)]),
    }
    for n, (r, a) in sig.items():
        f = getattr(L, n)
        f.restype, f.argtypes = r, a
    _bound = True
    return L


def model_options(max_context_tokens=2048, max_sessions=4, device_id=0, **kw) -> ModelOptions:
    o = ModelOptions(C.sizeof(ModelOptions), MC_ABI_VERSION, device_id, max_sessions,
                     max_context_tokens, 0, 0, 0, 0)
    for k, v in kw.items():
        setattr(o, k, v)
    return o


def gen_config(max_new_tokens=64, temperature=0.0, top_k=1, seed=0, **kw) -> GenerationConfig:
    c = GenerationConfig(C.sizeof(GenerationConfig), max_new_tokens, temperature, 1.0, top_k,
                         1.0, seed)
    for k, v in kw.items():
        setattr(c, k, v)
    return c


class Model:
    def __init__(self, model_dir: str, options: ModelOptions):
        L = _bind()
        self.h = Handle()
        check(L.mc_model_load(model_dir.encode(), C.byref(options), C.byref(self.h)),
              "mc_model_load")

    def close(self):
        if self.h.impl:
            _bind().mc_model_destroy(self.h)
            self.h = Handle()


class Session:
    def __init__(self, model: Model):
        L = _bind()
        self.h = Handle()
        check(L.mc_session_create(model.h, C.byref(self.h)), "mc_session_create")

    def prefill(self, tokens) -> None:
        arr = (C.c_int32 * len(tokens))(*tokens)
        check(_bind().mc_prefill(self.h, arr, len(tokens)), "mc_prefill")

    def decode_one(self, cfg: GenerationConfig) -> int:
        out = C.c_int32()
        check(_bind().mc_decode_one(self.h, C.byref(cfg), C.byref(out)), "mc_decode_one")
        return out.value

    def reset(self) -> None:
        check(_bind().mc_session_reset(self.h), "mc_session_reset")

    def stats(self) -> RuntimeStats:
        st = RuntimeStats()
        check(_bind().mc_get_stats(self.h, C.byref(st)), "mc_get_stats")
        return st

    def info(self):
        seq, pages, lay, pool, pt = C.c_uint32(), C.c_uint32(), LayoutT(), _P(), _P()
        check(_bind().mc_debug_session_info(self.h, C.byref(seq), C.byref(pages),
                                            C.byref(lay), C.byref(pool), C.byref(pt)),
              "mc_debug_session_info")
        return {"seq_len": seq.value, "pages_owned": pages.value, "layout": lay,
                "d_pool": pool.value, "d_page_table": pt.value}

    def seq(self, n: int):
        out = (C.c_int32 * n)()
        check(_bind().mc_debug_session_seq(self.h, out, n), "mc_debug_session_seq")
        return list(out)

    def arena_bytes(self) -> int:
        return int(_bind().mc_debug_session_arena_bytes(self.h))

    def attn_chunk(self) -> int:
        return int(_bind().mc_debug_session_attn_chunk(self.h))

    def set_graph_enabled(self, enabled: bool) -> None:
        """Graph A/B switch: False runs decode steps eagerly although the
        model was loaded with graphs on (session.cpp:636-641)."""
        _bind().mc_debug_session_set_graph_enabled(self.h, 1 if enabled else 0)

    def graph_nodes(self) -> int:
        """Nodes of the captured decode-step graph (0 before the first graph
        step)."""
        return int(_bind().mc_debug_session_graph_nodes(self.h))

    def rope_intact(self) -> int:
        """1 when the RoPE table equals its create-time snapshot, 0 when it
        was overwritten, -1 without a session/snapshot, -2 on a HIP error
        (session.cpp:668-686)."""
        return int(_bind().mc_debug_session_rope_intact(self.h))

    def seed_residual(self, rows_bf16) -> None:
        """mc_debug_seed_residual: rows x 2048 bf16 (uint16 numpy) into the
        session's residual rows (debug_dump.cpp:159-199)."""
        import numpy as np
        a = np.ascontiguousarray(rows_bf16, dtype=np.uint16)
        check(_bind().mc_debug_seed_residual(self.h, a.ctypes.data, a.size // 2048),
              "mc_debug_seed_residual")

    def last_logits(self):
        """bf16 logits (as float32 numpy) of the session's last forward (a
        model loaded with weights)."""
        import numpy as np
        out = np.empty(VOCAB, dtype=np.float32)
        check(_bind().mc_debug_session_last_logits(
            self.h, out.ctypes.data_as(C.POINTER(C.c_float))), "mc_debug_session_last_logits")
        return out

    def breakdown(self):
        """Segment times (ms) of the last decode step, or an int status
        (0 = MC_BREAKDOWN was not set at create, < 0 = error)."""
        L = _bind()
        n = L.mc_debug_breakdown_raw_segments(self.h)
        if n <= 0:
            return n
        out = (C.c_double * n)()
        r = L.mc_debug_breakdown_collect(self.h, out, n)
        return list(out) if r == n else r

    def close(self):
        if self.h.impl:
            _bind().mc_session_destroy(self.h)
            self.h = Handle()


class BatchGroup:
    def __init__(self, model: Model, max_slots: int, max_context_tokens: int, reserved=None):
        L = _bind()
        o = BatchOptions(C.sizeof(BatchOptions), MC_ABI_VERSION, max_slots,
                         max_context_tokens, (C.c_uint32 * 4)(*(reserved or [0, 0, 0, 0])))
        self.h = Handle()
        check(L.mc_batch_group_create(model.h, C.byref(o), C.byref(self.h)),
              "mc_batch_group_create")

    def add(self, s: Session) -> int:
        slot = C.c_uint32()
        check(_bind().mc_batch_group_add(self.h, s.h, C.byref(slot)), "mc_batch_group_add")
        return slot.value

    def remove(self, slot: int) -> None:
        check(_bind().mc_batch_group_remove(self.h, slot), "mc_batch_group_remove")

    def step(self, slots, cfgs):
        n = len(slots)
        ids = (C.c_uint32 * n)(*slots)
        cf = (GenerationConfig * n)(*cfgs)
        out = (C.c_int32 * n)()
        check(_bind().mc_batch_step(self.h, ids, n, cf, out), "mc_batch_step")
        return list(out)

    def stats(self):
        steps, us, members = C.c_uint64(), C.c_uint64(), C.c_uint32()
        check(_bind().mc_debug_batch_group_stats(self.h, C.byref(steps), C.byref(us),
                                                 C.byref(members)), "mc_debug_batch_group_stats")
        return {"steps": steps.value, "decode_us": us.value, "members": members.value}

    def last_logits(self, slot: int):
        """bf16 logits (as float32 numpy) of `slot` in the last step."""
        import numpy as np
        out = np.empty(VOCAB, dtype=np.float32)
        check(_bind().mc_debug_batch_last_logits(
            self.h, slot, out.ctypes.data_as(C.POINTER(C.c_float))), "mc_debug_batch_last_logits")
        return out

    def breakdown(self):
        """Per-bucket times (ms) of the last step, or an int status."""
        L = _bind()
        n = L.mc_debug_breakdown_bucket_count()
        out = (C.c_double * n)()
        r = L.mc_debug_batch_breakdown_collect(self.h, out, n)
        return list(out) if r == n else r

    def close(self):
        if self.h.impl:
            _bind().mc_batch_group_destroy(self.h)
            self.h = Handle()


__all__ = ["Model", "Session", "BatchGroup", "model_options", "gen_config", "McError",
           "EOS_STREAM_ID"]


def dump_set_steps(steps: int) -> None:
    """mc_debug_dump_set_steps: the debug dump's step limit (effective only
    when MC_DEBUG_DUMP_DIR was set when the library first checked it)."""
    _bind().mc_debug_dump_set_steps(int(steps))
