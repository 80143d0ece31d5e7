"""Argument validation of every C-ABI entry point, without a GPU: invalid
arguments return MC_E_INVALID_ARGUMENT (1) with a message from mc_last_error()
before any device work; NULL handles are rejected or ignored as the reference
ABI documents (minicpm_runtime.h: destroy functions accept NULL)."""
import ctypes as C

import pytest

INV = 1
FAKE = 0x1000  # never dereferenced: validation fails before any device access


@pytest.fixture(scope="module")
def lib(pkg):
    return pkg._native.lib()


def lay(pkg, maxp=8, P=32, L=2, reserved=0):
    return pkg._native.LayoutT(maxp, P, L, reserved)


def good_decode_args(pkg):
    return [FAKE, FAKE, 0, FAKE, FAKE, lay(pkg), FAKE, 12, FAKE, None, None, 64, None]


@pytest.mark.parametrize("field,value", [
    (0, None), (1, None), (3, None), (4, None), (6, None), (8, None),  # NULL pointers
    (2, 2),             # layer >= num_layers
    (7, 0), (7, 4096),  # max_chunks out of range
    (11, 8), (11, 40),  # chunk_pos not a multiple of 16
])
def test_decode_rejects(pkg, lib, field, value):
    args = good_decode_args(pkg)
    args[field] = value
    assert lib.mc_kv_attention_decode(*args) == INV
    assert b"mc_kv_attention_decode" in lib.mc_last_error()


@pytest.mark.parametrize("bad", [dict(P=48), dict(P=0), dict(P=8192), dict(maxp=0),
                                 dict(L=0), dict(reserved=1)])
def test_bad_layouts_rejected_everywhere(pkg, lib, bad):
    L = lay(pkg, **bad)
    assert lib.mc_kv_attention_decode(FAKE, FAKE, 0, FAKE, FAKE, L, FAKE, 12, FAKE, None,
                                      None, 64, None) == INV
    assert lib.mc_kv_attention_decode_chunks(FAKE, FAKE, 0, FAKE, FAKE, L, FAKE, 12, FAKE,
                                             None, None, 64) == INV
    assert lib.mc_kv_rope_append(FAKE, 1, FAKE, 0, FAKE, FAKE, L, 5e6, None, None) == INV
    assert lib.mc_kv_attention_prefill(FAKE, 1, FAKE, 0, FAKE, FAKE, L, FAKE, None, 1,
                                       None) == INV
    assert lib.mc_kv_elem_offset(L, 0, 0, 0, 0, 0, 0) == 2 ** 64 - 1


def test_batch_and_merge_rejects(pkg, lib):
    L = lay(pkg)
    ok = [FAKE, FAKE, 4, 0, FAKE, FAKE, L, FAKE, 12, FAKE, None, None, 64, None]
    for i, v in [(2, 0), (2, 65), (0, None), (1, None), (4, None), (5, None), (7, None),
                 (9, None), (3, 5)]:
        a = list(ok)
        a[i] = v
        assert lib.mc_kv_attention_decode_batch(*a) == INV, (i, v)
    assert lib.mc_kv_attention_decode_merge(None, FAKE, 12, 64, None, FAKE, None) == INV
    assert lib.mc_kv_attention_decode_merge(FAKE, FAKE, 12, 24, None, FAKE, None) == INV


def test_prefill_and_rope_rejects(pkg, lib):
    L = lay(pkg)
    # tokens 0, S_kv 0 / 9, S_kv > 1 without partials, layer out of range
    assert lib.mc_kv_attention_prefill(FAKE, 0, FAKE, 0, FAKE, FAKE, L, FAKE, None, 1,
                                       None) == INV
    assert lib.mc_kv_attention_prefill(FAKE, 5, FAKE, 0, FAKE, FAKE, L, FAKE, None, 0,
                                       None) == INV
    assert lib.mc_kv_attention_prefill(FAKE, 5, FAKE, 0, FAKE, FAKE, L, FAKE, FAKE, 9,
                                       None) == INV
    assert lib.mc_kv_attention_prefill(FAKE, 5, FAKE, 0, FAKE, FAKE, L, FAKE, None, 2,
                                       None) == INV
    assert lib.mc_kv_attention_prefill(FAKE, 5, FAKE, 2, FAKE, FAKE, L, FAKE, None, 1,
                                       None) == INV
    assert lib.mc_kv_rope_append(FAKE, 0, FAKE, 0, FAKE, FAKE, L, 5e6, None, None) == INV
    assert lib.mc_kv_rope_append(FAKE, 1, FAKE, 0, FAKE, FAKE, L, 0.0, None, None) == INV
    assert lib.mc_kv_rope_append(FAKE, 1, FAKE, 2, FAKE, FAKE, L, 5e6, None, None) == INV
    assert lib.mc_kv_rope_inv_freq_init(None, 5e6, None) == INV
    assert lib.mc_kv_rope_inv_freq_init(FAKE, -1.0, None) == INV
    assert lib.mc_kv_decode_advance(None, FAKE, FAKE, None) == INV
    assert lib.mc_kv_batch_advance(FAKE, FAKE, FAKE, 0, None) == INV


def test_allocator_and_pool_rejects(pkg, lib):
    h = C.c_void_p()
    assert lib.mc_kv_allocator_create(None, 8, 32, C.byref(h)) == 0  # host-only allocator
    lib.mc_kv_allocator_destroy(h)
    assert lib.mc_kv_allocator_create(FAKE, 8, 48, C.byref(h)) == INV
    assert lib.mc_kv_allocator_create(FAKE, 0, 32, C.byref(h)) == INV
    assert lib.mc_kv_allocator_create(FAKE, 8, 32, None) == INV
    assert lib.mc_kv_allocator_ensure_pages_for(None, 5, None) == INV
    assert lib.mc_kv_pool_create(8, 48, 2, C.byref(h)) == INV
    assert lib.mc_kv_pool_create(8, 32, 0, C.byref(h)) == INV
    assert lib.mc_kv_pool_ensure(None, 0, 5, None, None) == INV
    assert lib.mc_kv_pool_release(None, 0) == INV
    # destroy / release / queries with NULL are harmless
    lib.mc_kv_allocator_destroy(None)
    lib.mc_kv_allocator_release_all(None)
    lib.mc_kv_pool_destroy(None)
    assert lib.mc_kv_allocator_pages_owned(None) == 0
    assert lib.mc_kv_pool_pages_free(None) == 0


def test_session_abi_null_handles(pkg):
    rt = __import__("importlib").import_module("minicpm5-5080fast_amd.runtime")
    L = rt._bind()
    null = rt.Handle()
    opts = rt.model_options()
    assert L.mc_model_load(None, C.byref(opts), C.byref(rt.Handle())) == INV
    assert L.mc_model_load(b"/tmp", None, C.byref(rt.Handle())) == INV
    assert L.mc_model_load(b"/tmp", C.byref(opts), None) == INV
    assert L.mc_session_create(null, C.byref(rt.Handle())) == INV
    assert L.mc_session_reset(null) == INV
    arr = (C.c_int32 * 1)(5)
    assert L.mc_prefill(null, arr, 1) == INV
    cfg = rt.gen_config()
    out = C.c_int32()
    assert L.mc_decode_one(null, C.byref(cfg), C.byref(out)) == INV
    assert L.mc_get_stats(null, C.byref(rt.RuntimeStats())) == INV
    bo = rt.BatchOptions(C.sizeof(rt.BatchOptions), rt.MC_ABI_VERSION, 2, 2048,
                         (C.c_uint32 * 4)())
    assert L.mc_batch_group_create(null, C.byref(bo), C.byref(rt.Handle())) == INV
    slot = C.c_uint32()
    assert L.mc_batch_group_add(null, null, C.byref(slot)) == INV
    assert L.mc_batch_group_remove(null, 0) == INV
    ids = (C.c_uint32 * 1)(0)
    cfgs = (rt.GenerationConfig * 1)(cfg)
    outs = (C.c_int32 * 1)()
    assert L.mc_batch_step(null, ids, 1, cfgs, outs) == INV
    L.mc_model_destroy(null)
    L.mc_session_destroy(null)
    L.mc_batch_group_destroy(null)
    assert L.mc_last_error()


def test_debug_hooks_without_handles(pkg, lib):
    """The debug hooks validate their handles without touching a device."""
    assert lib.mc_debug_breakdown_bucket_count() == 3
    assert lib.mc_debug_breakdown_bucket_name(0) == b"qkv(synthetic or norm1+projection)"
    assert lib.mc_debug_breakdown_bucket_name(3) is None
    assert lib.mc_debug_breakdown_bucket_of(-1) == -1
    lib.mc_debug_breakdown_collect.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
    assert lib.mc_debug_breakdown_collect(None, None, 0) == -1
    lib.mc_debug_batch_breakdown_collect.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
    assert lib.mc_debug_batch_breakdown_collect(None, None, 3) == -1
    lib.mc_debug_batch_group_stats.argtypes = [C.c_void_p] * 4
    assert lib.mc_debug_batch_group_stats(None, None, None, None) == INV
    lib.mc_debug_session_arena_bytes.restype = C.c_size_t
    lib.mc_debug_session_arena_bytes.argtypes = [C.c_void_p]
    assert lib.mc_debug_session_arena_bytes(None) == 0
    lib.mc_kv_debug_decode_timeline.argtypes = [C.c_void_p, C.c_uint32]
    assert lib.mc_kv_debug_decode_timeline(None, 4) == INV
    assert b"both or neither" in lib.mc_last_error()
    assert lib.mc_kv_debug_decode_timeline(C.c_void_p(0x1000), 0) == INV
    assert lib.mc_kv_debug_decode_timeline(None, 0) == 0  # detach: no device needed


def test_weight_path_kernels_reject(pkg, lib):
    """The GEMV and row-GEMM entry points check rows, shapes and strides
    before any device work."""
    F = FAKE
    # mc_model_gemv: M 1..8, K 2048 or 6144, strides
    assert lib.mc_model_gemv(F, F, 2048, F, 2048, 0, 2048, 2048, None) == INV
    assert lib.mc_model_gemv(F, F, 2048, F, 2048, 9, 2048, 2048, None) == INV
    assert lib.mc_model_gemv(F, F, 4096, F, 2048, 1, 2048, 4096, None) == INV
    assert lib.mc_model_gemv(F, F, 2000, F, 2048, 1, 2048, 2048, None) == INV
    assert lib.mc_model_gemv(None, F, 2048, F, 2048, 1, 2048, 2048, None) == INV
    # mc_model_gemm_rows: M 9..32, N % 16, K 2048 / 6144 (2048 with swiglu),
    # swiglu 0/1, strides
    good = [F, F, 2048, F, 2048, 20, 2048, 2048, 0, None]
    for i, v in [(5, 8), (5, 33), (6, 2050), (7, 4096), (2, 2040), (4, 2000), (2, 2052),
                 (8, 2), (0, None), (1, None), (3, None)]:
        a = list(good)
        a[i] = v
        assert lib.mc_model_gemm_rows(*a) == INV, (i, v)
        assert b"mc_model_gemm_rows" in lib.mc_last_error()
    assert lib.mc_model_gemm_rows(F, F, 6144, F, 2048, 20, 2048, 6144, 1, None) == INV
    for i, v in [(0, F + 8), (1, F + 8), (3, F + 4)]:  # misaligned w, x, y
        a = list(good)
        a[i] = v
        assert lib.mc_model_gemm_rows(*a) == INV, (i, v)
