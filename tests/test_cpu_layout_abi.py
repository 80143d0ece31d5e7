"""CPU tests: pool addressing and tier tables against the reference's
known-answer literals (tests/golden/kv_addressing.json), and the exported
C ABI of libminicpm_native.so (every function declared in include/*.h)."""
import json
import os
import re

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
GOLD = json.load(open(os.path.join(HERE, "golden", "kv_addressing.json")))


def test_elem_offset_literals_product(kvm):
    lay = kvm.KvLayout(GOLD["max_pages"], GOLD["tokens_per_page"], GOLD["num_layers"])
    for l, p, s, kv, h, d, want in GOLD["elem_offset"]:
        assert lay.elem_offset(l, p, s, kv, h, d) == want
    assert lay.total_elems() == GOLD["total_elems"]
    for pos, page, slot in GOLD["pos_to_page_slot"]:
        assert lay.page_index(pos) == page and lay.slot_index(pos) == slot


def test_elem_offset_literals_oracle(orc):
    for l, p, s, kv, h, d, want in GOLD["elem_offset"]:
        assert orc.kv_off(32, 256, l, p, s, kv, h, d) == want


def test_elem_offset_formula_general(kvm, orc):
    """Product == oracle for other page sizes / layer counts (P=64, L=28)."""
    for P in (1, 16, 32, 64, 128):
        for mp in (1, 8, 2048):
            lay = kvm.KvLayout(mp, P, 28)
            for l in (0, 13, 27):
                for page in (0, mp - 1):
                    for slot in (0, P - 1):
                        for kv in (0, 1):
                            for h in (0, 1):
                                for d in (0, 127):
                                    assert lay.elem_offset(l, page, slot, kv, h, d) == \
                                        orc.kv_off(P, mp, l, page, slot, kv, h, d)
            assert lay.total_elems() == mp * P * 512 * 28


def test_bad_layout_rejected(pkg):
    L = pkg._native
    assert L.lib().mc_kv_total_elems(L.layout(8, 48, 2)) == 0  # P not a power of two
    assert L.lib().mc_kv_elem_offset(L.layout(0, 32, 2), 0, 0, 0, 0, 0, 0) == 2 ** 64 - 1


def test_tier_tables(kvm, orc):
    # the library reads MC_ATTN_CHUNK512_ON / _OFF once per process; the
    # literals are the default table
    c512 = "MC_ATTN_CHUNK512_ON" in os.environ and "MC_ATTN_CHUNK512_OFF" not in os.environ
    for ctx, c in GOLD["chunk_pos_tiers"]:
        assert kvm.attention_decode_chunk_pos(ctx) == orc.chunk_pos(ctx, c512)
        assert orc.chunk_pos(ctx) == c
    assert kvm.attention_decode_max_chunks(131072, 256) == 512
    assert kvm.attention_decode_max_chunks(8448, 64) == 132
    for t, s in GOLD["prefill_split_kv"]:
        assert kvm.prefill_flash_split_kv(t) == s == orc.prefill_split_kv(t)


def _declared(header):
    txt = open(os.path.join(ROOT, "include", header)).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(mc_[a-z0-9_]+)\s*\(", txt)))


def test_all_declared_symbols_exported(pkg):
    import ctypes
    lib = ctypes.CDLL(pkg._native.LIB_PATH)
    names = _declared("minicpm_runtime.h") + _declared("mc_kv.h")
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_error_convention(pkg, kvm):
    """Invalid arguments return MC_E_INVALID_ARGUMENT with a message and no
    device work (runs without a GPU)."""
    with pytest.raises(pkg.McError) as e:
        kvm.launch_attention_decode(None, None, 0, None, None, kvm.KvLayout(8, 32, 1), None,
                                    12, None, stream=0)
    assert e.value.status == 1 and "invalid args" in str(e.value)
    with pytest.raises(pkg.McError) as e:
        kvm.launch_attn_prefill_flash(None, 0, None, 0, None, None, kvm.KvLayout(8, 32, 1),
                                      None, None, 9, stream=0)
    assert e.value.status == 1
    with pytest.raises(pkg.McError):
        kvm.launch_rope_kv(None, 1, None, 0, None, None, kvm.KvLayout(8, 32, 1), 5e6,
                           stream=0)


def test_prefill_debug_hooks(pkg, kvm):
    """The prefill shape and packing hooks (host state only, no GPU): a set
    returns the previous value, and an unknown shape is rejected."""
    prev = kvm.debug_prefill_shape(1)
    try:
        assert kvm.debug_prefill_shape(2) == 1
        with pytest.raises(pkg.McError) as e:
            kvm.debug_prefill_shape(3)
        assert e.value.status == 1 and "shape" in str(e.value)
        assert kvm.debug_prefill_shape(kvm.PREFILL_SHAPE_AUTO) == 2
    finally:
        kvm.debug_prefill_shape(prev)
    assert prev == kvm.PREFILL_SHAPE_AUTO
    was = kvm.debug_prefill_packing(False)
    try:
        assert kvm.debug_prefill_packing(True) is False
    finally:
        kvm.debug_prefill_packing(was)
    assert was is True


def test_prefill_status_hook_without_gpu(pkg, kvm):
    """The prefill status read-back validates its argument and, with no GPU
    in the process, reports a HIP error instead of crashing."""
    assert kvm.lib().mc_kv_debug_prefill_status(None, 0) == 1
    assert b"NULL" in kvm.lib().mc_last_error()
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present: the GPU prefill tests read the status")
    with pytest.raises(pkg.McError) as e:
        kvm.debug_prefill_status()
    assert e.value.status == 3


def test_model_load_option_checks_without_gpu(pkg, tmp_path):
    """mc_model_load's option checks in the reference's order and codes
    (native/runtime/model.cpp:58-100, tests/abi_smoke.cpp:118-134): weight
    and cache precision first (MC_E_UNSUPPORTED), then device_id, sessions
    and a zero context (MC_E_INVALID_ARGUMENT), then a context beyond the
    model's 131072 positions (MC_E_UNSUPPORTED); all before any device call."""
    import importlib
    rt = importlib.import_module(pkg.__name__ + ".runtime")
    cases = [
        (dict(precision=1), 7, "precision"),                    # MC_FP16
        (dict(precision=3), 7, "precision"),                    # MC_NVFP4
        (dict(kv_precision=1), 7, "KV cache"),                  # MC_KV_FP8
        (dict(precision=1, max_sessions=0), 7, "precision"),    # precision first
        (dict(device_id=-1), 1, "device_id"),
        (dict(max_sessions=0), 1, "max_sessions"),
        (dict(max_context_tokens=0), 1, "max_context_tokens"),
        (dict(max_context_tokens=0, max_sessions=0), 1, "max_sessions"),
        (dict(max_context_tokens=131073), 7, "131072"),
        (dict(abi_version=0), 1, "ABI"),
    ]
    for kw, status, word in cases:
        with pytest.raises(pkg.McError) as e:
            rt.Model(str(tmp_path), rt.model_options(**kw))
        assert e.value.status == status and word in str(e.value), (kw, e.value)


def test_chunk512_tier_from_environment(orc):
    """MC_ATTN_CHUNK512_ON gives contexts above 114688 positions 512-position
    chunks, MC_ATTN_CHUNK512_OFF overrides it (kernels.h:292-304); the
    switches are read once per process, so each case runs in its own."""
    import subprocess
    import sys
    ctxs = (16384, 49152, 114688, 114689, 131072)
    code = ("import importlib, sys; sys.path.insert(0, %r); "
            "kvm = importlib.import_module('minicpm5-5080fast_amd').kv; "
            "print(*[kvm.attention_decode_chunk_pos(c) for c in %r])" % (ROOT, ctxs))
    for env, c512 in (({"MC_ATTN_CHUNK512_ON": "1"}, True),
                      ({"MC_ATTN_CHUNK512_ON": "1", "MC_ATTN_CHUNK512_OFF": "1"}, False),
                      ({"MC_ATTN_CHUNK512_OFF": "1"}, False), ({}, False)):
        e = {k: v for k, v in os.environ.items() if not k.startswith("MC_ATTN_CHUNK512")}
        e.update(env)
        out = subprocess.run([sys.executable, "-c", code], env=e, capture_output=True,
                             text=True, timeout=120, check=True).stdout.split()
        assert [int(x) for x in out] == [orc.chunk_pos(c, c512) for c in ctxs], (env, out)
    assert [orc.chunk_pos(c, True) for c in ctxs] == [64, 128, 256, 512, 512]
