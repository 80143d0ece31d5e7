"""model.wpk checks (mc_model_wpk_check, no device) and pins of the forward
oracle (oracle/model_ref.py), on the CPU.

The package checks follow the reference loader (weight_loader.cpp:201-330):
header magic / ABI / target, TOC placement, unique name hashes, exactly the
model's 255 sections, bf16 row-major tensors of the model's shapes, data
inside the file. Packages here are sparse files (data holes), so the checks
run on the full geometry without writing gigabytes.
"""
import ctypes as C
import os

import numpy as np
import pytest

import wpk_util as W

OK, IO, MISMATCH, UNSUPPORTED = 0, 2, 4, 7


@pytest.fixture(scope="module")
def lib(pkg):
    return pkg._native.lib()


def check(lib, path):
    n = C.c_uint64(0)
    st = lib.mc_model_wpk_check(str(path).encode(), C.byref(n))
    return st, n.value, lib.mc_last_error().decode()


def test_valid_package(lib, tmp_path):
    secs = W.model_sections()
    p = tmp_path / "model.wpk"
    W.write_wpk(p, secs, W.sparse_blobs())
    st, n, msg = check(lib, p)
    assert st == OK, msg
    assert n == W.arena_bytes(secs)
    # 2 x 535 MB tables + 42 x 94.4 MB layers + norms: the real model's size
    assert 5.0e9 < n < 5.1e9


@pytest.mark.parametrize("field,value", [("magic", 0x31504B4E), ("abi", 3), ("target_sm", 90),
                                         ("toc_offset", 128), ("reserved", 1),
                                         ("data_start", 1 << 40)])
def test_bad_header(lib, tmp_path, field, value):
    p = tmp_path / "model.wpk"
    W.write_wpk(p, W.model_sections(), W.sparse_blobs(), header={field: value})
    st, _, msg = check(lib, p)
    assert st == MISMATCH and "model.wpk" in msg, msg


def test_toc_longer_than_its_room(lib, tmp_path):
    p = tmp_path / "model.wpk"
    W.write_wpk(p, W.model_sections(), W.sparse_blobs(), header={"data_start": 64 + 132})
    assert check(lib, p)[0] == MISMATCH


def test_missing_file_and_short_header(lib, tmp_path):
    assert check(lib, tmp_path / "none.wpk")[0] == IO
    p = tmp_path / "model.wpk"
    p.write_bytes(b"MKP1" + b"\x00" * 20)
    assert check(lib, p)[0] == IO


def test_section_count(lib, tmp_path):
    p = tmp_path / "model.wpk"
    secs = W.model_sections()
    W.write_wpk(p, secs[:-1], W.sparse_blobs())  # one missing
    st, _, msg = check(lib, p)
    assert st == MISMATCH and "254" in msg, msg
    extra = secs + [("layer42.norm1", (W.HIDDEN,), "final_norm")]
    W.write_wpk(p, extra, W.sparse_blobs())
    assert check(lib, p)[0] == MISMATCH


def test_duplicate_and_unknown_names(lib, tmp_path):
    p = tmp_path / "model.wpk"
    secs = W.model_sections()

    def dup(i, d):
        if i == 7:
            d["hash"] = W.fnv1a64("layer0.qkv")
    W.write_wpk(p, secs, W.sparse_blobs(), entry_patch=dup)
    st, _, msg = check(lib, p)
    assert st == MISMATCH and "share" in msg, msg

    def rename(i, d):
        if i == 4:  # layer0.qkv
            d["hash"] = W.fnv1a64("layer0.qkv_proj")
    W.write_wpk(p, secs, W.sparse_blobs(), entry_patch=rename)
    st, _, msg = check(lib, p)
    assert st == MISMATCH and "layer0.qkv" in msg and "missing" in msg, msg


@pytest.mark.parametrize("patch", [
    lambda d: d.update(dtype=2), lambda d: d.update(layout=1), lambda d: d.update(rank=1),
    lambda d: d["dims"].__setitem__(1, 2049), lambda d: d.update(bytes=d["bytes"] - 2),
    lambda d: d.update(offset=64), lambda d: d.update(offset=1 << 42)])
def test_bad_entry(lib, tmp_path, patch):
    p = tmp_path / "model.wpk"

    def ep(i, d):
        if i == 10:  # layer1.qkv
            patch(d)
    W.write_wpk(p, W.model_sections(), W.sparse_blobs(), entry_patch=ep)
    st, _, msg = check(lib, p)
    assert st == MISMATCH and "layer1.qkv" in msg, msg


def test_data_past_end_of_file(lib, tmp_path):
    p = tmp_path / "model.wpk"
    W.write_wpk(p, W.model_sections(), W.sparse_blobs())
    size = os.path.getsize(p)
    with open(p, "r+b") as f:
        f.truncate(size - 4096)  # the last section now ends past the file
    assert check(lib, p)[0] == MISMATCH


def test_layer_window_switches_rejected(lib, tmp_path, monkeypatch):
    p = tmp_path / "model.wpk"
    W.write_wpk(p, W.model_sections(), W.sparse_blobs())
    monkeypatch.setenv("MC_LOAD_LAYERS_MAX", "2")
    st, _, msg = check(lib, p)
    assert st == UNSUPPORTED and "MC_LOAD_LAYERS_MAX" in msg, msg


# ---------------- model_fp8.wpk (precision MC_FP8) ----------------

def check8(lib, path):
    n = C.c_uint64(0)
    st = lib.mc_model_wpk_fp8_check(str(path).encode(), C.byref(n))
    return st, n.value, lib.mc_last_error().decode()


def test_fp8_package_valid(lib, tmp_path, monkeypatch):
    """The 168 projections plus the optional lm_head (weight_loader.cpp:
    525-560); sections the FP8 loader does not use are ignored; with
    MC_FP8_LMHEAD_OFF set a package's lm_head is skipped."""
    p = tmp_path / "model_fp8.wpk"
    secs = W.fp8_sections(lm_head=True)
    W.write_fp8_wpk(p, secs, W.fp8_sparse_blobs())
    st, n, msg = check8(lib, p)
    assert st == OK, msg
    assert n == W.fp8_arena_bytes(secs)
    assert 2.2e9 < n < 2.3e9  # half the bytes of the bf16 projections and lm_head
    monkeypatch.setenv("MC_FP8_LMHEAD_OFF", "1")
    st, n_off, msg = check8(lib, p)
    assert st == OK and n_off == W.fp8_arena_bytes(secs[:-1]), msg
    monkeypatch.delenv("MC_FP8_LMHEAD_OFF")
    secs = W.fp8_sections(lm_head=False)
    W.write_fp8_wpk(p, secs + [("layer0.norm1", (1, 2048), "o.0")], W.fp8_sparse_blobs())
    st, n, msg = check8(lib, p)
    assert st == OK and n == W.fp8_arena_bytes(secs), msg


@pytest.mark.parametrize("patch", [
    lambda d: d.update(dtype=0), lambda d: d.update(layout=1), lambda d: d.update(rank=1),
    lambda d: d["dims"].__setitem__(1, 2049), lambda d: d.update(bytes=d["bytes"] - 1),
    lambda d: d.update(scale_bytes=d["scale_bytes"] + 4), lambda d: d.update(offset=64),
    lambda d: d.update(scale_offset=1 << 42), lambda d: d.update(hash=W.fnv1a64("layer3.oo"))])
def test_fp8_package_bad_entry(lib, tmp_path, patch):
    p = tmp_path / "model_fp8.wpk"

    def ep(i, d):
        if i == 13:  # layer3.o
            patch(d)
    W.write_fp8_wpk(p, W.fp8_sections(), W.fp8_sparse_blobs(), entry_patch=ep)
    st, _, msg = check8(lib, p)
    assert st == MISMATCH and "layer3.o" in msg, msg


def test_fp8_package_header_duplicates_and_missing_file(lib, tmp_path):
    p = tmp_path / "model_fp8.wpk"
    assert check8(lib, p)[0] == MISMATCH  # no package: MC_FP8 cannot load
    secs = W.fp8_sections()

    def dup(i, d):
        if i == 5:
            d["hash"] = W.fnv1a64("layer0.qkv")
    W.write_fp8_wpk(p, secs, W.fp8_sparse_blobs(), entry_patch=dup)
    st, _, msg = check8(lib, p)
    assert st == MISMATCH and "share" in msg, msg
    W.write_fp8_wpk(p, secs, W.fp8_sparse_blobs())
    with open(p, "r+b") as f:
        f.write(b"MKP0")
    assert check8(lib, p)[0] == MISMATCH
    with open(p, "r+b") as f:
        f.truncate(40)
    assert check8(lib, p)[0] == IO


# ---------------- pins of the forward oracle ----------------

def test_rmsnorm_and_swiglu_closed_forms(orc):
    from oracle import model_ref as M
    rng = np.random.default_rng(3)
    x = M.bf16(rng.standard_normal((3, 2048)).astype(np.float32) * 3)
    w = M.bf16(1 + 0.1 * rng.standard_normal(2048).astype(np.float32))
    ref = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True)
                                         + 1e-6) * w
    got = M.rmsnorm(x, w)
    assert np.all(np.abs(got - ref) <= orc.bf16_ulp(ref) * 0.5 + 1e-30)
    # constant rows normalize to sign * w (up to eps)
    c = np.full((1, 2048), 4.0, dtype=np.float32)
    assert np.allclose(M.rmsnorm(c, w), M.bf16(w), rtol=2 ** -8)
    g = np.array([-30.0, -1.0, 0.0, 1.0, 30.0], dtype=np.float32)
    u = np.array([1.0, 2.0, 3.0, 4.0, 5.0], dtype=np.float32)
    np.testing.assert_allclose(M.silu_mul(g, u), g / (1 + np.exp(-g.astype(np.float64))) * u,
                               rtol=2 ** -8, atol=1e-12)


def small_model(rng, vocab, layers, zero_mix=False):
    """A model of the oracle's shapes with a small vocabulary."""
    from oracle import model_ref as M

    def mat(r, c, s):
        return M.bf16(rng.standard_normal((r, c), dtype=np.float32) * np.float32(s))

    w = {"embedding": mat(vocab, 2048, 1.0), "lm_head": mat(vocab, 2048, 1 / 45.25),
         "final_norm": M.bf16(1 + 0.1 * rng.standard_normal(2048).astype(np.float32))}
    for l in range(layers):
        p = f"layer{l}."
        w[p + "norm1"] = M.bf16(1 + 0.1 * rng.standard_normal(2048).astype(np.float32))
        w[p + "norm2"] = M.bf16(1 + 0.1 * rng.standard_normal(2048).astype(np.float32))
        w[p + "qkv"] = mat(2560, 2048, 1 / 45.25)
        w[p + "gate_up"] = mat(12288, 2048, 1 / 45.25)
        w[p + "o"] = np.zeros((2048, 2048), np.float32) if zero_mix else mat(2048, 2048, 1 / 45.25)
        w[p + "down"] = (np.zeros((2048, 6144), np.float32) if zero_mix
                         else mat(2048, 6144, 1 / 78.4))
    return w


def test_forward_with_zero_mixing_is_the_embedding_path(orc):
    """With the o and down projections zero every layer adds nothing to the
    residual: logits = bf16(rmsnorm(embedding[id], final_norm) . lm_head^T)
    for every position, whatever the attention and MLP compute."""
    from oracle import model_ref as M
    rng = np.random.default_rng(5)
    w = small_model(rng, 500, 2, zero_mix=True)
    ref = M.ModelRef(w, 2)
    ids = [3, 17, 499, 0]
    tok = ref.forward(ids)
    x = M.rmsnorm(w["embedding"][ids[-1]][None], w["final_norm"])
    exact = (x.astype(np.float64) @ w["lm_head"].T.astype(np.float64))[0]
    # the oracle accumulates in fp32: within one bf16 ulp of the exact product
    assert np.all(np.abs(ref.last_logits - exact) <= orc.bf16_ulp(exact) + 1e-6)
    assert tok == int(np.argmax(ref.last_logits))
    assert exact[tok] >= exact.max() - 2 * orc.bf16_ulp(exact.max())
    # decode: returns the pending prediction, then predicts from it
    assert ref.decode() == tok and ref.seq_len == 5


def test_forward_single_token_attention_is_v(orc):
    """At position 0 the attention output is V of that position (one key):
    the oracle's layer output equals the same graph with attention replaced
    by the V columns of the rotated qkv row."""
    from oracle import model_ref as M
    rng = np.random.default_rng(7)
    w = small_model(rng, 300, 1)
    ref = M.ModelRef(w, 1)
    ref.forward([42])
    res = w["embedding"][[42]]
    normed = M.rmsnorm(res, w["layer0.norm1"])
    qkv = M.project(normed, w["layer0.qkv"])
    v = qkv[:, 2304:2560]
    att = np.concatenate([np.tile(v[:, :128], 8), np.tile(v[:, 128:], 8)], axis=1)
    res = M.bf16(res + M.project(att, w["layer0.o"]))
    normed = M.rmsnorm(res, w["layer0.norm2"])
    gu = M.project(normed, w["layer0.gate_up"])
    res = M.bf16(res + M.project(M.silu_mul(gu[:, :6144], gu[:, 6144:]), w["layer0.down"]))
    logits = M.project(M.rmsnorm(res, w["final_norm"]), w["lm_head"])[0]
    assert np.array_equal(ref.last_logits, logits)


def test_forward_matches_reference_statement(orc):
    """The oracle against the reference's own whole-model numpy statement
    (tools/reference_forward.py MiniCPM5Ref; logits in
    tests/golden/model_forward_small.json, written by
    tests/golden/make_model_forward_golden.py): 2 layers, vocabulary 512,
    random weights, a 6-token prefill and 5 greedy decode steps. The two
    statements differ only where the reference leaves the arithmetic to
    numpy (cos/sin of the RoPE angles, the fp32 softmax's summation order),
    so most steps are bit-identical and every step's logits are within
    relative L2 1e-2 with the same greedy token. A graph mistake (a norm
    weight swapped, the residual added twice, the gate and up halves
    exchanged, the wrong KV head for a query head) moves the logits by
    order one."""
    import json
    from oracle import model_ref as M
    with open(os.path.join(os.path.dirname(__file__), "golden",
                           "model_forward_small.json")) as f:
        d = json.load(f)
    w = W.golden_small_model(d["seed"], d["vocab"], d["layers"])
    ref = M.ModelRef({k: orc.bf16_to_f32(v) for k, v in w.items()}, d["layers"])
    got = [(ref.forward(d["prompt"]), ref.last_logits)]
    for _ in range(len(d["tokens"]) - 1):
        ref.decode()
        got.append((ref.next_token, ref.last_logits))
    exact = 0
    for step, (tok, logits) in enumerate(got):
        want = orc.bf16_to_f32(np.array(d["logits_bf16"][step], dtype=np.uint16))
        assert tok == d["tokens"][step], step
        rel = np.linalg.norm(logits - want) / np.linalg.norm(want)
        assert rel < 1e-2, (step, rel)
        exact += int(np.array_equal(logits, want))
    assert exact >= len(got) // 2, exact


def test_e4m3_decode_known_answers_and_round_trip():
    """The oracle's e4m3 decoder on the reference's known-answer codes
    (kernel_ops.cpp:1237-1247) and on S.1111.111 (+-480, kernels.h:120-125),
    and the test quantizer's nearest-even encoding, which must return every
    finite code from its own value (a wrong exponent bias or mantissa width
    breaks both)."""
    from oracle import model_ref as M
    ka = {0x00: 0.0, 0x66: 56.0, 0xE6: -56.0, 0x7E: 448.0, 0x01: 0.001953125,
          0x02: 0.00390625, 0x07: 0.013671875, 0x08: 0.015625, 0x40: 2.0, 0x50: 8.0,
          0x7F: 480.0, 0xFF: -480.0}
    for code, want in ka.items():
        assert M.e4m3_to_f32(np.uint8(code)) == np.float32(want), hex(code)
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    assert np.array_equal(W.f32_to_e4m3(M.e4m3_to_f32(codes)), codes)
    # ties go to the even code: halfway between 1.0 (0x38) and 1.125 (0x39)
    assert W.f32_to_e4m3(np.float32(1.0625)) == 0x38
    assert W.f32_to_e4m3(np.float32(1.1875)) == 0x3A
    assert W.f32_to_e4m3(np.float32(1000.0)) == 0x7E   # saturates at 448


def test_forward_fp8_matches_reference_statement(orc):
    """FP8 mode against the reference's numpy statement with use_fp8 for the
    single-token steps (tests/golden/model_forward_small.json "fp8"): the
    prefill stays bf16, the decode projections and lm_head use the e4m3 codes
    and row scales of the same weights. Same tokens, every step within
    relative L2 1e-2, and the FP8 logits differ from the bf16 run (the mode
    is live)."""
    import json
    from oracle import model_ref as M
    with open(os.path.join(os.path.dirname(__file__), "golden",
                           "model_forward_small.json")) as f:
        d = json.load(f)
    w = W.golden_small_model(d["seed"], d["vocab"], d["layers"])
    q = W.golden_small_fp8(w, d["layers"])
    ref = M.ModelRef({k: orc.bf16_to_f32(v) for k, v in w.items()}, d["layers"], fp8=q)
    got = [(ref.forward(d["prompt"]), ref.last_logits)]
    for _ in range(len(d["fp8"]["tokens"]) - 1):
        ref.decode()
        got.append((ref.next_token, ref.last_logits))
    for step, (tok, logits) in enumerate(got):
        want = orc.bf16_to_f32(np.array(d["fp8"]["logits_bf16"][step], dtype=np.uint16))
        assert tok == d["fp8"]["tokens"][step], step
        rel = np.linalg.norm(logits - want) / np.linalg.norm(want)
        assert rel < 1e-2, (step, rel)
        if step > 0:
            bf = orc.bf16_to_f32(np.array(d["logits_bf16"][step], dtype=np.uint16))
            assert not np.array_equal(want, bf), step


def test_mutated_headers_rejected_cleanly(lib, tmp_path):
    """Random corruptions of a valid package's header and section table (byte
    flips, 32- and 64-bit fields set to edge values, truncated or extended
    files) come back as a status with a message, for both package checks;
    the parser is never driven outside its buffers."""
    import random
    import struct
    W.write_wpk(tmp_path / "b.wpk", W.model_sections(), W.sparse_blobs())
    W.write_fp8_wpk(tmp_path / "f.wpk", W.fp8_sections(), W.fp8_sparse_blobs())
    bases = [(open(tmp_path / k, "rb").read(65536), os.path.getsize(tmp_path / k))
             for k in ("b.wpk", "f.wpk")]
    rng = random.Random(20261202)
    edge = [0, 1, 0xFF, 0xFFFF, 0x7FFFFFFF, 0xFFFFFFFF, 1 << 32, 1 << 63, (1 << 64) - 1]
    seen = set()
    p = tmp_path / "m.wpk"
    for _ in range(150):
        head, size = rng.choice(bases)
        h = bytearray(head)
        for _ in range(rng.randint(1, 4)):
            off = rng.randrange(0, 64 + 132 * 170 - 8)
            r = rng.random()
            if r < 0.4:
                h[off] = rng.randrange(256)
            elif r < 0.7:
                struct.pack_into("<I", h, off & ~3, rng.choice(edge) & 0xFFFFFFFF)
            else:
                struct.pack_into("<Q", h, off & ~7, rng.choice(edge + [size, size + 1]))
        sz = rng.choice([size, size, size, rng.randrange(0, 70000), size - 4096])
        with open(p, "wb") as f:
            f.write(bytes(h[:min(len(h), sz)]))
            if sz > len(h):
                f.truncate(sz)
        n = C.c_uint64(0)
        for fn in (lib.mc_model_wpk_check, lib.mc_model_wpk_fp8_check):
            st = fn(str(p).encode(), C.byref(n))
            assert st in (OK, IO, MISMATCH, UNSUPPORTED), st
            if st != OK:
                assert lib.mc_last_error()
            seen.add(st)
    assert MISMATCH in seen
