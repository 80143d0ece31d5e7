"""GPU tests of the mc_* ABI shell (weight-free mode) driving the KV path:
option/handle validation (model.cpp, batch_group.cpp rules), prefill ->
pages + RoPE'd K/V in the pool, decode -> mock token rule + phase0 append,
reset, OOM, max_new_tokens sentinel, and batched steps equal to solo steps
(tokens, sequences and pool bytes), after batch_test.cpp scenarios A/B.

The synthetic qkv rows of the weight-free runtime are restated here (the hash
of synth.hip) so pool contents can be checked against the oracle's kernel-
exact RoPE append."""
import ctypes as C
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

P, L, THETA = 32, 42, 5e6
M32 = 0xFFFFFFFF


def mix32(x):
    x = np.asarray(x, dtype=np.uint64) & M32
    x ^= x >> 16
    x = (x * 0x85EBCA6B) & M32
    x ^= x >> 13
    x = (x * 0xC2B2AE35) & M32
    x ^= x >> 16
    return x


def synth_row(orc, tok, pos, layer):
    seed = mix32(((tok * 0x9E3779B1) & M32) ^ int(mix32(pos + 0x632BE5AB)) ^
                 ((layer * 0x85EBCA77) & M32))
    h = mix32(seed ^ ((np.arange(2560, dtype=np.uint64) * 0x27D4EB2F) & M32))
    u = (h >> 8).astype(np.float32) * np.float32(1.0 / 16777216.0)
    return orc.f32_to_bf16(u - np.float32(0.5))


def mock_token(seq_len, rng):
    return 100 + (((seq_len * 2654435761) & M32) ^ rng) % 1000


def xorshift32(x):
    x ^= (x << 13) & M32
    x ^= x >> 17
    x ^= (x << 5) & M32
    return x & M32


_hip = None


def d2h(ptr, nbytes, dtype):
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        _hip.hipDeviceSynchronize.argtypes = []
    out = np.empty(nbytes // np.dtype(dtype).itemsize, dtype=dtype)
    assert _hip.hipMemcpy(out.ctypes.data, ptr, nbytes, 2) == 0
    return out


@pytest.fixture(scope="module")
def rt(pkg, dev):
    import importlib
    return importlib.import_module("minicpm5-5080fast_amd.runtime")


@pytest.fixture()
def model(rt, tmp_path):
    m = rt.Model(str(tmp_path), rt.model_options(max_context_tokens=2048, max_sessions=8))
    yield m
    m.close()


def test_model_load_validation(rt, tmp_path):
    with pytest.raises(rt.McError) as e:
        rt.Model(str(tmp_path), rt.model_options(struct_size=36))
    assert e.value.status == 1
    with pytest.raises(rt.McError) as e:
        rt.Model(str(tmp_path / "missing"), rt.model_options())
    assert e.value.status == 2
    with pytest.raises(rt.McError) as e:
        rt.Model(str(tmp_path), rt.model_options(max_context_tokens=0))
    assert e.value.status == 1
    with pytest.raises(rt.McError) as e:
        rt.Model(str(tmp_path), rt.model_options(max_context_tokens=131073))
    assert e.value.status == 7
    (tmp_path / "model.wpk").write_bytes(b"x")  # a package too short for its header
    with pytest.raises(rt.McError) as e:
        rt.Model(str(tmp_path), rt.model_options())
    assert e.value.status == 2 and "model.wpk" in str(e.value)


def pool_token(info, layer, pos, pt):
    lay = info["layout"]
    off = (((layer * lay.max_pages + int(pt[pos // P])) * P) + pos % P) * 512
    return d2h(info["d_pool"] + off * 2, 1024, np.uint16)


def test_prefill_decode_reset(rt, model, orc):
    s = rt.Session(model)
    prompt = [int(x) for x in np.random.default_rng(1).integers(0, 130560, 300)]
    s.prefill(prompt)
    info = s.info()
    assert info["seq_len"] == 300 and info["pages_owned"] == 10
    pt = d2h(info["d_page_table"], 40, np.uint32)
    assert pt.tolist() == list(range(10))
    lay = info["layout"]
    # K/V of a few prompt positions in two layers == kernel-exact oracle
    for layer in (0, 41):
        for pos in (0, 31, 32, 299):
            row = synth_row(orc, prompt[pos], pos, layer).reshape(1, 2560)
            pool = np.zeros(lay.max_pages * P * 512 * L, np.uint16)
            orc.rope_append(row, 1, pos, layer, pt, P, lay.max_pages, THETA, 1, pool)
            off = orc.kv_off(P, lay.max_pages, layer, int(pt[pos // P]), pos % P, 0, 0, 0)
            assert np.array_equal(pool_token(info, layer, pos, pt), pool[off:off + 512])
    cfg = rt.gen_config(max_new_tokens=6, seed=1234)
    rng, toks = 1234, []
    for i in range(6):
        want = mock_token(300 + i, rng)
        rng = xorshift32(rng)
        got = s.decode_one(cfg)
        assert got == want
        toks.append(got)
    assert s.decode_one(cfg) == rt.EOS_STREAM_ID  # max_new_tokens sentinel
    info = s.info()
    assert info["seq_len"] == 306 and info["pages_owned"] == 10
    assert s.seq(306) == prompt + toks
    # phase0 appended K/V of decode positions: input token = previous token
    pt = d2h(info["d_page_table"], 40, np.uint32)
    prev = [prompt[-1]] + toks
    for i, pos in enumerate(range(300, 306)):
        row = synth_row(orc, prev[i], pos, 7).reshape(1, 2560)
        pool = np.zeros(lay.max_pages * P * 512 * L, np.uint16)
        orc.rope_append(row, 1, pos, 7, pt, P, lay.max_pages, THETA, 1, pool)
        off = orc.kv_off(P, lay.max_pages, 7, int(pt[pos // P]), pos % P, 0, 0, 0)
        assert np.array_equal(pool_token(info, 7, pos, pt), pool[off:off + 512])
    st = s.stats()
    assert st.prompt_tokens == 300 and st.generated_tokens == 6
    s.reset()
    assert s.info()["seq_len"] == 0 and s.info()["pages_owned"] == 0
    s.prefill(prompt[:40])
    assert s.info()["pages_owned"] == 2
    with pytest.raises(rt.McError) as e:
        s.prefill([1] * 2048)
    assert e.value.status == 5
    s.close()


def test_decode_errors(rt, model):
    s = rt.Session(model)
    with pytest.raises(rt.McError) as e:
        s.decode_one(rt.gen_config())
    assert e.value.status == 1  # empty sequence
    with pytest.raises(rt.McError) as e:
        s.prefill([130560])
    assert e.value.status == 1
    s.prefill([5, 6, 7])
    with pytest.raises(rt.McError) as e:
        s.decode_one(rt.gen_config(struct_size=28))
    assert e.value.status == 1
    s.close()


def test_batch_equals_solo(rt, model):
    """Scenario A/B of batch_test.cpp: tokens from batched steps equal solo
    decode, and the KV pools end bit-identical."""
    rng = np.random.default_rng(7)
    prompts = [[int(x) for x in rng.integers(0, 130560, n)] for n in (100, 333, 64)]
    solo = [rt.Session(model) for _ in prompts]
    bat = [rt.Session(model) for _ in prompts]
    for a, b, p in zip(solo, bat, prompts):
        a.prefill(p)
        b.prefill(p)
    cfgs = [rt.gen_config(max_new_tokens=100, seed=11 * (i + 1)) for i in range(3)]
    want = [[a.decode_one(cfgs[i]) for _ in range(5)] for i, a in enumerate(solo)]
    g = rt.BatchGroup(model, 4, 2048)
    slots = [g.add(b) for b in bat]
    got = [[] for _ in bat]
    for step in range(5):
        out = g.step(slots, cfgs)
        for i, t in enumerate(out):
            got[i].append(t)
    assert got == want
    for s_ in slots:
        g.remove(s_)
    for a, b, p in zip(solo, bat, prompts):
        ia, ib = a.info(), b.info()
        assert ia["seq_len"] == ib["seq_len"] == len(p) + 5
        nb = ia["pages_owned"] * P * 1024
        lay = ia["layout"]
        for layer in (0, 20, 41):
            base = layer * lay.max_pages * P * 1024
            assert np.array_equal(d2h(ia["d_pool"] + base, nb, np.uint16),
                                  d2h(ib["d_pool"] + base, nb, np.uint16))
        assert a.seq(len(p) + 5) == b.seq(len(p) + 5)
    # solo -> batch -> solo lifecycle continues consistently
    assert bat[0].decode_one(cfgs[0]) == solo[0].decode_one(cfgs[0])
    g.close()
    for s_ in solo + bat:
        s_.close()


def test_batch_group_rules(rt, model, tmp_path):
    with pytest.raises(rt.McError) as e:
        rt.BatchGroup(model, 4, 2048, reserved=[0, 1, 0, 0])
    assert e.value.status == 1
    with pytest.raises(rt.McError) as e:
        rt.BatchGroup(model, 9, 2048)
    assert e.value.status == 7
    with pytest.raises(rt.McError) as e:
        rt.BatchGroup(model, 2, 4096)
    assert e.value.status == 7
    g = rt.BatchGroup(model, 2, 2048)
    a, b, c = rt.Session(model), rt.Session(model), rt.Session(model)
    a.prefill([1, 2, 3])
    sa, sb = g.add(a), g.add(b)
    with pytest.raises(rt.McError) as e:
        g.add(c)
    assert e.value.status == 7  # full
    g2 = rt.BatchGroup(model, 2, 2048)
    with pytest.raises(rt.McError) as e:
        g2.add(a)
    assert e.value.status == 7  # already in a group
    cfg = rt.gen_config()
    with pytest.raises(rt.McError) as e:
        g.step([sa, sa], [cfg, cfg])
    assert e.value.status == 1  # duplicate
    with pytest.raises(rt.McError) as e:
        g.step([sa, sb], [cfg, cfg])
    assert e.value.status == 1  # b is empty
    with pytest.raises(rt.McError) as e:
        g.step([sa], [rt.gen_config(temperature=0.7, top_k=40)])
    assert e.value.status == 7  # non-greedy
    with pytest.raises(rt.McError) as e:
        a.decode_one(cfg)
    assert e.value.status == 7  # member used solo while in the group
    with pytest.raises(rt.McError) as e:
        g.remove(5)
    assert e.value.status == 1
    g.remove(sa)
    a.decode_one(cfg)
    g.close()
    g2.close()
    for s_ in (a, b, c):
        s_.close()


def test_session_limit(rt, tmp_path):
    m = rt.Model(str(tmp_path), rt.model_options(max_context_tokens=256, max_sessions=2))
    s1, s2 = rt.Session(m), rt.Session(m)
    with pytest.raises(rt.McError) as e:
        rt.Session(m)
    assert e.value.status == 7
    s1.close()
    s3 = rt.Session(m)
    for s_ in (s2, s3):
        s_.close()
    m.close()


def test_graph_mode_matches_eager(rt, tmp_path):
    """enable_cuda_graph: the per-layer decode launches of a step (solo and
    batched) are captured once into a HIP graph and replayed; tokens,
    sequences and pool bytes equal the eager runtime's."""
    rng = np.random.default_rng(3)
    prompts = [[int(x) for x in rng.integers(0, 130560, n)] for n in (70, 257)]
    res = []
    for graphs in (0, 1):
        m = rt.Model(str(tmp_path), rt.model_options(max_context_tokens=2048, max_sessions=4,
                                                     enable_cuda_graph=graphs))
        ss = [rt.Session(m) for _ in prompts]
        for s_, p in zip(ss, prompts):
            s_.prefill(p)
        cfgs = [rt.gen_config(max_new_tokens=100, seed=5 + i) for i in range(2)]
        toks = [[ss[0].decode_one(cfgs[0]) for _ in range(4)]]
        g = rt.BatchGroup(m, 4, 2048)
        slots = [g.add(s_) for s_ in ss]
        toks += [g.step(slots, cfgs) for _ in range(3)]
        toks += [g.step(slots[1:], cfgs[1:]) for _ in range(2)]
        for sl in slots:
            g.remove(sl)
        toks.append([ss[1].decode_one(cfgs[1]) for _ in range(2)])
        pools = []
        for s_ in ss:
            info = s_.info()
            nb = info["pages_owned"] * P * 1024
            lay = info["layout"]
            pools.append([d2h(info["d_pool"] + l * lay.max_pages * P * 1024, nb, np.uint16)
                          for l in (0, 41)])
            pools.append(s_.seq(info["seq_len"]))
        launches = [s_.stats().cuda_graph_launches for s_ in ss]
        res.append((toks, pools, launches))
        g.close()
        for s_ in ss:
            s_.close()
        m.close()
    (t0, p0, l0), (t1, p1, l1) = res
    assert t0 == t1
    for a, b in zip(p0, p1):
        if isinstance(a, list) and a and isinstance(a[0], np.ndarray):
            assert all(np.array_equal(x, y) for x, y in zip(a, b))
        else:
            assert a == b
    assert l0 == [0, 0] and l1 == [4 + 3, 3 + 2 + 2]


def test_long_prefill_multichunk(rt, tmp_path, orc):
    """A 20000-token prompt (three prefill chunks of up to 8448 tokens) in a
    131072-token session: K/V at chunk boundaries equal the kernel-exact
    oracle, then decode steps (512-chunk tier, two-level merge) follow the
    mock token rule."""
    m = rt.Model(str(tmp_path), rt.model_options(max_context_tokens=131072, max_sessions=1))
    s = rt.Session(m)
    rng = np.random.default_rng(17)
    prompt = [int(x) for x in rng.integers(0, 130560, 20000)]
    s.prefill(prompt)
    info = s.info()
    assert info["seq_len"] == 20000 and info["pages_owned"] == -(-20000 // P)
    lay = info["layout"]
    pt = d2h(info["d_page_table"], 4 * info["pages_owned"], np.uint32)
    assert pt.tolist() == list(range(info["pages_owned"]))
    for layer in (0, 41):
        for pos in (8447, 8448, 16895, 16896, 19999):
            row = synth_row(orc, prompt[pos], pos, layer).reshape(1, 2560)
            ref = np.zeros(lay.max_pages * P * 512 * L, np.uint16)
            orc.rope_append(row, 1, pos, layer, pt, P, lay.max_pages, THETA, 1, ref)
            off = orc.kv_off(P, lay.max_pages, layer, int(pt[pos // P]), pos % P, 0, 0, 0)
            assert np.array_equal(pool_token(info, layer, pos, pt), ref[off:off + 512]), pos
    cfg = rt.gen_config(max_new_tokens=8, seed=99)
    rng_state = 99
    for i in range(3):
        want = mock_token(20000 + i, rng_state)
        rng_state = xorshift32(rng_state)
        assert s.decode_one(cfg) == want
    assert s.info()["seq_len"] == 20003
    s.close()
    m.close()


def test_many_resets_and_two_threads(rt, tmp_path):
    """Soak-style checks after soak_test.cpp T4 (200 resets) and T2b (two
    sessions driven from two host threads at once): pages return to zero on
    every reset, and concurrent sessions produce exactly the tokens they
    produce when run one after the other."""
    import threading
    m = rt.Model(str(tmp_path), rt.model_options(max_context_tokens=1024, max_sessions=4))
    s = rt.Session(m)
    cfg = rt.gen_config(max_new_tokens=4, seed=3)
    for i in range(200):
        s.prefill([7 + (i % 50)] * (1 + i % 97))
        s.decode_one(cfg)
        s.reset()
        info = s.info()
        assert info["seq_len"] == 0 and info["pages_owned"] == 0
    s.close()

    def run(sess, prompt, seed, out):
        sess.prefill(prompt)
        c = rt.gen_config(max_new_tokens=40, seed=seed)
        out.extend(sess.decode_one(c) for _ in range(40))

    prompts = [[11] * 300, [int(x) for x in range(1000, 1200)]]
    solo = []
    for i, p in enumerate(prompts):
        x = rt.Session(m)
        r = []
        run(x, p, 100 + i, r)
        solo.append((r, x.seq(len(p) + 40)))
        x.close()
    ss = [rt.Session(m) for _ in prompts]
    outs = [[], []]
    th = [threading.Thread(target=run, args=(ss[i], prompts[i], 100 + i, outs[i]))
          for i in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    for i in range(2):
        assert outs[i] == solo[i][0]
        assert ss[i].seq(len(prompts[i]) + 40) == solo[i][1]
        ss[i].close()
    m.close()


@pytest.mark.parametrize("graphs", [0, 1])
def test_breakdown_and_group_stats(rt, tmp_path, graphs, monkeypatch):
    """The decode-step breakdown hooks (MC_BREAKDOWN / MC_BATCH_BREAKDOWN at
    create, reference session.cpp:686-723, batch_group.cpp:869-927): off by
    default (0), then one segment per (layer, {qkv, attention}) plus the tail,
    all positive and summing to at most the step's wall time; the batch
    group's bucket times and step statistics. With the step captured in a
    HIP graph no segment is recorded (-2) and the statistics still count."""
    import time
    m = rt.Model(str(tmp_path), rt.model_options(max_context_tokens=2048, max_sessions=4,
                                                 enable_cuda_graph=graphs))
    plain = rt.Session(m)
    assert plain.breakdown() == 0 and plain.arena_bytes() > 0 and plain.attn_chunk() == 64
    monkeypatch.setenv("MC_BREAKDOWN", "1")
    monkeypatch.setenv("MC_BATCH_BREAKDOWN", "1")
    s = rt.Session(m)
    s.prefill(list(range(5, 300)))
    cfg = rt.gen_config(max_new_tokens=50, seed=2)
    assert s.breakdown() == -2  # no decode step yet
    for _ in range(3):
        t0 = time.perf_counter()
        s.decode_one(cfg)
        wall_ms = (time.perf_counter() - t0) * 1e3
        segs = s.breakdown()
        if graphs:
            assert segs == -2
            continue
        assert isinstance(segs, list) and len(segs) == 2 * 42 + 1
        assert all(x >= 0.0 for x in segs) and sum(segs) <= wall_ms + 0.05
        assert all(x > 0.0 for x in segs[1:84:2])  # the attention segments
    L = rt._bind()
    assert L.mc_debug_breakdown_bucket_count() == 3
    assert L.mc_debug_breakdown_bucket_name(1).startswith(b"layer(attention")
    assert L.mc_debug_breakdown_bucket_of(1) == 1 and L.mc_debug_breakdown_bucket_of(84) == 2
    g = rt.BatchGroup(m, 4, 2048)
    assert g.breakdown() == -2
    slot = g.add(s)
    for k in range(4):
        g.step([slot], [cfg])
        st = g.stats()
        assert st["steps"] == k + 1 and st["members"] == 1 and st["decode_us"] > 0
        b = g.breakdown()
        if graphs:
            assert b == -2
            continue
        assert isinstance(b, list) and len(b) == 3 and b[1] > 0.0 and min(b) >= 0.0
    g.remove(slot)
    assert g.stats()["members"] == 0
    g.close()
    s.close()
    plain.close()
    m.close()


def test_session_graph_and_rope_hooks(rt, tmp_path):
    """Debug hooks of session.cpp:636-686: the graph A/B switch gives the same
    tokens and pool bytes with the graph on and off, the captured graph
    reports its nodes (> 0 after the first graph step, 0 before), and the RoPE
    table stays bit-identical to its create-time snapshot through prefill,
    graph and eager decode and batch steps (sampling_regression.cpp:207-247)."""
    m = rt.Model(str(tmp_path), rt.model_options(max_context_tokens=2048, max_sessions=4,
                                                 enable_cuda_graph=1))
    rng = np.random.default_rng(11)
    prompt = [int(x) for x in rng.integers(0, 130560, 150)]
    a, b = rt.Session(m), rt.Session(m)
    assert a.rope_intact() == 1 and a.graph_nodes() == 0
    a.prefill(prompt)
    b.prefill(prompt)
    assert a.rope_intact() == 1
    cfg = rt.gen_config(max_new_tokens=100, seed=9)
    b.set_graph_enabled(False)
    ta, tb = [], []
    for i in range(6):
        if i == 3:  # switch both sessions midway: a to eager, b back to graphs
            a.set_graph_enabled(False)
            b.set_graph_enabled(True)
        ta.append(a.decode_one(cfg))
        tb.append(b.decode_one(cfg))
        assert a.rope_intact() == 1 and b.rope_intact() == 1
    assert ta == tb
    assert a.graph_nodes() > 0 and b.graph_nodes() == a.graph_nodes()
    assert a.stats().cuda_graph_launches == 3 and b.stats().cuda_graph_launches == 3
    for s_ in (a, b):
        info = s_.info()
        assert info["seq_len"] == 156
    pa, pb = a.info(), b.info()
    nb = pa["pages_owned"] * P * 1024
    lay = pa["layout"]
    for layer in (0, 41):
        off = layer * lay.max_pages * P * 1024
        assert np.array_equal(d2h(pa["d_pool"] + off, nb, np.uint16),
                              d2h(pb["d_pool"] + off, nb, np.uint16))
    g = rt.BatchGroup(m, 2, 2048)
    slots = [g.add(a), g.add(b)]
    for _ in range(2):
        g.step(slots, [cfg, cfg])
    for sl in slots:
        g.remove(sl)
    assert a.rope_intact() == 1 and b.rope_intact() == 1
    g.close()
    a.close()
    b.close()
    m.close()


def test_prefill_barrier_timeout_reported(rt, kvm, model):
    """A half-barrier timeout count left on the device after a prefill chunk
    makes mc_prefill fail with MC_E_INTERNAL (instead of returning MC_OK with
    unreliable rows) and clears the count; the next prefill succeeds. The
    count is set from the host: no wait is made to time out."""
    s = rt.Session(model)
    kvm.debug_prefill_status(reset=True)
    kvm.debug_prefill_force_timeouts(3)
    with pytest.raises(rt.McError) as e:
        s.prefill([1, 2, 3, 4])
    assert e.value.status == 100 and "half-barrier" in str(e.value)
    assert kvm.debug_prefill_status() == 0
    s.reset()
    s.prefill([1, 2, 3, 4])
    assert s.info()["seq_len"] == 4
    s.close()
