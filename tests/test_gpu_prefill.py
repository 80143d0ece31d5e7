"""GPU parity of the prefill attention over the paged cache (page gather).

Cases follow native/tests/kernel_ops.cpp:3594 (T=80 with a causal-leak
sentinel) and :3808-... (T in {16, 17, 80}, base 5 and 13, the 8448-prefix
cross-chunk case, split-KV T=512/1024 with S from prefill_flash_split_kv).
Criterion: vs the double oracle relL2 < 1e-2, cos > 0.9999, max-abs 2e-2,
mean-abs 2e-3.
"""
import numpy as np
import pytest

from _util import from_dev, randn_bf16, to_dev

pytestmark = pytest.mark.gpu
POISON = 0xDCBA


@pytest.fixture(autouse=True)
def barrier_status_clear(kvm, dev):
    """Every prefill test must leave the per-half barrier timeout count at
    zero (a timed-out wait may have produced wrong output silently)."""
    kvm.debug_prefill_status(reset=True)
    yield
    assert kvm.debug_prefill_status(reset=True) == 0, "prefill half-barrier wait timed out"


def run_prefill(kvm, orc, dev, T, base, S, P=32, seed=0, sentinel=False, check=True,
                abs_check=True, kgrow=0.0, inputs=False):
    import torch
    rng = np.random.default_rng(seed)
    ctx = base + T
    maxp = -(-ctx // P) + 3
    pt = rng.permutation(maxp).astype(np.uint32)
    L, layer = 2, 1
    pool = np.full(maxp * P * 512 * L, POISON, dtype=np.uint16)
    for j in range(ctx):
        off = orc.kv_off(P, maxp, layer, int(pt[j // P]), j % P, 0, 0, 0)
        pool[off:off + 512] = randn_bf16(rng, 512, 0.6)
        if kgrow:  # K magnitude growing with position: the running max keeps moving
            k = orc.bf16_to_f32(pool[off:off + 256]) * np.float32(1.0 + kgrow * j / ctx)
            pool[off:off + 256] = orc.f32_to_bf16(k.astype(np.float32))
        if sentinel and j >= base + 40:  # V = 40 for future positions
            pool[off + 256:off + 512] = orc.f32_to_bf16(np.float32([40.0]))[0]
    q = randn_bf16(rng, T * 2560, 1.0).reshape(T, 2560)
    lay = kvm.KvLayout(maxp, P, L)
    d_q, d_pool, d_pt = to_dev(q.ravel(), dev), to_dev(pool, dev), to_dev(pt, dev)
    d_base = to_dev(np.array([base], dtype=np.uint32), dev)
    out = torch.zeros(T * 2048, dtype=torch.int16, device=dev)
    parts = (torch.full((T * 16 * S * 130,), float("nan"), dtype=torch.float32, device=dev)
             if S > 1 else None)
    kvm.launch_attn_prefill_flash(d_q, T, d_base, layer, d_pt, d_pool, lay, out, parts, S)
    torch.cuda.synchronize()
    got = from_dev(out).reshape(T, 2048)
    if check:
        ref = orc.attn_ref(q, T, base, layer, pool, pt, P, maxp)
        st = orc.compare_bf16(got, ref)
        print(T, base, S, st)
        assert st["rel_l2"] < 1e-2 and st["cos"] > 0.9999, st
        if abs_check:
            assert st["max_abs"] < 2e-2 and st["mean_abs"] < 2e-3, st
        else:  # the sentinel rows hold |V| = 40; check the unaffected rows
            st40 = orc.compare_bf16(got[:40], ref[:40])
            assert st40["max_abs"] < 2e-2 and st40["mean_abs"] < 2e-3, st40
    if inputs:
        return got, (q, pool, pt, maxp, layer)
    return got


@pytest.mark.parametrize("T,base", [(16, 0), (17, 0), (80, 0), (16, 5), (80, 13), (1, 0),
                                    (33, 100)])
def test_prefill_small(kvm, orc, dev, T, base):
    run_prefill(kvm, orc, dev, T, base, 1, seed=T + base)


def test_prefill_causal_sentinel(kvm, orc, dev):
    """Rows before position base+40 must not see the V=40 sentinel rows."""
    got = run_prefill(kvm, orc, dev, 80, 0, 1, seed=5, sentinel=True, abs_check=False)
    f = orc.bf16_to_f32(got[:40])
    assert np.abs(f).max() < 10.0


@pytest.mark.parametrize("T,S", [(512, 8), (1024, 4), (300, 8), (100, 3)])
def test_prefill_split_kv(kvm, orc, dev, T, S):
    assert kvm.prefill_flash_split_kv(512) == 8 and kvm.prefill_flash_split_kv(1024) == 4
    a = run_prefill(kvm, orc, dev, T, 7, S, seed=T)
    b = run_prefill(kvm, orc, dev, T, 7, 1, seed=T, check=False)
    d = np.abs(orc.bf16_to_f32(a) - orc.bf16_to_f32(b))
    assert d.max() < 2e-2


def test_prefill_cross_chunk_8448_prefix(kvm, orc, dev):
    """Second prefill chunk after an 8448-token prefix, 64-token pages."""
    run_prefill(kvm, orc, dev, 96, 8448, 1, P=64, seed=11)


@pytest.mark.parametrize("P,S", [(8, 1), (16, 2), (1, 1)])
def test_prefill_small_pages(kvm, orc, dev, P, S):
    """Pages smaller than a 32-key step: page ids looked up per key."""
    run_prefill(kvm, orc, dev, 150, 29, S, P=P, seed=P)


def test_prefill_long_chunk(kvm, orc, dev):
    """2048 rows over a 300-token prefix: many steps per tile, reference max
    moving late in long rows."""
    run_prefill(kvm, orc, dev, 2048, 300, 1, P=64, seed=21)


@pytest.mark.parametrize("T,base,S", [(512, 0, 1), (300, 40, 4), (96, 8448, 1)])
def test_prefill_growing_scores(kvm, orc, dev, T, base, S):
    """Keys whose magnitude grows tenfold along the context: the softmax
    reference moves many times mid-row (accumulator rescales) and lane sums
    overflow the fast-path bound, so both softmax paths run."""
    run_prefill(kvm, orc, dev, T, base, S, P=64, seed=T + S, kgrow=9.0)


@pytest.mark.parametrize("T,base,S,P,kgrow", [(80, 13, 1, 32, 0.0), (1024, 7, 8, 32, 0.0),
                                              (300, 40, 4, 64, 9.0), (150, 29, 1, 8, 0.0),
                                              (96, 8448, 1, 64, 0.0), (1, 0, 1, 32, 0.0),
                                              (512, 0, 1, 64, 9.0)])
def test_prefill_all_shapes(kvm, orc, dev, T, base, S, P, kgrow):
    """The three workgroup shapes: 32 query rows on 8 waves (ping-pong P.V),
    16 rows on 4 waves, and 16 rows on two 4-wave halves that take alternate
    key steps and merge their softmax states in LDS. The launch picks one per
    call; the debug hook forces each here. Every shape is held to the oracle
    tolerance, and without key splits the two 1-set shapes (same steps, same
    order) are bit-identical."""
    outs = {}
    prev = kvm.debug_prefill_shape(0)
    try:
        for shape in (0, 1, 2):
            kvm.debug_prefill_shape(shape)
            outs[shape] = run_prefill(kvm, orc, dev, T, base, S, P=P, seed=T + S, kgrow=kgrow)
    finally:
        kvm.debug_prefill_shape(prev)
    if S == 1:
        assert np.array_equal(outs[0], outs[1]), "32-row and 16-row shapes differ"
    for shape in (1, 2):
        d = np.abs(orc.bf16_to_f32(outs[0]) - orc.bf16_to_f32(outs[shape]))
        assert d.max() < 2e-2 and d.mean() < 2e-3, (shape, d.max(), d.mean())


def test_prefill_packed_jobs(kvm, orc, dev):
    """8448 rows after an 8448-token prefix: 528 jobs of similar size for 256
    CUs, where one workgroup per CU runs a fixed two- or three-job packing
    instead of greedy dispatch. Both schedules give bit-identical outputs;
    row windows at the start, middle and end are checked against the oracle
    (rows t0..t1 of a chunk are the chunk of those rows at base + t0)."""
    T, base, P = 8448, 8448, 64
    prev = kvm.debug_prefill_packing(True)
    try:
        packed, (q, pool, pt, maxp, layer) = run_prefill(kvm, orc, dev, T, base, 1, P=P,
                                                         seed=3, check=False, inputs=True)
        kvm.debug_prefill_packing(False)
        greedy = run_prefill(kvm, orc, dev, T, base, 1, P=P, seed=3, check=False)
    finally:
        kvm.debug_prefill_packing(prev)
    assert np.array_equal(packed, greedy), "packed and greedy schedules differ"
    for t0 in (0, 4200, T - 8):
        ref = orc.attn_ref(q[t0:t0 + 8], 8, base + t0, layer, pool, pt, P, maxp)
        st = orc.compare_bf16(packed[t0:t0 + 8], ref)
        assert st["rel_l2"] < 1e-2 and st["cos"] > 0.9999, (t0, st)
        assert st["max_abs"] < 2e-2 and st["mean_abs"] < 2e-3, (t0, st)


def test_prefill_bench_workload_base0(kvm, orc, dev):
    """The benchmark's prefill workload: 8448 rows at base 0 (32-row
    workgroups, greedy dispatch, causal tiles of very different weight).
    Packed and greedy settings give bit-identical outputs (packing only
    applies after a long prefix); row windows at the start, middle and end
    are checked against the oracle."""
    T, base, P = 8448, 0, 64
    prev = kvm.debug_prefill_packing(True)
    try:
        packed, (q, pool, pt, maxp, layer) = run_prefill(kvm, orc, dev, T, base, 1, P=P,
                                                         seed=4, check=False, inputs=True)
        kvm.debug_prefill_packing(False)
        greedy = run_prefill(kvm, orc, dev, T, base, 1, P=P, seed=4, check=False)
    finally:
        kvm.debug_prefill_packing(prev)
    assert np.array_equal(packed, greedy)
    for t0 in (0, 31, 4200, T - 8):
        ref = orc.attn_ref(q[t0:t0 + 8], 8, base + t0, layer, pool, pt, P, maxp)
        st = orc.compare_bf16(packed[t0:t0 + 8], ref)
        assert st["rel_l2"] < 1e-2 and st["cos"] > 0.9999, (t0, st)
        assert st["max_abs"] < 2e-2 and st["mean_abs"] < 2e-3, (t0, st)


def _random_prefill_cases(n, seed):
    import random
    rnd = random.Random(seed)
    out = []
    for i in range(n):
        T = rnd.choice([1, 2, 15, 33, 64, 100, 255, 300, 513, 700])
        base = rnd.choice([0, 0, 1, 37, 64, 500, 2047, 3000])
        S = 1 if T >= 2048 else min(8, 4096 // T)  # prefill_flash_split_kv
        if rnd.random() < 0.4:
            S = 1  # the session may pass S = 1 at any T
        P = rnd.choice([8, 16, 32, 64])
        kgrow = rnd.choice([0.0, 0.0, 4.0])
        out.append((T, base, S, P, kgrow, 3000 + i))
    return out


@pytest.mark.parametrize("shape", ["auto", 2])
@pytest.mark.parametrize("T,base,S,P,kgrow,seed", _random_prefill_cases(12, 11))
def test_prefill_random_cases(kvm, orc, dev, T, base, S, P, kgrow, seed, shape):
    """Seeded random chunks (row count, prefix, key splits, page size, growing
    key magnitude) against the oracle, under the automatic shape choice and
    with the two-half shape forced (its per-half step barriers)."""
    print(f"T={T} base={base} S={S} P={P} kgrow={kgrow} seed={seed} shape={shape}",
          flush=True)
    prev = kvm.debug_prefill_shape(kvm.PREFILL_SHAPE_AUTO if shape == "auto" else shape)
    try:
        run_prefill(kvm, orc, dev, T, base, S, P=P, seed=seed, kgrow=kgrow)
    finally:
        kvm.debug_prefill_shape(prev)
