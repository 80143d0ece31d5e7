"""GPU parity of the paged decode attention (single session, merge, phase0,
batched) against the CPU oracle.

Cases follow the reference kernel tests (native/tests/kernel_ops.cpp):
attention_decode :1618-1819 (pos 96, multi-chunk pos 599 with a permuted
19-page table, GQA probe, pos 0 == V[0]), attention_decode_chunk_tiers
:2229-2283, attention_decode_merge2 :2061-2218, attention_rope_phase0
:1958-1994 and attention_batch_vs_single :5257-5275.

Tolerances: vs the double oracle relL2 < 1e-2 and cos > 0.9999 (the
reference's criterion, kernel_ops.cpp:1595-1616) plus the task bound
max-abs 2e-2 / mean-abs 2e-3 in bf16; vs the bf16-P chunk oracle (same
16-position batch semantics) partial relL2 < 2e-3.
"""
import numpy as np
import pytest

from _util import Lcg, from_dev, randn_bf16, to_dev

pytestmark = pytest.mark.gpu

POISON = 0xDCBA


def n_records(NC, C):
    """Records per query head of a decode launch: one per workgroup range of
    ceil(NC / 256) chunks (C % 64 == 0), else one per chunk."""
    cpw = -(-NC // 256) if (C % 64 == 0 and NC > 256) else 1
    return -(-NC // cpw)


class fp32p_mode:
    """Temporarily sets the decode P.V precision (1 = fp32 P)."""

    def __init__(self, kvm, fp32_p):
        self.kvm, self.fp32_p = kvm, fp32_p

    def __enter__(self):
        self.prev = self.kvm.debug_decode_fp32p(self.fp32_p)

    def __exit__(self, *a):
        self.kvm.debug_decode_fp32p(self.prev)


def make_case(orc, P, maxp, L, layer, pt, seq, seed, lo=-1.0, hi=1.0):
    lcg = Lcg(seed)
    pool = np.full(maxp * P * 512 * L, POISON, dtype=np.uint16)
    for j in range(seq):
        base = orc.kv_off(P, maxp, layer, int(pt[j // P]), j % P, 0, 0, 0)
        pool[base:base + 512] = lcg.bf16(lo, hi, 512)
    q = np.full(2560, 0xABCD, dtype=np.uint16)  # k/v columns poisoned: not read
    q[:2048] = lcg.bf16(lo, hi, 2048)
    return pool, q


def run_decode(kvm, dev, q, pool, pt, P, maxp, L, layer, limit, C, NC, two_level=True,
               inv=None):
    import torch
    lay = kvm.KvLayout(maxp, P, L)
    d_q, d_pool = to_dev(q, dev), to_dev(pool, dev)
    d_pt = to_dev(np.asarray(pt, dtype=np.uint32), dev)
    d_pos = to_dev(np.array([limit], dtype=np.uint32), dev)
    parts = torch.full((16 * NC * 130,), float("nan"), dtype=torch.float32, device=dev)
    parts2 = torch.zeros(16 * 32 * 130, dtype=torch.float32, device=dev)
    out = torch.zeros(2048, dtype=torch.int16, device=dev)
    kvm.launch_attention_decode(d_q, d_pos, layer, d_pt, d_pool, lay, parts, NC, out,
                                d_inv_freq=inv, chunk_pos=C,
                                d_partials2=parts2 if two_level else None)
    torch.cuda.synchronize()
    return (from_dev(out), from_dev(parts, np.float32).reshape(16, NC, 130),
            from_dev(d_pool))


def check_vs_ref(orc, got, ref, tag):
    st = orc.compare_bf16(got, ref)
    print(tag, st)
    assert st["rel_l2"] < 1e-2 and st["cos"] > 0.9999, (tag, st)
    assert st["max_abs"] < 2e-2 and st["mean_abs"] < 2e-3, (tag, st)


@pytest.mark.parametrize("two_level", [True, False])
def test_decode_pos96(kvm, orc, dev, two_level):
    P, maxp, L, layer, pos = 32, 8, 1, 0, 96
    pt = np.array([7, 3, 5, 1], dtype=np.uint32)
    pool, q = make_case(orc, P, maxp, L, layer, pt, pos + 1, 0xA7E5)
    got, _, pool_after = run_decode(kvm, dev, q, pool, pt, P, maxp, L, layer, pos, 64, 12,
                                    two_level)
    ref = orc.attn_ref(q.reshape(1, 2560), 1, pos, layer, pool, pt, P, maxp)[0]
    check_vs_ref(orc, got, ref, "pos96")
    assert np.array_equal(pool_after, pool), "non-phase0 decode must not write the pool"


@pytest.mark.parametrize("two_level", [True, False])
def test_decode_multichunk_pos599(kvm, orc, dev, two_level):
    P, maxp, L, layer, pos = 32, 24, 1, 0, 599
    pt = np.array([4, 11, 2, 9, 6, 1, 13, 0, 7, 3, 5, 8, 17, 10, 15, 12, 19, 14, 22],
                  dtype=np.uint32)
    pool, q = make_case(orc, P, maxp, L, layer, pt, pos + 1, 0x3C51)
    got, parts, _ = run_decode(kvm, dev, q, pool, pt, P, maxp, L, layer, pos, 64, 12,
                               two_level)
    ref = orc.attn_ref(q.reshape(1, 2560), 1, pos, layer, pool, pt, P, maxp)[0]
    check_vs_ref(orc, got, ref, "pos599")
    # level-1 partials vs the bf16-P chunk oracle (valid chunks only)
    rparts, _ = orc.decode_chunks(q, pos, layer, pool, pt, P, maxp, 64, 12)
    nv = pos // 64 + 1
    a, r = parts[:, :nv].astype(np.float64), rparts[:, :nv].astype(np.float64)
    # m is a max (exact up to score summation order); compare l/acc after
    # rescaling both to the oracle's m.
    scale = np.exp(a[..., 0] - r[..., 0])[..., None]
    a_l = a[..., 1:] * scale
    rel = np.linalg.norm(a_l - r[..., 1:]) / np.linalg.norm(r[..., 1:])
    assert np.abs(a[..., 0] - r[..., 0]).max() < 1e-4
    assert rel < 2e-3, rel


def test_decode_gqa_probe(kvm, orc, dev):
    """K = 0.25 everywhere -> uniform softmax; V = +1 on kv head 0 and -1 on kv
    head 1, so q heads 0..7 give exactly +1 and 8..15 exactly -1."""
    P, maxp, L, layer, pos = 32, 8, 1, 0, 96
    pt = np.array([7, 3, 5, 1], dtype=np.uint32)
    pool = np.full(maxp * P * 512, POISON, dtype=np.uint16)
    kb, one, mone = orc.f32_to_bf16(np.float32([0.25, 1.0, -1.0]))
    for j in range(pos + 1):
        base = orc.kv_off(P, maxp, layer, int(pt[j // P]), j % P, 0, 0, 0)
        pool[base:base + 256] = kb
        pool[base + 256:base + 384] = one
        pool[base + 384:base + 512] = mone
    q = np.full(2560, 0xABCD, dtype=np.uint16)
    q[:2048] = Lcg(0x60A1).bf16(-1, 1, 2048)
    got, _, _ = run_decode(kvm, dev, q, pool, pt, P, maxp, L, layer, pos, 64, 12)
    f = orc.bf16_to_f32(got).reshape(16, 128)
    assert np.all(f[:8] == 1.0) and np.all(f[8:] == -1.0)


def test_decode_pos0_equals_v0(kvm, orc, dev):
    P, maxp, L, layer = 32, 8, 1, 0
    pt = np.array([7], dtype=np.uint32)
    pool, q = make_case(orc, P, maxp, L, layer, pt, 1, 0x0E9E)
    got, _, _ = run_decode(kvm, dev, q, pool, pt, P, maxp, L, layer, 0, 64, 12)
    base = orc.kv_off(P, maxp, layer, 7, 0, 0, 0, 0)
    v = pool[base + 256:base + 512].reshape(2, 128)
    assert np.array_equal(got.reshape(16, 128), np.repeat(v, 8, axis=0))


@pytest.mark.parametrize("C", [64, 128, 256, 512])
@pytest.mark.parametrize("P", [32, 64])
def test_decode_chunk_tiers(kvm, orc, dev, C, P):
    rng = np.random.default_rng(C * 7 + P)
    ctx = 2900
    maxp = -(-ctx // P) + 5
    pt = rng.permutation(maxp)[: -(-ctx // P)].astype(np.uint32)
    L, layer = 3, 2
    pool = np.full(maxp * P * 512 * L, POISON, dtype=np.uint16)
    for j in range(ctx):
        base = orc.kv_off(P, maxp, layer, int(pt[j // P]), j % P, 0, 0, 0)
        pool[base:base + 512] = randn_bf16(rng, 512, 1 / np.sqrt(128) ** 0.5)
    q = randn_bf16(rng, 2560, 1.0)
    NC = -(-4096 // C)
    limit = ctx - 1
    got, _, _ = run_decode(kvm, dev, q, pool, pt, P, maxp, L, layer, limit, C, NC)
    ref = orc.attn_ref(q.reshape(1, 2560), 1, limit, layer, pool, pt, P, maxp)[0]
    check_vs_ref(orc, got, ref, f"tier C={C} P={P}")


@pytest.mark.parametrize("C", [64, 128, 48])
@pytest.mark.parametrize("P", [1, 4, 8])
@pytest.mark.parametrize("ph0", [False, True])
def test_decode_small_pages(kvm, orc, dev, C, P, ph0):
    """Pages smaller than a 16-position tile: page ids looked up per position
    (both tile-load layouts: C = 64 uses whole-row loads, C = 128 operand-
    layout loads, C = 48 the generic schedule)."""
    import torch
    rng = np.random.default_rng(C * 31 + P + ph0)
    ctx = 777
    maxp = -(-ctx // P) + 3
    pt = rng.permutation(maxp)[: -(-ctx // P)].astype(np.uint32)
    L, layer = 2, 1
    pool = np.full(maxp * P * 512 * L, POISON, dtype=np.uint16)
    n_fill = ctx - 1 if ph0 else ctx
    for j in range(n_fill):
        base = orc.kv_off(P, maxp, layer, int(pt[j // P]), j % P, 0, 0, 0)
        pool[base:base + 512] = randn_bf16(rng, 512, 0.5)
    q = randn_bf16(rng, 2560, 1.0)
    NC = -(-1024 // C)
    limit = ctx - 1
    inv = None
    if ph0:
        inv = torch.empty(64, dtype=torch.float32, device=dev)
        kvm.launch_rope_inv_freq_init(inv, 5e6)
    got, _, pool_after = run_decode(kvm, dev, q, pool, pt, P, maxp, L, layer, limit, C, NC,
                                    inv=inv)
    qkv_o, pool_o = q.reshape(1, 2560).copy(), pool.copy()
    if ph0:
        orc.rope_append(qkv_o, 1, limit, layer, pt, P, maxp, 5e6, 1, pool_o)
        assert np.array_equal(pool_after, pool_o)
    ref = orc.attn_ref(qkv_o, 1, limit, layer, pool_o, pt, P, maxp)[0]
    check_vs_ref(orc, got, ref, f"small pages C={C} P={P} ph0={ph0}")


@pytest.mark.parametrize("N,limit", [(257, 257 * 64 - 1), (257, 5 * 64 + 10),
                                     (512, 512 * 64 - 1), (512, 33 * 64),
                                     (2048, 2048 * 64 - 1), (2048, 700 * 64 + 3)])
def test_merge2_synthetic(kvm, orc, dev, N, limit):
    """Fixed random level-1 partials with l == 0 holes and a poisoned tail
    (kernel_ops.cpp:2061-2218): two-level merge vs the double oracle, with
    16 (N <= 512) and 64 (N = 2048) chunks per level-2 split."""
    import torch
    C = 64
    nv = min(limit // C + 1, N)
    lcg = Lcg(0xA12E + (0 if limit > 1000 else 7919))
    parts = np.empty((16, N, 130), dtype=np.float32)
    for qh in range(16):
        for c in range(N):
            if c >= nv:
                parts[qh, c] = 1e30
                continue
            parts[qh, c, 0] = lcg.uniform(-8, 8, 1)[0]
            parts[qh, c, 1] = 0.0 if c % 7 == 3 else lcg.uniform(0.5, 4.0, 1)[0]
            parts[qh, c, 2:] = lcg.uniform(-2, 2, 128)
    lvl2_ref, out_ref = orc.merge2(parts, N, nv)
    d_parts = to_dev(parts, dev)
    d_pos = to_dev(np.array([limit], dtype=np.uint32), dev)
    d_p2 = torch.zeros(16 * 32 * 130, dtype=torch.float32, device=dev)
    out = torch.zeros(2048, dtype=torch.int16, device=dev)
    kvm.launch_attention_decode_merge(d_parts, d_pos, N, C, d_p2, out)
    torch.cuda.synchronize()
    got = from_dev(out)
    a = orc.bf16_to_f32(got).astype(np.float64)
    r = orc.bf16_to_f32(out_ref).astype(np.float64)
    ulp = orc.bf16_ulp(r)
    assert np.all(np.abs(a - r) <= ulp + 1e-30), np.abs(a - r).max()
    p2 = from_dev(d_p2, np.float32).reshape(16, 32, 130)
    valid = lvl2_ref[..., 1] != 0
    g, w = p2[valid].astype(np.float64), lvl2_ref[valid].astype(np.float64)
    rel = np.linalg.norm(g - w) / np.linalg.norm(w)
    assert rel < 1e-6, rel


@pytest.mark.parametrize("limit", [75, 1000])
def test_phase0_matches_rope_then_attend(kvm, orc, dev, limit):
    """Fused append (phase0) vs the two-kernel chain rope_append -> attention:
    output, pool and qkv row bit-identical (kernel_ops.cpp:1958-1994)."""
    import torch
    rng = np.random.default_rng(limit)
    P, maxp, L, layer = 32, 40, 2, 1
    pt = rng.permutation(maxp).astype(np.uint32)
    pool = np.full(maxp * P * 512 * L, POISON, dtype=np.uint16)
    for j in range(limit):
        base = orc.kv_off(P, maxp, layer, int(pt[j // P]), j % P, 0, 0, 0)
        pool[base:base + 512] = randn_bf16(rng, 512, 0.5)
    qkv = randn_bf16(rng, 2560, 1.0)
    lay = kvm.KvLayout(maxp, P, L)
    inv = torch.empty(64, dtype=torch.float32, device=dev)
    kvm.launch_rope_inv_freq_init(inv, 5e6)
    NC = 20
    # chain A: rope kernel then plain attention
    d_qkv_a, d_pool_a = to_dev(qkv, dev), to_dev(pool, dev)
    d_pt = to_dev(pt, dev)
    d_pos = to_dev(np.array([limit], dtype=np.uint32), dev)
    kvm.launch_rope_kv(d_qkv_a, 1, d_pos, layer, d_pt, d_pool_a, lay, 5e6, d_inv_freq=inv)
    pa = torch.empty(16 * NC * 130, dtype=torch.float32, device=dev)
    p2 = torch.zeros(16 * 32 * 130, dtype=torch.float32, device=dev)
    out_a = torch.zeros(2048, dtype=torch.int16, device=dev)
    kvm.launch_attention_decode(d_qkv_a, d_pos, layer, d_pt, d_pool_a, lay, pa, NC, out_a,
                                chunk_pos=64, d_partials2=p2)
    # chain B: phase0
    d_qkv_b, d_pool_b = to_dev(qkv, dev), to_dev(pool, dev)
    pb = torch.empty(16 * NC * 130, dtype=torch.float32, device=dev)
    out_b = torch.zeros(2048, dtype=torch.int16, device=dev)
    kvm.launch_attention_decode(d_qkv_b, d_pos, layer, d_pt, d_pool_b, lay, pb, NC, out_b,
                                d_inv_freq=inv, chunk_pos=64, d_partials2=p2)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(d_pool_a), from_dev(d_pool_b))
    assert np.array_equal(from_dev(out_a), from_dev(out_b))
    assert np.array_equal(from_dev(d_qkv_b), qkv), "phase0 must not modify the qkv row"
    # pool vs kernel-exact oracle, output vs double oracle
    qkv_o, pool_o = qkv.reshape(1, 2560).copy(), pool.copy()
    orc.rope_append(qkv_o, 1, limit, layer, pt, P, maxp, 5e6, 1, pool_o)
    assert np.array_equal(from_dev(d_pool_b), pool_o)
    ref = orc.attn_ref(qkv_o, 1, limit, layer, pool_o, pt, P, maxp)[0]
    check_vs_ref(orc, from_dev(out_b), ref, f"phase0 limit={limit}")


def _batch_case(kvm, orc, dev, B, C, ctx, ph0, seed, step=37, P=32):
    import torch
    rng = np.random.default_rng(seed)
    L, layer = 2, 1
    pages_per = -(-(ctx + 1) // P)
    maxp = pages_per * B + 3  # shared pool, pages of all slots interleaved
    perm = rng.permutation(maxp).astype(np.uint32)
    pts = [perm[s::B][:pages_per].copy() for s in range(B)]
    pool = np.full(maxp * P * 512 * L, POISON, dtype=np.uint16)
    limits = [ctx - step * s for s in range(B)]
    for s in range(B):
        for j in range(limits[s] + (0 if ph0 else 1)):
            base = orc.kv_off(P, maxp, layer, int(pts[s][j // P]), j % P, 0, 0, 0)
            pool[base:base + 512] = randn_bf16(rng, 512, 0.5)
    q = randn_bf16(rng, B * 2560, 1.0).reshape(B, 2560)
    lay = kvm.KvLayout(maxp, P, L)
    NC = -(-(ctx + 64) // C)
    inv = None
    if ph0:
        inv = torch.empty(64, dtype=torch.float32, device=dev)
        kvm.launch_rope_inv_freq_init(inv, 5e6)
    # batched run on one pool
    d_pool = to_dev(pool, dev)
    d_q = to_dev(q.ravel(), dev)
    d_pts = [to_dev(t, dev) for t in pts]
    d_lims = [to_dev(np.array([l], dtype=np.uint32), dev) for l in limits]
    tab = lambda ts: torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64,
                                  device=dev)
    parts = torch.zeros(B * 16 * NC * 130, dtype=torch.float32, device=dev)
    parts2 = torch.zeros(B * (16 * 32 * 130), dtype=torch.float32, device=dev)
    out = torch.zeros(B * 2048, dtype=torch.int16, device=dev)
    kvm.launch_attention_decode_batch(d_q, tab(d_lims), B, layer, tab(d_pts),
                                      tab([d_pool] * B), lay, parts, NC, out, d_inv_freq=inv,
                                      chunk_pos=C, d_partials2=parts2)
    torch.cuda.synchronize()
    got = from_dev(out).reshape(B, 2048)
    pool_b = from_dev(d_pool)
    # single-session runs on a second copy of the pool
    d_pool1 = to_dev(pool, dev)
    singles = []
    nrec = 16 * n_records(NC, C) * 130  # a slot's records (the rest is unused)
    parts_b = from_dev(parts, np.float32)[:B * nrec].reshape(B, nrec)
    parts2_b = from_dev(parts2, np.float32).reshape(B, 16 * 32 * 130)
    for s in range(B):
        p1 = torch.zeros(16 * NC * 130, dtype=torch.float32, device=dev)
        p2 = torch.zeros(16 * 32 * 130, dtype=torch.float32, device=dev)
        o1 = torch.zeros(2048, dtype=torch.int16, device=dev)
        kvm.launch_attention_decode(to_dev(q[s], dev), d_lims[s], layer, d_pts[s], d_pool1,
                                    lay, p1, NC, o1, d_inv_freq=inv, chunk_pos=C,
                                    d_partials2=p2)
        torch.cuda.synchronize()
        singles.append(from_dev(o1))
        # partials and level-2 partials too (bytes, so NaN payloads compare)
        assert np.array_equal(from_dev(p1, np.uint32)[:nrec], parts_b[s].view(np.uint32)), s
        assert np.array_equal(from_dev(p2, np.uint32), parts2_b[s].view(np.uint32)), s
    assert np.array_equal(got, np.stack(singles)), "batched != single (bitwise)"
    assert np.array_equal(pool_b, from_dev(d_pool1))
    # vs oracle
    pool_o = pool.copy()
    for s in range(B):
        qkv_o = q[s].reshape(1, 2560).copy()
        if ph0:
            orc.rope_append(qkv_o, 1, limits[s], layer, pts[s], P, maxp, 5e6, 1, pool_o)
        ref = orc.attn_ref(qkv_o, 1, limits[s], layer, pool_o, pts[s], P, maxp)[0]
        check_vs_ref(orc, got[s], ref, f"batch B={B} C={C} slot={s}")
    if ph0:
        assert np.array_equal(pool_b, pool_o)


@pytest.mark.parametrize("B", [2, 4, 8])
@pytest.mark.parametrize("C", [64, 128, 256])
@pytest.mark.parametrize("ph0", [False, True])
def test_batch_vs_single_ctx600(kvm, orc, dev, B, C, ph0):
    _batch_case(kvm, orc, dev, B, C, 600, ph0, seed=B * 100 + C + ph0)


@pytest.mark.parametrize("P", [32, 64])
def test_batch_vs_single_8x2048(kvm, orc, dev, P):
    """Config C3's shape (8 sessions x 2048 context, 64-position chunks) at
    both page sizes, P = 64 being the benchmark's."""
    _batch_case(kvm, orc, dev, 8, 64, 2047, True, seed=8 + P, P=P)


@pytest.mark.parametrize("B,C,ctx", [(4, 64, 600), (3, 256, 9000), (2, 128, 20000)])
def test_batch_vs_single_page64(kvm, orc, dev, B, C, ctx):
    """64-token pages (one page id per 16-position tile, several tiles per
    page) through the batched and single-session kernels."""
    _batch_case(kvm, orc, dev, B, C, ctx, True, seed=B + C, P=64)


@pytest.mark.parametrize("C,ph0", [(64, True), (256, False)])
def test_batch_vs_single_two_level(kvm, orc, dev, C, ph0):
    """More than 32 chunks: batched level-1 and level-2 partials and outputs
    bit-identical to single-session runs."""
    _batch_case(kvm, orc, dev, 4, C, 9000, ph0, seed=C + 1)


@pytest.mark.parametrize("B,C", [(24, 64), (17, 256), (64, 64), (9, 512)])
def test_batch_vs_single_many_slots(kvm, orc, dev, B, C):
    """More than 16 slots (the batched kernel maps workgroups to slots with a
    wave-wide scan instead of scalar registers) and ragged limits: outputs and
    partials bit-identical to single-session runs, and within tolerance of
    the oracle."""
    _batch_case(kvm, orc, dev, B, C, 700, True, seed=B * 7 + C, step=9)


def test_batch_vs_single_both_heads_per_workgroup(kvm, orc, dev):
    """128K tier (C = 256, 512 chunks): single-session launches put both KV
    heads in one 512-thread workgroup, batched launches one head per
    workgroup; partials, level-2 partials and outputs stay bit-identical."""
    _batch_case(kvm, orc, dev, 2, 256, 131000, True, seed=0x2C4)


@pytest.mark.parametrize("ctx,C,ph0,P", [(40000, 64, True, 64), (131072, 256, True, 64),
                                         (70001, 256, False, 64), (131072, 512, True, 64),
                                         (90001, 512, False, 64), (131072, 256, True, 16)])
def test_decode_long_multichunk_blocks(kvm, orc, dev, ctx, C, ph0, P):
    """Long contexts where one workgroup streams several chunks (2x512+
    chunk units), permuted pages of P tokens; phase0 appends position ctx-1."""
    import torch
    rng = np.random.default_rng(ctx + P)
    L, layer = 2, 1
    maxp = -(-ctx // P) + 2
    pt = rng.permutation(maxp).astype(np.uint32)
    lay = kvm.KvLayout(maxp, P, L)
    pool = np.full(lay.total_elems(), POISON, dtype=np.uint16)
    n_fill = ctx - 1 if ph0 else ctx
    vals = randn_bf16(rng, n_fill * 512, 0.3)
    for j in range(n_fill):
        base = orc.kv_off(P, maxp, layer, int(pt[j // P]), j % P, 0, 0, 0)
        pool[base:base + 512] = vals[j * 512:(j + 1) * 512]
    q = randn_bf16(rng, 2560, 1.0)
    limit = ctx - 1
    NC = -(-131072 // C)
    inv = None
    if ph0:
        inv = torch.empty(64, dtype=torch.float32, device=dev)
        kvm.launch_rope_inv_freq_init(inv, 5e6)
    got, _, pool_after = run_decode(kvm, dev, q, pool, pt, P, maxp, L, layer, limit, C, NC,
                                    inv=inv)
    qkv_o, pool_o = q.reshape(1, 2560).copy(), pool.copy()
    if ph0:
        orc.rope_append(qkv_o, 1, limit, layer, pt, P, maxp, 5e6, 1, pool_o)
        assert np.array_equal(pool_after, pool_o)
    ref = orc.attn_ref(qkv_o, 1, limit, layer, pool_o, pt, P, maxp)[0]
    check_vs_ref(orc, got, ref, f"long ctx={ctx} C={C}")


@pytest.mark.parametrize("ctx,C", [(2048, 64), (3000, 64), (40000, 128)])
def test_repeat_launch_and_graph_replay(kvm, orc, dev, ctx, C):
    """Repeated eager launches on the same scratch buffers give identical
    outputs, and a captured HIP graph replayed several times (the limit
    advanced by an eager device op between replays) matches eager launches
    every time."""
    import torch
    rng = np.random.default_rng(ctx)
    P, L, layer = 64, 1, 0
    maxp = -(-(ctx + 8) // P)
    pt = rng.permutation(maxp).astype(np.uint32)
    lay = kvm.KvLayout(maxp, P, L)
    pool = randn_bf16(rng, lay.total_elems(), 0.4)
    q = randn_bf16(rng, 2560, 1.0)
    NC = -(-(ctx + 8) // C)
    d_pool, d_q, d_pt = to_dev(pool, dev), to_dev(q, dev), to_dev(pt, dev)
    parts = torch.zeros(16 * NC * 130, dtype=torch.float32, device=dev)
    parts2 = torch.zeros(16 * 32 * 130, dtype=torch.float32, device=dev)
    d_pos = torch.tensor([ctx - 1], dtype=torch.int32, device=dev)

    def run(out):
        kvm.launch_attention_decode(d_q, d_pos, layer, d_pt, d_pool, lay, parts, NC, out,
                                    chunk_pos=C, d_partials2=parts2)
    eager = []
    for _ in range(3):
        o = torch.zeros(2048, dtype=torch.int16, device=dev)
        run(o)
        torch.cuda.synchronize()
        eager.append(from_dev(o))
    assert all(np.array_equal(eager[0], e) for e in eager[1:])
    ref = orc.attn_ref(q.reshape(1, 2560), 1, ctx - 1, layer, pool, pt, P, maxp)[0]
    check_vs_ref(orc, eager[0], ref, f"fused ctx={ctx}")
    # graph capture of one launch; replays at limits ctx-1, ctx, ..., ctx+3
    gout = torch.zeros(2048, dtype=torch.int16, device=dev)
    run(gout)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run(gout)
    for k in range(4):
        d_pos.fill_(ctx - 1 + k)
        g.replay()
        torch.cuda.synchronize()
        got = from_dev(gout)
        e = torch.zeros(2048, dtype=torch.int16, device=dev)
        run(e)
        torch.cuda.synchronize()
        assert np.array_equal(got, from_dev(e)), f"replay {k}"


def _random_batch_cases(n, seed):
    import random
    rnd = random.Random(seed)
    out = []
    for i in range(n):
        B = rnd.choice([1, 2, 3, 5, 8, 13, 20])
        C = rnd.choice([64, 128, 256, 512, 48, 80])
        ctx = rnd.choice([40, 300, 1000, 2500, 6000, 12000])
        ph0 = rnd.random() < 0.5
        step = max(0, min(rnd.choice([0, 1, 9, 37, 200]), (ctx - 2) // B))
        out.append((B, C, ctx, ph0, step, 2000 + i))
    return out


@pytest.mark.parametrize("B,C,ctx,ph0,step,seed", _random_batch_cases(12, 7))
def test_batch_random_cases(kvm, orc, dev, B, C, ctx, ph0, step, seed):
    """Seeded random batched cases (slot count, chunk tier incl. non-multiples
    of 64, context, phase0, ragged limits): bit-identical to single-session
    calls and within tolerance of the oracle."""
    print(f"B={B} C={C} ctx={ctx} ph0={ph0} step={step} seed={seed}", flush=True)
    _batch_case(kvm, orc, dev, B, C, ctx, ph0, seed=seed, step=step)


def test_reuse_buffers_new_data(kvm, orc, dev):
    """Back-to-back launches on the same scratch buffers with different
    queries and limits: each output matches a fresh computation (no stale
    record of an earlier call is ever folded)."""
    import torch
    rng = np.random.default_rng(77)
    P, L, layer, C = 64, 1, 0, 256
    ctx = 40000
    maxp = -(-ctx // P) + 1
    pt = rng.permutation(maxp).astype(np.uint32)
    lay = kvm.KvLayout(maxp, P, L)
    pool = randn_bf16(rng, lay.total_elems(), 0.4)
    d_pool, d_pt = to_dev(pool, dev), to_dev(pt, dev)
    NC = -(-ctx // C)
    parts = torch.zeros(16 * NC * 130, dtype=torch.float32, device=dev)
    parts2 = torch.zeros(16 * 32 * 130, dtype=torch.float32, device=dev)
    out = torch.zeros(2048, dtype=torch.int16, device=dev)
    for it, limit in enumerate([ctx - 1, 300, 17000, 5, ctx - 2, 256 * 40]):
        q = randn_bf16(rng, 2560, 1.0)
        d_q = to_dev(q, dev)
        d_pos = to_dev(np.array([limit], dtype=np.uint32), dev)
        for _ in range(3):
            kvm.launch_attention_decode(d_q, d_pos, layer, d_pt, d_pool, lay, parts, NC, out,
                                        chunk_pos=C, d_partials2=parts2)
        torch.cuda.synchronize()
        ref = orc.attn_ref(q.reshape(1, 2560), 1, limit, layer, pool, pt, P, maxp)[0]
        check_vs_ref(orc, from_dev(out), ref, f"reuse it={it} limit={limit}")


@pytest.mark.parametrize("C,limit,P", [(64, 599, 32), (64, 40, 64), (256, 3000, 64),
                                       (48, 777, 8), (128, 2000, 4)])
def test_fp32p_chunks_vs_oracle(kvm, orc, dev, C, limit, P):
    """fp32-P mode (the reference's MC_ATTN_HMMA_OFF fallback): per-chunk
    partials of the chunk kernel vs the fp32-P chunk oracle, which differs
    from the GPU only in summation order (relL2 < 2e-5 after rescaling to the
    oracle's m; the bf16-P partials differ from it by far more)."""
    import torch
    rng = np.random.default_rng(C + limit + P)
    maxp = -(-(limit + 1) // P) + 2
    pt = rng.permutation(maxp).astype(np.uint32)
    L, layer = 2, 1
    lay = kvm.KvLayout(maxp, P, L)
    pool = randn_bf16(rng, lay.total_elems(), 0.5)
    q = randn_bf16(rng, 2560, 1.0)
    NC = -(-(limit + 1) // C) + 1
    d_q, d_pool, d_pt = to_dev(q, dev), to_dev(pool, dev), to_dev(pt, dev)
    d_pos = to_dev(np.array([limit], dtype=np.uint32), dev)
    got = {}
    for fp in (1, 0):
        with fp32p_mode(kvm, fp):
            parts = torch.full((16 * NC * 130,), float("nan"), dtype=torch.float32, device=dev)
            out = torch.zeros(2048, dtype=torch.int16, device=dev)
            kvm.launch_attention_decode_chunks(d_q, d_pos, layer, d_pt, d_pool, lay, parts, NC,
                                               out, chunk_pos=C)
            torch.cuda.synchronize()
            got[fp] = (from_dev(parts, np.float32).reshape(16, NC, 130), from_dev(out))
    rparts, rout = orc.decode_chunks(q, limit, layer, pool, pt, P, maxp, C, NC, fp32_p=True)
    nv = limit // C + 1
    if nv == 1:  # single chunk: the kernel writes the output, not partials
        a = orc.bf16_to_f32(got[1][1]).astype(np.float64)
        r = orc.bf16_to_f32(rout).astype(np.float64)
        assert np.all(np.abs(a - r) <= orc.bf16_ulp(r) + 1e-30), np.abs(a - r).max()
        return
    rel = {}
    for fp in (1, 0):
        a, r = got[fp][0][:, :nv].astype(np.float64), rparts[:, :nv].astype(np.float64)
        assert np.abs(a[..., 0] - r[..., 0]).max() < 1e-4
        scale = np.exp(a[..., 0] - r[..., 0])[..., None]
        rel[fp] = np.linalg.norm(a[..., 1:] * scale - r[..., 1:]) / np.linalg.norm(r[..., 1:])
    assert rel[1] < 2e-5, rel
    assert rel[0] > 4 * rel[1], rel


@pytest.mark.parametrize("B,C,ctx,ph0", [(1, 64, 2048, True), (1, 256, 131072, True),
                                         (4, 128, 9000, False), (8, 64, 2048, True),
                                         (2, 48, 3000, True)])
def test_fp32p_decode_vs_oracle(kvm, orc, dev, B, C, ctx, ph0):
    """fp32-P decode outputs (single and batched) within the attention
    tolerance of the double oracle, and batched == single."""
    with fp32p_mode(kvm, 1):
        _batch_case(kvm, orc, dev, B, C, ctx, ph0, seed=ctx + B, P=64)


@pytest.mark.parametrize("ctx,C,nc_ctx,chunk_wgs,merge_wgs",
                         [(600, 64, 600, 20, 16), (40000, 64, 131072, 512, 64)])
def test_decode_timeline_hook(kvm, dev, ctx, C, nc_ctx, chunk_wgs, merge_wgs):
    """With the timeline buffer attached, a decode records one stamp pair per
    chunk-kernel and merge workgroup (entry <= exit, the chunk kernel ending
    before the merge starts) in the first region of the ring, the outputs
    stay bit-identical to a launch without it, and detaching stops the
    stamps."""
    import torch
    rng = np.random.default_rng(ctx)
    P, L, layer = 64, 1, 0
    maxp = -(-ctx // P) + 1
    pt = rng.permutation(maxp).astype(np.uint32)
    pool = randn_bf16(rng, maxp * P * 512 * L, 0.3)
    q = randn_bf16(rng, 2560, 1.0)
    NC = kvm.attention_decode_max_chunks(nc_ctx, C)
    ref, _, _ = run_decode(kvm, dev, q, pool, pt, P, maxp, L, layer, ctx - 1, C, NC)
    buf = torch.zeros(3 * kvm.TIMELINE_WORDS, dtype=torch.int64, device=dev)
    kvm.debug_decode_timeline(buf, 3)
    try:
        got, _, _ = run_decode(kvm, dev, q, pool, pt, P, maxp, L, layer, ctx - 1, C, NC)
    finally:
        kvm.debug_decode_timeline(None, 0)
    assert np.array_equal(got, ref)
    st = from_dev(buf, np.int64).reshape(3, kvm.TIMELINE_WORDS)
    ck = st[0, :4 * kvm.TIMELINE_CHUNK_WGS].reshape(-1, 4)
    mg = st[0, 4 * kvm.TIMELINE_CHUNK_WGS:].reshape(-1, 2)
    assert (ck[:chunk_wgs, 0] > 0).all() and not ck[chunk_wgs:].any()
    assert (ck[:chunk_wgs, 1] >= ck[:chunk_wgs, 0]).all()
    # first K/V tile in registers: between the workgroup's entry and exit
    # (one per workgroup whose range holds streamed positions 0..ctx-2)
    cpw = -(-NC // 256) if NC > 256 else 1
    fd = ck[:chunk_wgs][ck[:chunk_wgs, 3] > 0]
    assert len(fd) == 2 * -(-(ctx - 1) // (C * cpw))
    assert (fd[:, 3] >= fd[:, 0]).all() and (fd[:, 3] <= fd[:, 1]).all()
    assert (mg[:merge_wgs, 0] > 0).all() and not mg[merge_wgs:].any()
    assert (mg[:merge_wgs, 1] >= mg[:merge_wgs, 0]).all()
    assert mg[:merge_wgs, 0].min() >= ck[:chunk_wgs, 1].max()
    assert not st[1:].any()
    summ = kvm.timeline_summary(st)
    assert summ["decodes"] == 1 and summ["chunk_span"] > 0 and summ["merge_span"] > 0
    assert summ["wg_entry_to_first_data"] > 0 and summ["wg_first_data_to_exit"] >= 0
    run_decode(kvm, dev, q, pool, pt, P, maxp, L, layer, ctx - 1, C, NC)
    assert np.array_equal(from_dev(buf, np.int64).reshape(3, -1), st)
