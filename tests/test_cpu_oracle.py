"""CPU tests that pin the oracle (oracle/kv_oracle.c) before it is trusted as
the checker of the HIP kernels. Each check uses an independent formulation
(libm / numpy / torch) or a closed form, chosen so a dropped term, a wrong
sign or index or a transposed operand in the oracle fails one of them."""
import math

import numpy as np
import pytest

from _util import Lcg, randn_bf16


# ---------------- bf16 rounding ----------------

def test_bf16_rne_matches_torch(orc):
    import torch
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * 10,
        np.float32([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 65504.0, 3e38, -3e38, 1e-40]),
        # exact ties: low 16 bits == 0x8000 with even / odd upper parts
        np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x3F80FFFF, 0x3F807FFF],
                 dtype=np.uint32).view(np.float32),
    ])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.f32_to_bf16(x), want)
    lib = orc.lib()
    for v in x[-20:]:
        assert lib.orc_f2bf(float(v)) == orc.f32_to_bf16(np.float32([v]))[0]


# ---------------- RoPE ----------------

def test_rope_sincos_vs_libm(orc):
    """cos/sin of fp32 angles pos*inv_freq over the whole 128K position range
    equal libm's double cos/sin rounded to fp32 (all within 1 fp32 ulp, and
    bit-equal for >= 99.99%)."""
    inv = orc.inv_freq(5e6).astype(np.float32)
    pos = np.arange(0, 131072, 3, dtype=np.float32)
    ang = (pos[:, None] * inv[None, :]).astype(np.float32).ravel()
    extra = np.float32([0.0, 1e-30, 0.7853981, 0.7853982, 1.5707964, 3.1415927, 4.712389,
                        6.2831855, 100000.0, 131071.0, 1.6e6])
    ang = np.concatenate([ang, extra])
    c, s = orc.rope_sincos(ang)
    rc = np.cos(ang.astype(np.float64)).astype(np.float32)
    rs = np.sin(ang.astype(np.float64)).astype(np.float32)
    ulp = lambda r: np.spacing(np.abs(r)).astype(np.float64)
    assert np.all(np.abs(c.astype(np.float64) - rc) <= ulp(rc))
    assert np.all(np.abs(s.astype(np.float64) - rs) <= ulp(rs))
    assert (np.mean(c == rc) > 0.9999) and (np.mean(s == rs) > 0.9999)


def test_inv_freq_matches_python_formula(orc):
    """tools/reference_forward.py:187: theta ** -(arange(0,128,2)/128) in
    float64, cast to float32."""
    for th in (1e4, 5e6):
        want = (th ** -(np.arange(0, 128, 2, dtype=np.float64) / 128.0)).astype(np.float32)
        assert np.array_equal(orc.inv_freq(th), want)


def _rope_complex(qkv, T, base, theta):
    """Independent statement: rotate_half on (x_lo + i x_hi) is a complex
    multiply by e^{i*angle} with angle = pos * theta^(-p/64) in double."""
    x = orc_bf = None
    out = qkv.reshape(T, 2560).copy()
    import oracle
    f = oracle.bf16_to_f32(out[:, :2304]).astype(np.float64).reshape(T, 18, 128)
    p = np.arange(64, dtype=np.float64)
    ang = (base + np.arange(T, dtype=np.float64))[:, None] * theta ** (-p / 64.0)[None, :]
    z = (f[:, :, :64] + 1j * f[:, :, 64:]) * np.exp(1j * ang)[:, None, :]
    rot = np.concatenate([z.real, z.imag], axis=2).astype(np.float32)
    return oracle.f32_to_bf16(rot).reshape(T, 2304)


@pytest.mark.parametrize("T,base", [(1, 75), (70, 0), (5, 8447)])
def test_rope_double_oracle_is_complex_rotation(orc, T, base):
    rng = np.random.default_rng(T)
    qkv = randn_bf16(rng, T * 2560, 1.0).reshape(T, 2560)
    P, maxp = 32, (base + T) // 32 + 2
    pt = np.arange(maxp, dtype=np.uint32)[::-1].copy()
    pool = np.zeros(maxp * P * 512, dtype=np.uint16)
    q0 = qkv.copy()
    orc.rope_append(q0, T, base, 0, pt, P, maxp, 5e6, 0, pool)
    want = _rope_complex(qkv, T, base, 5e6)
    got_q = q0[:, :2048]
    got_k = np.stack([pool[orc.kv_off(P, maxp, 0, int(pt[(base + t) // P]), (base + t) % P, 0, 0, 0):][:256]
                      for t in range(T)])
    a = orc.bf16_to_f32(np.concatenate([got_q, got_k], axis=1))
    r = orc.bf16_to_f32(want)
    assert np.all(np.abs(a - r) <= orc.bf16_ulp(r) * 1.0 + 1e-30)  # <= 1 ulp (double rounding)
    v = np.stack([pool[orc.kv_off(P, maxp, 0, int(pt[(base + t) // P]), (base + t) % P, 1, 0, 0):][:256]
                  for t in range(T)])
    assert np.array_equal(v, qkv[:, 2304:])


def test_rope_pos0_identity(orc):
    qkv = Lcg(0x00B1).bf16(-2, 2, 2560).reshape(1, 2560)
    for mode in (0, 1):
        q, pool = qkv.copy(), np.zeros(8 * 32 * 512, dtype=np.uint16)
        orc.rope_append(q, 1, 0, 0, np.array([2], np.uint32), 32, 8, 5e6, mode, pool)
        assert np.array_equal(q, qkv)
        off = orc.kv_off(32, 8, 0, 2, 0, 0, 0, 0)
        assert np.array_equal(pool[off:off + 256], qkv[0, 2048:2304])


@pytest.mark.parametrize("theta", [1e4, 5e6])
def test_rope_exact_within_reference_tolerance(orc, theta):
    """The kernel-exact statement (mode 1, what the GPU matches bit-for-bit)
    vs the reference's double rope_ref (mode 0): <= 2 bf16 ulp + 1e-4 plus the
    fp32-angle rounding term (|x| + |x2|) * 2^-23 * pos * inv_freq."""
    T, base = 600, 8000
    rng = np.random.default_rng(int(theta))
    qkv = randn_bf16(rng, T * 2560, 1.0).reshape(T, 2560)
    P, maxp = 64, (base + T) // 64 + 1
    pt = np.arange(maxp, dtype=np.uint32)
    q0, q1 = qkv.copy(), qkv.copy()
    p0 = np.zeros(maxp * P * 512, np.uint16)
    p1 = p0.copy()
    orc.rope_append(q0, T, base, 0, pt, P, maxp, theta, 0, p0)
    orc.rope_append(q1, T, base, 0, pt, P, maxp, theta, 1, p1)
    inv = orc.inv_freq(theta).astype(np.float64)
    pos = (base + np.arange(T, dtype=np.float64))[:, None]
    d = np.arange(128)
    src = orc.bf16_to_f32(qkv[:, :2048]).astype(np.float64).reshape(T, 16, 128)
    tol = (2 * orc.bf16_ulp(orc.bf16_to_f32(q0[:, :2048])).reshape(T, 16, 128) + 1e-4 +
           (np.abs(src) + np.abs(src[:, :, d ^ 64])) * (2.0 ** -23 * pos * inv[d % 64])[:, None, :])
    diff = np.abs(orc.bf16_to_f32(q1[:, :2048]) - orc.bf16_to_f32(q0[:, :2048])).reshape(T, 16, 128)
    assert np.all(diff <= tol)
    assert np.mean(q1 == q0) > 0.95  # mostly identical bits


# ---------------- attention ----------------

def _np_attention(q, pool, pt, P, maxp, limit, layer=0):
    """numpy float64 softmax attention of one query row (independent)."""
    out = np.zeros((16, 128))
    for h in range(16):
        kvh = h // 8
        K = np.stack([orc_kv(pool, P, maxp, layer, pt, j, 0, kvh) for j in range(limit + 1)])
        V = np.stack([orc_kv(pool, P, maxp, layer, pt, j, 1, kvh) for j in range(limit + 1)])
        s = K @ q[h] / math.sqrt(128.0)
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ V
    return out


def orc_kv(pool, P, maxp, layer, pt, j, kv, kvh):
    import oracle
    off = oracle.kv_off(P, maxp, layer, int(pt[j // P]), j % P, kv, kvh, 0)
    return oracle.bf16_to_f32(pool[off:off + 128]).astype(np.float64)


def _rand_case(orc, seed, ctx, P=32):
    rng = np.random.default_rng(seed)
    maxp = -(-ctx // P) + 2
    pt = rng.permutation(maxp).astype(np.uint32)
    pool = randn_bf16(rng, maxp * P * 512, 0.5)
    q = randn_bf16(rng, 2560, 1.0)
    return q, pool, pt, P, maxp


def test_attn_ref_matches_numpy(orc):
    q, pool, pt, P, maxp = _rand_case(orc, 1, 130)
    got = orc.bf16_to_f32(orc.attn_ref(q.reshape(1, 2560), 1, 129, 0, pool, pt, P, maxp)[0])
    want = _np_attention(orc.bf16_to_f32(q[:2048]).reshape(16, 128).astype(np.float64),
                         pool, pt, P, maxp, 129)
    assert np.all(np.abs(got.reshape(16, 128) - want) <= orc.bf16_ulp(want) * 0.5 + 1e-7)


def test_attn_ref_gqa_probe_and_pos0(orc):
    P, maxp = 32, 8
    pt = np.array([7, 3, 5, 1], np.uint32)
    pool = np.full(maxp * P * 512, 0xDCBA, np.uint16)
    kb, one, mone = orc.f32_to_bf16(np.float32([0.25, 1.0, -1.0]))
    for j in range(97):
        b = orc.kv_off(P, maxp, 0, int(pt[j // P]), j % P, 0, 0, 0)
        pool[b:b + 256], pool[b + 256:b + 384], pool[b + 384:b + 512] = kb, one, mone
    q = Lcg(0x60A1).bf16(-1, 1, 2560)
    out = orc.bf16_to_f32(orc.attn_ref(q.reshape(1, 2560), 1, 96, 0, pool, pt, P, maxp)[0])
    assert np.all(out[:1024] == 1.0) and np.all(out[1024:] == -1.0)
    # pos 0: output equals V[0] exactly
    rng = np.random.default_rng(3)
    pool = randn_bf16(rng, maxp * P * 512, 1.0)
    out = orc.attn_ref(q.reshape(1, 2560), 1, 0, 0, pool, pt, P, maxp)[0]
    b = orc.kv_off(P, maxp, 0, 7, 0, 1, 0, 0)
    assert np.array_equal(out.reshape(16, 128), np.repeat(pool[b:b + 256].reshape(2, 128), 8, 0))


def test_attn_ref_causal_rows(orc):
    """Row t of a prefill only sees keys <= base+t: perturbing later keys
    leaves earlier rows unchanged, and each row equals the one-row decode."""
    q, pool, pt, P, maxp = _rand_case(orc, 4, 60)
    rng = np.random.default_rng(9)
    T, base = 10, 40
    qs = randn_bf16(rng, T * 2560, 1.0).reshape(T, 2560)
    full = orc.attn_ref(qs, T, base, 0, pool, pt, P, maxp)
    for t in (0, 4, 9):
        one = orc.attn_ref(qs[t:t + 1], 1, base + t, 0, pool, pt, P, maxp)[0]
        assert np.array_equal(full[t], one)
    pool2 = pool.copy()
    j = base + 5
    b = orc.kv_off(P, maxp, 0, int(pt[j // P]), j % P, 0, 0, 0)
    pool2[b:b + 512] = orc.f32_to_bf16(np.full(512, 7.0, np.float32))
    full2 = orc.attn_ref(qs, T, base, 0, pool2, pt, P, maxp)
    assert np.array_equal(full2[:5], full[:5]) and not np.array_equal(full2[5:], full[5:])


@pytest.mark.parametrize("C,limit", [(64, 599), (64, 40), (128, 1000), (256, 2047)])
def test_chunked_decode_plus_merge_equals_exact(orc, C, limit):
    """decode_chunks (bf16-P chunk statement) + merge2 reproduce the exact
    attention within the reference's criterion; the single-chunk direct path
    equals bf16(acc/l)."""
    q, pool, pt, P, maxp = _rand_case(orc, C + limit, limit + 1)
    NC = -(-4096 // C)
    parts, direct = orc.decode_chunks(q, limit, 0, pool, pt, P, maxp, C, NC)
    ref = orc.attn_ref(q.reshape(1, 2560), 1, limit, 0, pool, pt, P, maxp)[0]
    nv = limit // C + 1
    if nv == 1:
        got = direct
    else:
        _, got = orc.merge2(parts, NC, nv)
    st = orc.compare_bf16(got, ref)
    assert st["rel_l2"] < 1e-2 and st["cos"] > 0.9999 and st["max_abs"] < 2e-2, st


def test_decode_chunk_partial_is_chunk_softmax(orc):
    """A level-1 partial is (m, l, acc) of the softmax restricted to its chunk:
    m = max score, l = sum exp(s - m), acc = sum bf16(exp(s - m)) v (the
    16-position batching only reorders rounding)."""
    q, pool, pt, P, maxp = _rand_case(orc, 11, 300)
    C, NC, limit = 64, 8, 299
    parts, _ = orc.decode_chunks(q, limit, 0, pool, pt, P, maxp, C, NC)
    qf = orc.bf16_to_f32(q[:2048]).reshape(16, 128).astype(np.float64)
    for h in (0, 9):
        for c in (0, 4):
            js = range(c * C, min(c * C + C, limit + 1))
            K = np.stack([orc_kv(pool, P, maxp, 0, pt, j, 0, h // 8) for j in js])
            V = np.stack([orc_kv(pool, P, maxp, 0, pt, j, 1, h // 8) for j in js])
            s = K @ qf[h] / math.sqrt(128)
            m = s.max()
            w = np.exp(s - m)
            p = parts[h, c].astype(np.float64)
            assert abs(p[0] - m) < 1e-5
            assert abs(p[1] - w.sum()) / w.sum() < 1e-5
            acc = w @ V
            assert np.linalg.norm(p[2:] - acc) / np.linalg.norm(acc) < 4e-3  # bf16 P


def test_decode_chunk_fp32p_is_exact_chunk_softmax(orc):
    """fp32-P partials are the chunk softmax statistics with P unrounded:
    acc = sum exp(s - m) v to fp32 summation accuracy (1e-5), far tighter than
    the bf16-P bound above; and they differ from the bf16-P partials (which
    round P), so the flag is live."""
    q, pool, pt, P, maxp = _rand_case(orc, 11, 300)
    C, NC, limit = 64, 8, 299
    parts, _ = orc.decode_chunks(q, limit, 0, pool, pt, P, maxp, C, NC, fp32_p=True)
    parts_b, _ = orc.decode_chunks(q, limit, 0, pool, pt, P, maxp, C, NC)
    qf = orc.bf16_to_f32(q[:2048]).reshape(16, 128).astype(np.float64)
    for h in (0, 9, 15):
        for c in (0, 4):
            js = range(c * C, min(c * C + C, limit + 1))
            K = np.stack([orc_kv(pool, P, maxp, 0, pt, j, 0, h // 8) for j in js])
            V = np.stack([orc_kv(pool, P, maxp, 0, pt, j, 1, h // 8) for j in js])
            s = K @ qf[h] / math.sqrt(128)
            m = s.max()
            w = np.exp(s - m)
            p = parts[h, c].astype(np.float64)
            assert abs(p[0] - m) < 1e-5
            assert abs(p[1] - w.sum()) / w.sum() < 1e-5
            acc = w @ V
            assert np.linalg.norm(p[2:] - acc) / np.linalg.norm(acc) < 1e-5
            pb = parts_b[h, c].astype(np.float64)
            assert np.linalg.norm(pb[2:] - acc) / np.linalg.norm(acc) > 1e-5


def test_merge2_vs_logsumexp(orc):
    """The two-level merge equals a direct numpy fold of all partials (order
    independent in exact arithmetic), with l == 0 partials ignored."""
    rng = np.random.default_rng(5)
    N, nv = 257, 200
    parts = rng.uniform(-2, 2, (16, N, 130)).astype(np.float32)
    parts[:, :, 0] = rng.uniform(-8, 8, (16, N))
    parts[:, :, 1] = rng.uniform(0.5, 4, (16, N))
    parts[:, 3::7, 1] = 0.0
    parts[:, nv:] = 1e30
    lvl2, out = orc.merge2(parts, N, nv)
    p = parts[:, :nv].astype(np.float64)
    live = p[:, :, 1] != 0
    M = np.where(live, p[:, :, 0], -np.inf).max(axis=1, keepdims=True)
    f = np.where(live, np.exp(p[:, :, 0] - M), 0.0)
    want = (f[..., None] * p[:, :, 2:]).sum(1) / (f * p[:, :, 1]).sum(1)[:, None]
    got = orc.bf16_to_f32(out).reshape(16, 128)
    assert np.all(np.abs(got - want) <= orc.bf16_ulp(want) * 0.5 + 1e-12)
    assert np.all(lvl2[:, nv:, 1] == 0) if nv < 32 else True


def test_cpu_baseline_decode_matches_exact(orc):
    q, pool, pt, P, maxp = _rand_case(orc, 21, 700)
    out = orc.decode_cpu_mt(q.reshape(1, 2560), [699], [pt], pool, 0, P, maxp, 4)[0]
    ref = orc.attn_ref(q.reshape(1, 2560), 1, 699, 0, pool, pt, P, maxp)[0]
    st = orc.compare_bf16(out, ref)
    assert st["rel_l2"] < 1e-2 and st["max_abs"] < 2e-2, st


@pytest.mark.parametrize("native", [False, True])
def test_fast_cpu_baseline_decode_matches_exact(orc, native):
    """The speed-oriented CPU baseline (cpu_baseline.c: blocked online softmax,
    K/V rows shared by the 8 query heads of a group, position segments merged
    at the end) is within the attention tolerance of the double oracle, for 3
    sessions with ragged limits, portable and -march=native builds."""
    rng = np.random.default_rng(31)
    P, maxp = 32, 3 * 40
    pool = randn_bf16(rng, maxp * P * 512, 0.5)
    perm = rng.permutation(maxp).astype(np.uint32)
    pts = [perm[s::3].copy() for s in range(3)]
    limits = [1200, 37, 0]
    q = randn_bf16(rng, 3 * 2560, 1.0).reshape(3, 2560)
    out = orc.cpb_decode(q, limits, pts, pool, 0, P, maxp, threads=5, native=native)
    for s in range(3):
        ref = orc.attn_ref(q[s].reshape(1, 2560), 1, limits[s], 0, pool, pts[s], P, maxp)[0]
        st = orc.compare_bf16(out[s], ref)
        assert st["rel_l2"] < 1e-2 and st["cos"] > 0.9999, (s, st)
        assert st["max_abs"] < 2e-2 and st["mean_abs"] < 2e-3, (s, st)


def test_fast_cpu_baseline_append_matches_reference(orc):
    """The CPU baseline's RoPE append is within the reference's rope tolerance
    (2 bf16 ulp + 1e-4, plus the fp32 angle's half-ulp error times the input
    magnitude, as for the GPU kernel) of the double-precision rope_ref
    statement on q and K, and copies V exactly."""
    rng = np.random.default_rng(32)
    T, base, P, theta = 300, 1000, 16, 1e4
    maxp = -(-(base + T) // P) + 1
    pt = rng.permutation(maxp).astype(np.uint32)
    qkv = randn_bf16(rng, T * 2560, 1.0).reshape(T, 2560)
    pool_a = np.zeros(maxp * P * 512, dtype=np.uint16)
    pool_r = pool_a.copy()
    qa, qr = qkv.copy(), qkv.copy()
    orc.cpb_rope_append(qa, T, base, 0, pt, P, maxp, theta, pool_a, threads=3)
    orc.rope_append(qr, T, base, 0, pt, P, maxp, theta, 0, pool_r)
    inv = orc.inv_freq(theta).astype(np.float64)
    d = np.arange(128)
    ang_err = 2.0 ** -23 * (base + np.arange(T, dtype=np.float64))[:, None] * inv[d % 64][None, :]
    src = orc.bf16_to_f32(qkv[:, :2304]).astype(np.float64).reshape(T, 18, 128)
    extra = (np.abs(src) + np.abs(src[:, :, d ^ 64])) * ang_err[:, None, :]
    a, r = orc.bf16_to_f32(qa[:, :2048]), orc.bf16_to_f32(qr[:, :2048])
    assert np.all(np.abs(a - r) <= 2 * orc.bf16_ulp(r) + 1e-4 + extra[:, :16].reshape(T, 2048))
    for t in range(T):
        pos = base + t
        off = orc.kv_off(P, maxp, 0, int(pt[pos // P]), pos % P, 0, 0, 0)
        ka, kr = orc.bf16_to_f32(pool_a[off:off + 256]), orc.bf16_to_f32(pool_r[off:off + 256])
        tol = 2 * orc.bf16_ulp(kr) + 1e-4 + extra[t, 16:].reshape(256)
        assert np.all(np.abs(ka - kr) <= tol), t
    for t in (0, 150, T - 1):
        pos = base + t
        off = orc.kv_off(P, maxp, 0, int(pt[pos // P]), pos % P, 0, 0, 0)
        assert np.array_equal(pool_a[off + 256:off + 512], qkv[t, 2304:2560])
