"""GPU parity of the RoPE-fused K/V append (rope_kv) against the CPU oracle.

Cases follow native/tests/kernel_ops.cpp:1534-1565 (T=1 at pos 75 with table
{2,0,3}; pos 0; T=70 at layer 1 with table {5,2,9}) and the C2 prefill chunk
(8448 tokens, 64-token pages, theta 1e4 and 5e6). Criteria:
  * K, q and V bit-exact against the kernel-exact oracle (orc mode 1);
  * q/k within 2 bf16 ulp + 1e-4 of the reference's double rope_ref (mode 0),
    V bit-exact (kernel_ops.cpp:1493-1512). The reference kernel, like this one,
    rounds the angle pos*inv_freq to fp32 (rope_kv.cu:68), which the double
    oracle does not; the reference only tests pos < 76, where that is below
    1e-4. For far positions the bound adds the angle rounding term
    (|x| + |x2|) * 2^-23 * pos * inv_freq[p] (half an fp32 ulp of the angle
    plus the rounding of inv_freq, with margin);
  * every pool element not written keeps its poison; k/v qkv columns unchanged.
"""
import numpy as np
import pytest

from _util import Lcg, from_dev, randn_bf16, to_dev

pytestmark = pytest.mark.gpu
POISON = 0xABCD


def run_case(kvm, orc, dev, qkv, T, base, layer, pt, P, maxp, L, theta, use_table):
    import torch
    pt = np.asarray(pt, dtype=np.uint32)
    pool = np.full(maxp * P * 512 * L, POISON, dtype=np.uint16)
    lay = kvm.KvLayout(maxp, P, L)
    d_qkv, d_pool, d_pt = to_dev(qkv.ravel(), dev), to_dev(pool, dev), to_dev(pt, dev)
    d_base = to_dev(np.array([base], dtype=np.uint32), dev)
    inv = None
    if use_table:
        inv = torch.empty(64, dtype=torch.float32, device=dev)
        kvm.launch_rope_inv_freq_init(inv, theta)
        assert np.array_equal(from_dev(inv, np.float32), orc.inv_freq(theta))
    kvm.launch_rope_kv(d_qkv, T, d_base, layer, d_pt, d_pool, lay, theta, d_inv_freq=inv)
    torch.cuda.synchronize()
    q_got, pool_got = from_dev(d_qkv).reshape(T, 2560), from_dev(d_pool)

    # kernel-exact oracle: bit-exact everywhere
    q1, p1 = qkv.reshape(T, 2560).copy(), pool.copy()
    written = np.zeros(pool.size, dtype=np.uint8)
    orc.rope_append(q1, T, base, layer, pt, P, maxp, theta, 1, p1, written)
    assert np.array_equal(q_got, q1), "q / k,v columns differ from kernel-exact oracle"
    assert np.array_equal(pool_got, p1), "pool differs from kernel-exact oracle"
    assert np.all(pool_got[written == 0] == POISON)
    assert int(written.sum()) == T * 512

    # reference double oracle: <= 2 ulp + 1e-4 on q and K, V exact
    q0, p0 = qkv.reshape(T, 2560).copy(), pool.copy()
    orc.rope_append(q0, T, base, layer, pt, P, maxp, theta, 0, p0)
    inv = orc.inv_freq(theta).astype(np.float64)
    pos = (base + np.arange(T, dtype=np.float64))[:, None]
    d = np.arange(128)
    ang_err = 2.0 ** -23 * pos * inv[d % 64][None, :]  # [T][128]
    src = orc.bf16_to_f32(qkv.reshape(T, 2560)[:, :2304]).astype(np.float64).reshape(T, 18, 128)
    mag = np.abs(src) + np.abs(src[:, :, d ^ 64])
    tol_extra = mag * ang_err[:, None, :]  # [T][18][128]
    a, r = orc.bf16_to_f32(q_got[:, :2048]), orc.bf16_to_f32(q0[:, :2048])
    tol = 2 * orc.bf16_ulp(r) + 1e-4 + tol_extra[:, :16].reshape(T, 2048)
    assert np.all(np.abs(a - r) <= tol)
    k_got = np.empty((T, 256), dtype=np.uint16)
    k_ref = np.empty((T, 256), dtype=np.uint16)
    for t in range(T):
        pp = base + t
        off = orc.kv_off(P, maxp, layer, int(pt[pp // P]), pp % P, 0, 0, 0)
        k_got[t], k_ref[t] = pool_got[off:off + 256], p0[off:off + 256]
    ka, kr = orc.bf16_to_f32(k_got), orc.bf16_to_f32(k_ref)
    ktol = 2 * orc.bf16_ulp(kr) + 1e-4 + tol_extra[:, 16:].reshape(T, 256)
    assert np.all(np.abs(ka - kr) <= ktol)
    idx = np.nonzero(written)[0]
    kv = (idx % 512) // 256
    assert np.array_equal(pool_got[idx[kv == 1]], p0[idx[kv == 1]])


@pytest.mark.parametrize("use_table", [True, False])
def test_rope_decode_pos75(kvm, orc, dev, use_table):
    qkv = Lcg(0x90DE).bf16(-2, 2, 2560)
    run_case(kvm, orc, dev, qkv, 1, 75, 0, [2, 0, 3], 32, 8, 1, 5e6, use_table)


def test_rope_pos0_identity(kvm, orc, dev):
    qkv = Lcg(0x00B1).bf16(-2, 2, 2560)
    run_case(kvm, orc, dev, qkv, 1, 0, 0, [2], 32, 8, 1, 5e6, True)


def test_rope_prefill_T70_layer1(kvm, orc, dev):
    qkv = Lcg(0xFEED).bf16(-2, 2, 70 * 2560)
    run_case(kvm, orc, dev, qkv, 70, 0, 1, [5, 2, 9], 32, 16, 2, 5e6, True)


@pytest.mark.parametrize("theta", [1e4, 5e6])
def test_rope_prefill_chunk_8448_p64(kvm, orc, dev, theta):
    """Config C2: one 8448-token chunk, 64-token pages of a seeded table,
    written into layer 27 of a 28-layer pool."""
    rng = np.random.default_rng(2)
    T, P, L = 8448, 64, 28
    npages = T // P
    maxp = npages + 4
    pt = rng.permutation(maxp)[:npages]
    qkv = randn_bf16(rng, T * 2560, 1.0)
    # only layer 27 matters: keep the pool small by using L=28 with few pages
    run_case(kvm, orc, dev, qkv, T, 0, 27, pt, P, maxp, L, theta, True)


def test_rope_second_chunk_base(kvm, orc, dev):
    """A chunk after a prefix (base 8448, not page aligned when P=64 -> 132 pages)."""
    rng = np.random.default_rng(3)
    T, base, P = 300, 8448 + 5, 64
    maxp = (base + T) // P + 2
    pt = rng.permutation(maxp)
    qkv = randn_bf16(rng, T * 2560, 1.0)
    run_case(kvm, orc, dev, qkv, T, base, 0, pt, P, maxp, 1, 5e6, True)
