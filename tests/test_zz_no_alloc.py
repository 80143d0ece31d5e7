"""The allocation-free decode entry point (mc_kv_attention_decode_noalloc,
records in a library-owned device array) against mc_kv_attention_decode on
the same inputs: bit-identical outputs on two calls in a row, the second with
a smaller context (fewer records than the first left in the array), and the
size limit rejected before any launch."""
import numpy as np
import pytest

from _util import from_dev, randn_bf16, to_dev

pytestmark = pytest.mark.gpu


def _case(kvm, dev, rng, ctx, C, P=64, ph0=True):
    import torch
    maxp = -(-ctx // P) + 1
    pt = rng.permutation(maxp).astype(np.uint32)
    lay = kvm.KvLayout(maxp, P, 2)
    pool = randn_bf16(rng, lay.total_elems(), 0.4)
    q = randn_bf16(rng, 2560, 1.0)
    NC = -(-ctx // C)
    inv = None
    if ph0:
        inv = torch.empty(64, dtype=torch.float32, device=dev)
        kvm.launch_rope_inv_freq_init(inv, 5e6)
    return dict(lay=lay, pt=to_dev(pt, dev), pool=pool, q=to_dev(q, dev), NC=NC, C=C,
                pos=to_dev(np.array([ctx - 1], dtype=np.uint32), dev), inv=inv)


def _run(kvm, dev, c, noalloc):
    import torch
    d_pool = to_dev(c["pool"], dev)
    out = torch.zeros(2048, dtype=torch.int16, device=dev)
    if noalloc:
        kvm.launch_attention_decode_noalloc(c["q"], c["pos"], 1, c["pt"], d_pool, c["lay"],
                                            c["NC"], out, d_inv_freq=c["inv"], chunk_pos=c["C"])
    else:
        parts = torch.full((16 * c["NC"] * 130,), float("nan"), dtype=torch.float32,
                           device=dev)
        parts2 = torch.zeros(16 * 32 * 130, dtype=torch.float32, device=dev)
        kvm.launch_attention_decode(c["q"], c["pos"], 1, c["pt"], d_pool, c["lay"], parts,
                                    c["NC"], out, d_inv_freq=c["inv"], chunk_pos=c["C"],
                                    d_partials2=parts2)
    torch.cuda.synchronize()
    return from_dev(out), from_dev(d_pool)


@pytest.mark.parametrize("first,second", [((131072, 256), (5000, 64)),
                                          ((20000, 128), (700, 64)),
                                          ((9000, 48), (3000, 48))])
def test_noalloc_matches_decode_twice(kvm, dev, first, second):
    rng = np.random.default_rng(first[0] + second[0])
    for ctx, C in (first, second):
        c = _case(kvm, dev, rng, ctx, C)
        want, pool_w = _run(kvm, dev, c, False)
        got, pool_g = _run(kvm, dev, c, True)
        assert np.array_equal(got, want), (ctx, C)
        assert np.array_equal(pool_g, pool_w), (ctx, C)  # phase0 append identical


def test_noalloc_rejects_beyond_scratch(kvm, dev, pkg):
    """chunk_pos 48 with 300 chunks would need 300 records per head."""
    import torch
    rng = np.random.default_rng(1)
    c = _case(kvm, dev, rng, 48 * 300, 48, ph0=False)
    out = torch.zeros(2048, dtype=torch.int16, device=dev)
    with pytest.raises(pkg.McError) as e:
        kvm.launch_attention_decode_noalloc(c["q"], c["pos"], 1, c["pt"], to_dev(c["pool"], dev),
                                            c["lay"], c["NC"], out, chunk_pos=48)
    assert e.value.status == 1 and "scratch" in str(e.value)
