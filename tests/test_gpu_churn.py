"""Mixed-length churn on the GPU: 8 sessions with lengths
log-uniform in [16, 131072) share one pool; over 64 batched decode steps
sessions finish and new ones are admitted (their pages freed and reused), and
every step appends one token per session (phase0) and attends it with the
batched split-KV decode (ragged limits, one chunk tier for max_ctx 131072).

Checked against the CPU oracle: page tables == the shared-pool model
(lowest free page, bit-exact), K/V written by phase0 == kernel-exact RoPE
append, decode outputs vs the double attention reference (relL2 < 1e-2,
cos > 0.9999, max-abs < 2e-2, mean-abs < 2e-3), and the whole pool
bit-identical to the oracle's mirror at the end. Scenario after the
reference's allocator semantics (kv_cache.cpp:8-91) and batched decode
(attention_decode.cu:2120-2170)."""
import numpy as np
import pytest

from _util import from_dev, randn_bf16, to_dev

pytestmark = pytest.mark.gpu

B, P, L, LAYER, STEPS = 8, 64, 1, 0, 64
MAX_CTX = 131072
THETA = 5e6


def check_vs_ref(orc, got, ref, tag):
    st = orc.compare_bf16(got, ref)
    assert st["rel_l2"] < 1e-2 and st["cos"] > 0.9999, (tag, st)
    assert st["max_abs"] < 2e-2 and st["mean_abs"] < 2e-3, (tag, st)


def test_churn_batched_decode(kvm, orc, dev):
    import torch
    rng = np.random.default_rng(0xC5)
    draw_len = lambda: int(min(MAX_CTX - STEPS - 1,
                               round(np.exp(rng.uniform(np.log(16), np.log(MAX_CTX))))))
    maxp = B * (MAX_CTX // P + 2)
    lay = kvm.KvLayout(maxp, P, L)
    C = kvm.attention_decode_chunk_pos(MAX_CTX)
    NC = kvm.attention_decode_max_chunks(MAX_CTX, C)
    assert (C, NC) == (256, 512)
    pool_d = torch.empty(lay.total_elems(), dtype=torch.bfloat16, device=dev)
    pool_d.normal_(0.0, 0.5)
    pool_d = pool_d.view(torch.int16)
    mirror = from_dev(pool_d)  # oracle copy of the pool
    page_elems = P * 512
    pages2d = pool_d.view(maxp, page_elems)

    alloc = kvm.SharedPagePool(maxp, P, B)
    model = orc.SharedPoolModel(maxp, P, B)
    d_tabs = [torch.zeros(maxp, dtype=torch.int32, device=dev) for _ in range(B)]
    lens = [0] * B

    def admit(s):
        n = draw_len()
        alloc.ensure(s, n, d_tabs[s])
        assert model.ensure(s, n) == "OK"
        pages = alloc.table(s)
        assert pages == model.tables[s]
        # "prefill": fresh K/V in the new session's pages (reused pages too)
        idx = torch.tensor(pages, dtype=torch.int64, device=dev)
        fresh = torch.empty(len(pages), page_elems, dtype=torch.bfloat16, device=dev)
        fresh.normal_(0.0, 0.5)
        pages2d[idx] = fresh.view(torch.int16)
        torch.cuda.synchronize()
        mirror.reshape(maxp, page_elems)[pages] = from_dev(fresh.view(torch.int16)).reshape(
            len(pages), page_elems)
        lens[s] = n

    for s in range(B):
        admit(s)
    inv = torch.empty(64, dtype=torch.float32, device=dev)
    kvm.launch_rope_inv_freq_init(inv, THETA)
    d_lims = [torch.zeros(1, dtype=torch.int32, device=dev) for _ in range(B)]
    tab = lambda ts: torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64, device=dev)
    t_lims, t_pts, t_kv = tab(d_lims), tab(d_tabs), tab([pool_d] * B)
    parts = torch.zeros(B * 16 * NC * 130, dtype=torch.float32, device=dev)
    parts2 = torch.zeros(B * (16 * 32 * 130), dtype=torch.float32, device=dev)
    out = torch.zeros(B * 2048, dtype=torch.int16, device=dev)
    freed, reused = set(), 0
    for step in range(STEPS):
        for s in range(B):
            if step > 0 and rng.random() < 0.1:  # finish -> admit a new session
                freed |= set(model.tables[s])
                alloc.release(s)
                model.release(s)
                admit(s)
                reused += len(freed & set(model.tables[s]))
        for s in range(B):
            alloc.ensure(s, lens[s] + 1, d_tabs[s])
            assert model.ensure(s, lens[s] + 1) == "OK"
            d_lims[s].fill_(lens[s])
        assert [alloc.table(s) for s in range(B)] == model.tables
        assert alloc.pages_free() == model.used.count(False)
        q = randn_bf16(rng, B * 2560, 1.0).reshape(B, 2560)
        kvm.launch_attention_decode_batch(to_dev(q.ravel(), dev), t_lims, B, LAYER, t_pts,
                                          t_kv, lay, parts, NC, out, d_inv_freq=inv,
                                          chunk_pos=C, d_partials2=parts2)
        torch.cuda.synchronize()
        got = from_dev(out).reshape(B, 2048)
        for s in range(B):
            pt = np.array(model.tables[s], dtype=np.uint32)
            qkv_o = q[s].reshape(1, 2560).copy()
            orc.rope_append(qkv_o, 1, lens[s], LAYER, pt, P, maxp, THETA, 1, mirror)
            if step % 4 == 0 or step == STEPS - 1:
                ref = orc.attn_ref(qkv_o, 1, lens[s], LAYER, mirror, pt, P, maxp)[0]
                check_vs_ref(orc, got[s], ref, f"step {step} slot {s} len {lens[s]}")
            lens[s] += 1
    assert np.array_equal(from_dev(pool_d), mirror), "pool != oracle mirror"
    assert reused > 0, "no freed page was handed out again"
    alloc.close()
