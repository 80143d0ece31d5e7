"""CPU tests of the host allocators against the allocator model
(oracle.PagedKvAllocatorModel restates native/runtime/kv_cache.cpp:8-91) and
closed forms: a fresh session's table is [0, ceil(n/P)), growth is monotone,
OOM when the request exceeds capacity, release frees pages for reuse."""
import numpy as np
import pytest


def test_pool_single_session_is_identity(kvm):
    p = kvm.SharedPagePool(100, 32, 1)
    for n in (1, 31, 32, 33, 700, 3200):
        p.ensure(0, n)
        assert p.table(0) == list(range(-(-n // 32)))
    with pytest.raises(kvm.McError) as e:
        p.ensure(0, 3201)
    assert e.value.status == 5  # MC_E_OUT_OF_MEMORY
    p.release(0)
    assert p.pages_free() == 100 and p.table(0) == []


def test_pool_interleaved_growth_matches_model(kvm, orc):
    rng = np.random.default_rng(0)
    P, maxp, S = 64, 300, 8
    p = kvm.SharedPagePool(maxp, P, S)
    m = orc.SharedPoolModel(maxp, P, S)
    lens = [0] * S
    for step in range(400):
        s = int(rng.integers(S))
        lens[s] += int(rng.integers(1, 90))
        want = m.ensure(s, lens[s])
        if want == "OOM":
            with pytest.raises(kvm.McError):
                p.ensure(s, lens[s])
            m.release(s)
            p.release(s)
            lens[s] = 0
            continue
        p.ensure(s, lens[s])
        for t in range(S):
            assert p.table(t) == m.tables[t]
    assert p.pages_free() == m.used.count(False)


def test_churn_c5_reuses_pages(kvm, orc):
    """Config C5 host side: 8 sessions, lengths log-uniform in [16, 131072],
    64 decode steps with seeded finish/admit events; freed pages are reused
    and tables never share a page."""
    rng = np.random.default_rng(5)
    P, S = 64, 8
    maxp = 8 * 2048
    p = kvm.SharedPagePool(maxp, P, S)
    m = orc.SharedPoolModel(maxp, P, S)
    lens = [int(round(np.exp(rng.uniform(np.log(16), np.log(131072))))) for _ in range(S)]
    for s in range(S):
        assert m.ensure(s, lens[s]) == "OK"
        p.ensure(s, lens[s])
    reused = 0
    for step in range(64):
        for s in range(S):
            lens[s] += 1
            m.ensure(s, lens[s])
            p.ensure(s, lens[s])
        if rng.random() < 0.3:  # a session finishes, a new one is admitted
            s = int(rng.integers(S))
            freed = set(m.tables[s])
            m.release(s)
            p.release(s)
            lens[s] = int(round(np.exp(rng.uniform(np.log(16), np.log(131072)))))
            m.ensure(s, lens[s])
            p.ensure(s, lens[s])
            reused += len(freed & set(m.tables[s]))
        tabs = [p.table(s) for s in range(S)]
        assert tabs == m.tables
        flat = [x for t in tabs for x in t]
        assert len(flat) == len(set(flat))
    assert reused > 0


def test_allocator_oom_before_any_copy(kvm):
    """ensure_pages_for beyond capacity fails with MC_E_OUT_OF_MEMORY before
    touching the device (so it runs on the CPU)."""
    import ctypes
    fake = ctypes.c_void_p(0x1000)  # never dereferenced on this path

    class T:
        def data_ptr(self):
            return fake.value
    a = kvm.PagedKvAllocator(T(), 4, 32)
    with pytest.raises(kvm.McError) as e:
        a.ensure_pages_for(129, stream=0)
    assert e.value.status == 5 and "exhausted" in str(e.value)  # OOM message
    assert a.pages_owned() == 0


def test_allocator_model_closed_form(orc):
    m = orc.PagedKvAllocatorModel(10, 32)
    assert m.ensure_pages_for(1) == "OK" and m.shadow == [0] and m.uploads == 1
    assert m.ensure_pages_for(32) == "OK" and m.uploads == 1  # no growth, no copy
    assert m.ensure_pages_for(33) == "OK" and m.shadow == [0, 1] and m.uploads == 2
    assert m.ensure_pages_for(321) == "OOM"
    m.release_all()
    assert m.ensure_pages_for(64) == "OK" and m.shadow == [0, 1]


def test_allocator_lazy_upload_matches_model(kvm, orc):
    """The product allocator's lazy H2D rule (kv_cache.cpp:47-83): the table
    prefix is re-uploaded only when pages were added, release_all resets the
    synced count. Host-only allocator (no device table): pages_synced and the
    shadow table are compared with the model after every grow / no-grow /
    reset step; the model counts one upload per increase of its synced
    prefix, so equal synced counts at every step mean equal uploads."""
    rng = np.random.default_rng(3)
    P, maxp = 32, 40
    a = kvm.PagedKvAllocator(None, maxp, P)
    m = orc.PagedKvAllocatorModel(maxp, P)
    total, uploads_seen, prev_synced = 0, 0, 0
    for step in range(300):
        r = rng.random()
        if r < 0.1:
            a.release_all()
            m.release_all()
            total, prev_synced = 0, 0
        else:
            total = total + int(rng.integers(0, 70)) if r < 0.8 else total  # no-grow steps too
            want = m.ensure_pages_for(total)
            if want == "OOM":
                with pytest.raises(kvm.McError) as e:
                    a.ensure_pages_for(total, stream=0)
                assert e.value.status == 5
                a.release_all()
                m.release_all()
                total, prev_synced = 0, 0
                continue
            a.ensure_pages_for(total, stream=0)
        assert a.pages_owned() == len(m.shadow)
        assert a.pages_synced() == m.synced
        assert a.host_table() == m.shadow
        if a.pages_synced() > prev_synced:
            uploads_seen += 1
        prev_synced = a.pages_synced()
    assert uploads_seen == m.uploads and uploads_seen > 10
