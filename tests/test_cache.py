"""The HBM expert cache's policy and accounting on the CPU (bookkeeping-only caches: no
device memory is touched). The engine's behaviour it must keep is in src/cache/k3_cache.c;
the recorded numbers come from the engine's own data (docs/data/expert-cache-capacity.txt)
and from textbook LRU on small sequences."""
import json
import os

import numpy as np
import pytest

import k3moe
import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
K3_EXPERT = 17547264                 # one real K3 expert run, src/cache/k3_cache.h:4-8
SLOT = (K3_EXPERT + 65535) // 65536 * 65536


def dry_cache(n_layers, n_experts, slots, topk=2, expert_bytes=100000):
    bank = k3moe.Bank(n_layers, n_experts, expert_bytes=expert_bytes)
    slot = (expert_bytes + 65535) // 65536 * 65536
    return k3moe.Cache(bank, topk=topk, budget_bytes=slots * slot, device=-1)


def test_replay_of_the_engine_trace_matches_its_capacity_table():
    """docs/data/expert-cache-capacity.txt:23-28: LRU hit rates of the 100,096-request K3
    routing trace (tests/fixtures/expert_trace.bin) at 8/64/128/192 GB of slots, served
    through the cache's own get()."""
    pairs = np.load(os.path.join(GOLDEN, "expert_trace.npz"))["pairs"]
    n = pairs.shape[0]
    for gb, pct in ((8, 36.24), (128, 49.19), (192, 90.00)):
        slots = int(gb * 1e9 // K3_EXPERT)
        bank = k3moe.Bank(93, 896, expert_bytes=K3_EXPERT)
        c = k3moe.Cache(bank, topk=16, budget_bytes=slots * SLOT, device=-1)
        assert c.stats().nslot == slots
        for layer, e in pairs:
            assert c.get(int(layer), int(e)) is not None
        st = c.stats()
        assert st.requests == n and st.hits + st.misses == n
        assert abs(100.0 * st.hits / n - pct) < 0.005, (gb, st.hits)
        # the oracle's textbook LRU agrees request for request
        keys = (pairs[:, 0].astype(np.int64) * 896 + pairs[:, 1]).astype(np.int32)
        assert st.hits == O.lru_hits(keys, 93 * 896, slots)
        assert st.evictions == st.misses - min(slots, st.misses)


def test_lru_small_sequences():
    seq = [0, 1, 2, 0, 1, 3, 0, 4, 1]
    for cap in (2, 3, 5):
        c = dry_cache(1, 5, cap, topk=1)
        for e in seq:
            c.get(0, e)
        assert c.stats().hits == O.lru_hits(np.array(seq, np.int32), 5, cap), cap


def test_capacity_must_exceed_topk():
    bank = k3moe.Bank(1, 16, expert_bytes=100000)
    with pytest.raises(RuntimeError):
        k3moe.Cache(bank, topk=4, budget_bytes=4 * 131072, device=-1)
    k3moe.Cache(bank, topk=4, budget_bytes=5 * 131072, device=-1)


def test_pinned_slots_are_never_evicted():
    c = dry_cache(1, 10, 3)
    for e in (0, 1, 2):
        c.get(0, e)
    assert c.pin(0, 0) == 1 and c.pin(0, 9) == 0        # 9 is not resident
    for e in (3, 4, 5, 6):
        c.get(0, e)
    assert c.resident(0, 0)
    assert c.stats().pinned == 1
    c.pin(0, 0, False)
    for e in (7, 8, 9):
        c.get(0, e)
    assert not c.resident(0, 0)


def test_batch_prefetch_is_counted_apart_from_hits():
    """k3_cache.c:403-429: a get() served by the batch prefetch counts as a hit, and the
    true hit rate subtracts those prefetch reads."""
    c = dry_cache(2, 8, 6)
    assert c.getmany(1, [3, 4, 3, 5]) == 3               # duplicates reserved once
    for e in (3, 4, 5, 6):
        assert c.get(1, e) is not None
    st = c.stats()
    assert (st.hits, st.misses, st.prefetch_reads) == (3, 1, 3)
    assert st.bytes_read == 4 * 100000
    assert c.getmany(1, [3, 4]) == 0                     # already resident
    c.reset_stats()
    st = c.stats()
    assert (st.hits, st.misses, st.prefetch_reads, st.bytes_read) == (0, 0, 0, 0)


def test_open_step_protects_what_it_handed_out():
    """A slot handed out in the open step is never the victim: with every slot in use by
    the step, a further miss fails instead of evicting an expert still being read."""
    c = dry_cache(1, 8, 3, topk=2)
    c.step_begin()
    for e in (0, 1, 2):
        assert c.get(0, e) is not None
    assert c.get(0, 3) is None                           # nothing evictable
    assert c.get(0, 1) is not None                       # hits still serve
    c.step_end()
    assert c.get(0, 3) is not None                       # step over: LRU again (evicts 0)
    assert not c.resident(0, 0) and c.resident(0, 1) and c.resident(0, 2)


def test_trace_and_histogram_dumps(tmp_path):
    c = dry_cache(3, 5, 4)
    reqs = [(0, 1), (2, 4), (0, 1), (1, 0), (2, 4), (2, 4)]
    for l, e in reqs:
        c.get(l, e)
    tp, hp = str(tmp_path / "trace.bin"), str(tmp_path / "hist.json")
    assert k3moe.lib().k3gc_dump_trace(c.ptr, tp.encode()) == 0
    assert k3moe.lib().k3gc_dump_hist(c.ptr, hp.encode()) == 0
    got = np.fromfile(tp, dtype=np.int32).reshape(-1, 2)
    assert got.tolist() == [list(r) for r in reqs]
    h = json.load(open(hp))
    assert h["n_layers"] == 3 and h["n_experts"] == 5
    assert h["counts"] == {"0,1": 2, "2,4": 3, "1,0": 1}


def test_device_src_vtable_is_exposed():
    c = dry_cache(1, 4, 3)
    src = k3moe.K3ExpertSrc.from_address(c.src_ptr)
    assert src.get and src.getmany and src.resident
