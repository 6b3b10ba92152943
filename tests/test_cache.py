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


def test_no_prefetch_switch(monkeypatch):
    """src/cache/k3_cache.c:268-274: K3_NOPREFETCH set at init leaves the source without
    its batch path (getmany NULL), so one binary times the layer both ways; get() still
    serves every request."""
    monkeypatch.setenv("K3_NOPREFETCH", "1")
    c = dry_cache(1, 6, 4)
    src = k3moe.K3ExpertSrc.from_address(c.src_ptr)
    assert src.get and src.resident and not src.getmany
    for e in (0, 1, 0, 2):
        assert c.get(0, e) is not None
    st = c.stats()
    assert (st.hits, st.misses, st.prefetch_reads) == (1, 3, 0)
    monkeypatch.delenv("K3_NOPREFETCH")
    c2 = dry_cache(1, 6, 4)
    assert k3moe.K3ExpertSrc.from_address(c2.src_ptr).getmany


# ------------------------------------------------------------ policy beyond LRU ----
# docs/data/expert-cache-capacity.txt:20-28 (the engine's tools/sim_cache.py on its
# recorded trace): capacity in GB, slots of one K3 expert, LRU / BELADY / PIN+LRU hit rates
CAPACITY_TABLE = [
    (8, 455, 36.24, 39.42, 37.82), (16, 911, 36.24, 42.61, 39.42),
    (32, 1823, 36.24, 48.99, 42.57), (64, 3647, 36.24, 61.74, 48.66),
    (128, 7294, 49.19, 84.59, 62.86), (192, 10941, 90.00, 90.00, 90.00),
    (256, 14589, 90.00, 90.00, 90.00), (384, 21883, 90.00, 90.00, 90.00),
    (512, 29178, 90.00, 90.00, 90.00), (768, 43767, 90.00, 90.00, 90.00),
    (1024, 58356, 90.00, 90.00, 90.00), (1450, 82633, 90.00, 90.00, 90.00)]


def test_policy_replays_reproduce_the_engine_table():
    """k3gc_replay_lru / _belady / _pinned_lru (npin = capacity // 2, sim_cache.py:163) on
    the engine's 100,096-request trace give every entry of its published table."""
    pairs = np.load(os.path.join(GOLDEN, "expert_trace.npz"))["pairs"]
    n = pairs.shape[0]
    for gb, slots, p_lru, p_bel, p_pin in CAPACITY_TABLE:
        cap = int(gb * 1e9 // K3_EXPERT)
        assert cap == slots
        got = (k3moe.replay("lru", pairs, cap), k3moe.replay("belady", pairs, cap),
               k3moe.replay("pinned_lru", pairs, cap, cap // 2))
        pct = tuple(round(100.0 * h / n, 2) for h in got)
        assert pct == (p_lru, p_bel, p_pin), (gb, got, pct)


def _small_traces():
    rng = np.random.default_rng(5)
    for n, nkeys, s in ((300, 12, 0.8), (2000, 60, 1.1), (1500, 200, 0.5)):
        p = np.arange(1, nkeys + 1, dtype=np.float64) ** -s
        k = rng.choice(nkeys, size=n, p=p / p.sum())
        yield np.stack([k % 3, k // 3], axis=1).astype(np.int32)


def test_policy_replays_agree_with_the_restatement():
    for pairs in _small_traces():
        keys = [(int(a), int(b)) for a, b in pairs]
        for cap in (1, 2, 3, 7, 16, 40, 250):
            assert k3moe.replay("lru", pairs, cap) == O.sim_lru(keys, cap), cap
            assert k3moe.replay("belady", pairs, cap) == O.sim_belady(keys, cap), cap
            for npin in (0, 1, cap // 2, cap, cap + 5):
                assert k3moe.replay("pinned_lru", pairs, cap, npin) == \
                    O.sim_pinned_lru(keys, cap, npin), (cap, npin)


def _best_possible(keys, cap):
    """Brute force over every choice at every miss with a full cache (evict any resident
    key, or do not cache the request): the most hits any policy gets."""
    from functools import lru_cache

    @lru_cache(maxsize=None)
    def go(i, res):
        if i == len(keys):
            return 0
        k = keys[i]
        if k in res:
            return 1 + go(i + 1, res)
        if len(res) < cap:
            return go(i + 1, res | {k})
        best = go(i + 1, res)
        for v in res:
            best = max(best, go(i + 1, (res - {v}) | {k}))
        return best
    return go(0, frozenset())


def test_belady_is_optimal_on_tiny_traces():
    rng = np.random.default_rng(9)
    for _ in range(60):
        n, nk, cap = int(rng.integers(4, 11)), int(rng.integers(2, 6)), int(rng.integers(1, 4))
        k = rng.integers(0, nk, size=n)
        pairs = np.stack([np.zeros(n), k], axis=1).astype(np.int32)
        keys = tuple(int(v) for v in k)
        assert k3moe.replay("belady", pairs, cap) == _best_possible(keys, cap), (keys, cap)


def test_pin_hottest_from_a_previous_histogram():
    """The hot set of one workload pinned for the next: the pinned keys are the npin
    most requested of the histogram (ties to the lower key), they stay resident, and the
    next workload's hits equal the pinned-LRU replay with that hot set already resident."""
    pairs = np.load(os.path.join(GOLDEN, "expert_trace.npz"))["pairs"]
    half = pairs.shape[0] // 2
    slots = int(32e9 // K3_EXPERT)
    bank = k3moe.Bank(93, 896, expert_bytes=K3_EXPERT)
    first = k3moe.Cache(bank, topk=16, budget_bytes=slots * SLOT, device=-1)
    for layer, e in pairs[:half]:
        first.get(int(layer), int(e))
    hist = first.hist()
    assert hist.sum() == half
    npin = slots // 2
    c = k3moe.Cache(bank, topk=16, budget_bytes=slots * SLOT, device=-1)
    assert c.pin_hottest(hist, npin) == npin
    order = np.lexsort((np.arange(hist.size), -hist.astype(np.int64)))
    want = set(int(v) for v in order[:npin])
    got = {L * 896 + e for L in range(93) for e in range(896)
           if c.resident(L, e)}
    assert got == want and c.stats().pinned == npin
    c.reset_stats()
    for layer, e in pairs[half:]:
        c.get(int(layer), int(e))
    st = c.stats()
    keys = [int(L) * 896 + int(e) for L, e in pairs[half:]]
    assert st.hits == O.sim_pinned_lru(keys, slots, npin, hot=want, preloaded=True)
    assert all(c.resident(k // 896, k % 896) for k in want)
    lru_only = O.sim_lru(keys, slots)
    print(f"pinned {npin} of {slots} slots from the first half's histogram: second half "
          f"hits {st.hits} vs LRU {lru_only}")
