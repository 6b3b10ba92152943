"""The engine's expert cache entry points (k3_cache_init and the rest, with the engine's
K3Cache layout) on the GPU, fed the way the engine's main() feeds them: a K3St filled by the
engine's own k3_st_open (compiled into oracle/_ref from src/io/k3_st.c), then
k3_cache_init(&cache, &st, &cfg, budget), the counters read straight from the struct and
&cache.src handed to k3_moe (src/cli/k3_run.c:1144-1155, :582-590, :1524-1534).

  * the engine's 24-expert fixture (runs in their own layout) under eviction pressure:
    device bytes equal the engine's k3_expert_load of the same expert, ref[slot] equals
    its k3_expert_ref, and hits / misses / evictions / prefetch reads / bytes read equal a
    replay of the engine's policy (first empty slot, else least recently used, unpinned;
    getmany reserves, reads, publishes; src/cache/k3_cache.c:49-218), as do the trace and
    histogram files;
  * a tiny layer written as safetensors shards: the cache tiles its experts on the GPU,
    and the drop-in k3_moe on &cache.src matches the oracle on the runs read back, with a
    roomy cache and with top-k + 1 slots (no expert dropped)."""
import ctypes as C
import json
import os

import numpy as np
import pytest

import k3moe
import oracle as O
from test_checkpoint import FIXTURE, write_checkpoint
from test_gpu_parity import rel_l2, say

pytestmark = pytest.mark.gpu


def _dev_bytes(ptr, n):
    out = np.empty(n, np.uint8)
    k3moe._check(k3moe.hip().hipMemcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), n,
                                       k3moe.D2H), "D2H")
    return out


def _engine_io():
    io = O.engine_io()
    if io is None:
        pytest.skip("oracle/_ref was not built (the engine's k3_st.c is needed to fill a K3St)")
    return io


class PolicyModel:
    """The engine's replacement policy and counters, for checking the struct's fields."""

    def __init__(self, nslot, n_experts):
        self.key_of = [-1] * nslot
        self.used = [0] * nslot
        self.pinned = [False] * nslot
        self.slot_of = {}
        self.clock = 0
        self.ne = n_experts
        self.hits = self.misses = self.evictions = self.prefetch_reads = self.reads = 0

    def _victim(self):
        best, old = -1, None
        for i, k in enumerate(self.key_of):
            if k == -2:
                continue
            if k == -1:
                return i
            if self.pinned[i]:
                continue
            if old is None or self.used[i] < old:
                best, old = i, self.used[i]
        return best

    def _evict(self, s):
        if self.key_of[s] >= 0:
            del self.slot_of[self.key_of[s]]
            self.evictions += 1

    def get(self, layer, e):
        key = layer * self.ne + e
        if key in self.slot_of:
            self.hits += 1
            self.clock += 1
            self.used[self.slot_of[key]] = self.clock
            return
        self.misses += 1
        s = self._victim()
        self._evict(s)
        self.reads += 1
        self.key_of[s] = key
        self.slot_of[key] = s
        self.clock += 1
        self.used[s] = self.clock

    def getmany(self, layer, ids):
        res = []
        for e in ids:
            key = layer * self.ne + e
            if key in self.slot_of or any(r[1] == key for r in res):
                continue
            s = self._victim()
            self._evict(s)
            self.key_of[s] = -2
            self.clock += 1
            self.used[s] = self.clock
            res.append((s, key))
        for s, key in res:
            self.reads += 1
            self.key_of[s] = key
            self.slot_of[key] = s
            self.clock += 1
            self.used[s] = self.clock
            self.prefetch_reads += 1

    def pin(self, layer, e, on):
        key = layer * self.ne + e
        if key not in self.slot_of:
            return 0
        self.pinned[self.slot_of[key]] = bool(on)
        return 1


def _call_get(cache, layer, e):
    q = k3moe.K3ExpertQ()
    fn = k3moe.SRC_GET(cache.src.get)
    rc = fn(C.addressof(cache), layer, e, C.addressof(q))
    return q if rc == 0 else None


def _call_getmany(cache, layer, ids):
    a = np.ascontiguousarray(ids, np.int32)
    return k3moe.SRC_GETMANY(cache.src.getmany)(C.addressof(cache), layer, a.ctypes.data, a.size)


def test_engine_cache_on_the_fixture(gpu, tmp_path):
    say("case: the engine's 24-expert fixture through k3_cache_init on the engine's own K3St, "
        "8 HBM slots: bytes vs k3_expert_load, ref[] vs k3_expert_ref, counters vs the policy")
    io = _engine_io()
    L = k3moe.lib()
    st = k3moe.K3St()
    assert io.L.k3_st_open(C.byref(st), FIXTURE.encode()) == 0
    cfg = k3moe.K3Cfg()
    cfg.n_layers, cfg.n_experts, cfg.topk, cfg.first_dense = 1, 24, 4, 0
    cache = k3moe.K3Cache()
    # too small first: fewer than top-k + 1 slots is refused, as in the engine
    assert L.k3_cache_init(C.byref(cache), C.byref(st), C.byref(cfg), 4 * 65536) != 0
    assert L.k3_cache_init(C.byref(cache), C.byref(st), C.byref(cfg), 8 * 65536) == 0
    assert cache.nslot == 8 and cache.slot_bytes == 65536 and cache.n_experts == 24
    model = PolicyModel(cache.nslot, 24)
    want = {}
    for e in range(24):
        r = k3moe.K3ExpertRef()
        assert io.L.k3_expert_ref(C.byref(st), 0, e, C.byref(r)) == 0
        buf = np.zeros(r.nbytes, np.uint8)
        assert io.L.k3_expert_load(C.byref(st), C.byref(r), buf.ctypes.data) == r.nbytes
        want[e] = (r, buf)

    def check(e, q):
        r, buf = want[e]
        k3moe.sync()
        got = [(q.p1, r.m[0].p_off, r.m[0].p_bytes), (q.s1, r.m[0].s_off, r.m[0].s_bytes),
               (q.p2, r.m[1].p_off, r.m[1].p_bytes), (q.s2, r.m[1].s_off, r.m[1].s_bytes),
               (q.p3, r.m[2].p_off, r.m[2].p_bytes), (q.s3, r.m[2].s_off, r.m[2].s_bytes)]
        for ptr, off, n in got:
            assert np.array_equal(_dev_bytes(ptr, n), buf[off:off + n]), e
        slot = cache.slot_of[e]
        f = cache.ref[slot]
        assert (f.layer, f.expert, f.shard, f.off, f.nbytes, f.contiguous) == \
            (r.layer, r.expert, r.shard, r.off, r.nbytes, r.contiguous), e
        for i in range(3):
            a, b = f.m[i], r.m[i]
            assert (a.p_off, a.p_bytes, a.s_off, a.s_bytes, a.rows, a.pcols, a.scols) == \
                (b.p_off, b.p_bytes, b.s_off, b.s_bytes, b.rows, b.pcols, b.scols), (e, i)

    def counters():
        assert (cache.hits, cache.misses, cache.evictions, cache.prefetch_reads) == \
            (model.hits, model.misses, model.evictions, model.prefetch_reads)
        assert cache.bytes_read == model.reads * want[0][0].nbytes

    seq = []
    for rnd in range(3):
        for e in (list(range(24)) if rnd != 1 else [0, 1, 2, 0, 1, 2, 5, 5, 23, 0]):
            q = _call_get(cache, 0, e)
            model.get(0, e)
            seq.append(e)
            assert q is not None
            check(e, q)
            counters()
    for start in range(0, 24, 4):
        ids = [start, start + 1, start + 1, start + 2, start + 3]
        _call_getmany(cache, 0, ids)
        model.getmany(0, ids)
        counters()
        for e in ids[1:]:
            q = _call_get(cache, 0, e)
            model.get(0, e)
            seq.append(e)
            check(e, q)
            counters()
    # pinning keeps an expert resident through a sweep of the others
    assert L.k3_cache_pin(C.byref(cache), 0, 21, 1) == 1 and model.pin(0, 21, 1) == 1
    assert L.k3_cache_pin(C.byref(cache), 0, 2, 1) == model.pin(0, 2, 1)
    for e in range(24):
        if e != 21:
            _call_get(cache, 0, e)
            model.get(0, e)
            seq.append(e)
    assert cache.slot_of[21] >= 0
    counters()
    assert L.k3_cache_prefetch(C.byref(cache), 0, 7) == 0
    model.get(0, 7)
    counters()
    # the request trace (get() only, in order) and the histogram, in the engine's formats
    assert cache.ntrace == 2 * len(seq)                    # prefetch is not a request
    tr, hi = str(tmp_path / "trace.bin"), str(tmp_path / "hist.json")
    assert L.k3_cache_dump_trace(C.byref(cache), tr.encode()) == 0
    got = np.fromfile(tr, np.int32).reshape(-1, 2)
    assert np.array_equal(got[:, 1], np.array(seq)) and np.all(got[:, 0] == 0)
    assert L.k3_cache_dump_hist(C.byref(cache), hi.encode()) == 0
    h = json.load(open(hi))
    assert h["n_layers"] == 1 and h["n_experts"] == 24
    assert sum(h["counts"].values()) == len(seq)
    assert h["counts"]["0,5"] == seq.count(5)
    L.k3_cache_report(C.byref(cache), b"fixture")
    L.k3_cache_reset_stats(C.byref(cache))
    assert (cache.hits, cache.misses, cache.evictions, cache.bytes_read,
            cache.prefetch_reads) == (0, 0, 0, 0, 0)
    say(f"  requests {len(seq)}, evictions {model.evictions}, prefetch reads "
        f"{model.prefetch_reads}")
    L.k3_cache_free(C.byref(cache))
    assert cache.nslot == 0
    io.L.k3_st_close(C.byref(st))


@pytest.mark.parametrize("slots", [12, 5])
def test_engine_cache_runs_a_layer(gpu, tmp_path, slots):
    say(f"case: tiny layer as safetensors shards -> engine k3_st_open -> k3_cache_init "
        f"({slots} HBM slots, tiled on the GPU) -> drop-in k3_moe on &cache.src, T=3 and 9")
    io = _engine_io()
    L = k3moe.lib()
    layer = k3moe.SynthLayer(k3moe.TINY, seed=91, layer=1, device=False)
    other = k3moe.SynthLayer(k3moe.TINY, seed=91, layer=0, device=False)
    write_checkpoint(str(tmp_path), [other, layer], scramble=(1, 5))
    st = k3moe.K3St()
    assert io.L.k3_st_open(C.byref(st), str(tmp_path).encode()) == 0
    cfg = layer.cfg()
    cfg.n_layers, cfg.first_dense = 2, 0
    tiled = 2 * L.k3g_tiled_mxfp4_bytes(128, 256) + L.k3g_tiled_mxfp4_bytes(256, 128)
    slot = (tiled + 65535) // 65536 * 65536
    cache = k3moe.K3Cache()
    assert L.k3_cache_init(C.byref(cache), C.byref(st), C.byref(cfg), slots * slot) == 0
    assert cache.slot_bytes == slot and cache.nslot == slots
    w = k3moe.K3MoeW()
    w.gate, w.bias = layer.gate.ctypes.data, layer.bias.ctypes.data
    w.sh1, w.sh3, w.sh2 = layer.sh1.ctypes.data, layer.sh3.ctypes.data, layer.sh2.ctypes.data
    w.wdt, w.src, w.layer = k3moe.K3_WBF16, C.addressof(cache), 1
    ours = k3moe.St(str(tmp_path))
    runs = {(1, e): ours.read_run(ours.expert(1, e)) for e in range(16)}
    drops0 = C.c_long.in_dll(L, "k3_expert_drops").value
    for T in (3, 9):
        x = layer.tokens(T, stream_base=60 + T)
        out = np.zeros_like(x)
        idx = np.zeros(4, np.int32)
        wt = np.zeros(4, np.float32)
        L.k3_moe(out.ctypes.data, x.ctypes.data, C.byref(w), C.byref(cfg), T, idx.ctypes.data,
                 wt.ctypes.data, None)
        src = O.MemSrc(runs, 2, 16, layer.geo)
        wo = k3moe.K3MoeW()
        C.memmove(C.byref(wo), C.byref(w), C.sizeof(w))
        wo.src = src.ptr
        oo, oi, ow = O.oracle().moe(wo, cfg, x)
        r = rel_l2(out, oo)
        say(f"  T={T}: rel-L2 {r:.3e}, kernels {L.k3moe_last_kernels()}, hits {cache.hits} "
            f"misses {cache.misses} evictions {cache.evictions}")
        assert np.array_equal(idx, oi) and np.array_equal(wt.view(np.uint32), ow.view(np.uint32))
        assert r <= 1e-4
        assert L.k3moe_last_kernels() & 6          # the matrix-core kernels ran
    assert C.c_long.in_dll(L, "k3_expert_drops").value == drops0
    assert cache.misses > 0 and cache.hits + cache.misses == cache.ntrace // 2
    assert cache.bytes_read == (cache.misses + cache.prefetch_reads) * runs[(1, 0)].size
    if slots == 5:
        assert cache.evictions > 0
    L.k3_cache_free(C.byref(cache))
    io.L.k3_st_close(C.byref(st))
