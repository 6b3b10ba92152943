"""Experts read from safetensors shards into the bank, then served by the HBM cache, on the
GPU: the engine's cache fixture under eviction pressure returns device pointers to bytes
equal to the checkpoint's runs (the check of the engine's tests/unit/test_cache.c:60-140,
serial and batched); and a synthetic checkpoint of the tiny layer loaded into a tiled bank
runs the layer through the drop-in k3_moe to the oracle's output for the same runs."""
import ctypes as C
import os

import numpy as np
import pytest

import k3moe
import oracle as O
from test_checkpoint import FIXTURE, _fixture_runs, write_checkpoint
from test_gpu_parity import rel_l2, say

pytestmark = pytest.mark.gpu


def _dev_bytes(ptr, n):
    out = np.empty(n, np.uint8)
    k3moe._check(k3moe.hip().hipMemcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), n,
                                       k3moe.D2H), "D2H")
    return out


def test_fixture_experts_through_the_hbm_cache(gpu):
    say("case: the engine's 24-expert cache fixture -> raw bank -> HBM cache of 8 slots "
        "(eviction pressure), get() and getmany() bytes vs the checkpoint runs")
    runs = _fixture_runs()
    bank = k3moe.Bank(1, 24, expert_bytes=1632, raw=True)
    bank.load(k3moe.St(FIXTURE), 0, 0, 1)
    slot = 65536
    cache = k3moe.Cache(bank, topk=4, budget_bytes=8 * slot)
    off = [0, 512, 544, 1056, 1088, 1600]          # w1p w1s w2p w2s w3p w3s in the run

    def same(e, q):
        k3moe.sync()
        got = [q.p1, q.s1, q.p2, q.s2, q.p3, q.s3]
        sizes = [512, 32, 512, 32, 512, 32]
        return all(np.array_equal(_dev_bytes(p, n), runs[e][o:o + n])
                   for p, o, n in zip(got, off, sizes))

    bad = 0
    for _ in range(3):
        for e in range(24):
            q = cache.get(0, e)
            bad += q is None or not same(e, q)
    assert bad == 0
    for start in range(0, 24, 4):
        ids = list(range(start, start + 4))
        cache.getmany(0, ids)
        for e in ids:
            q = cache.get(0, e)
            assert q is not None and same(e, q), e
    st = cache.stats()
    say(f"  requests {st.requests}, evictions {st.evictions}")
    assert st.evictions > 0
    cache.free()
    bank.free()


def test_layer_from_a_checkpoint(gpu, tmp_path):
    say("case: tiny layer written as two safetensors shards -> tiled bank -> HBM cache -> "
        "drop-in k3_moe, T=3 and T=9, vs the oracle on the runs read back from the shards")
    layer = k3moe.SynthLayer(k3moe.TINY, seed=90, layer=1, device=False)
    other = k3moe.SynthLayer(k3moe.TINY, seed=90, layer=0, device=False)
    write_checkpoint(str(tmp_path), [other, layer], scramble=(1, 5))
    st = k3moe.St(str(tmp_path))
    bank = k3moe.Bank(1, 16, 256, 128, k3moe.K3G_EXPERT_MXFP4_TILED)
    bank.load(st, 1, 0, 1)
    slot = (bank.expert_bytes + 65535) // 65536 * 65536
    cache = k3moe.Cache(bank, topk=4, budget_bytes=10 * slot)
    w = k3moe.K3MoeW()
    w.gate, w.bias = layer.gate.ctypes.data, layer.bias.ctypes.data
    w.sh1, w.sh3, w.sh2 = layer.sh1.ctypes.data, layer.sh3.ctypes.data, layer.sh2.ctypes.data
    w.wdt, w.src, w.layer = k3moe.K3_WBF16, cache.src_ptr, 0
    cfg = layer.cfg()
    runs = {(0, e): st.read_run(st.expert(1, e)) for e in range(16)}
    for T in (3, 9):
        x = layer.tokens(T, stream_base=40 + T)
        out = np.zeros_like(x)
        idx = np.zeros(4, np.int32)
        wt = np.zeros(4, np.float32)
        k3moe.lib().k3_moe(out.ctypes.data, x.ctypes.data, C.byref(w), C.byref(cfg), T,
                           idx.ctypes.data, wt.ctypes.data, None)
        src = O.MemSrc(runs, 1, 16, layer.geo)
        wo = k3moe.K3MoeW()
        C.memmove(C.byref(wo), C.byref(w), C.sizeof(w))
        wo.src = src.ptr
        oo, oi, ow = O.oracle().moe(wo, cfg, x)
        r = rel_l2(out, oo)
        say(f"  T={T}: rel-L2 {r:.3e}")
        assert np.array_equal(idx, oi)
        assert r <= 1e-4
    cache.free()
    bank.free()
