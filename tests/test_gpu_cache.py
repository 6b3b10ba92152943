"""The HBM expert cache on the GPU: experts copied from the pinned bank into HBM slots on
the cache's stream, evicted and re-copied, give the same layer output, bit for bit, as the
same kernels on all-resident experts; the drop-in k3_moe through the cache matches the
drop-in through a host-memory expert source."""
import ctypes as C

import numpy as np
import pytest

import k3moe
import oracle as O

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def _layers(n, layout):
    return [k3moe.SynthLayer(k3moe.TINY, seed=77, layer=l, layout=layout) for l in range(n)]


@pytest.mark.parametrize("max_pinned", [-1, 1])
def test_streamed_layers_match_resident(gpu, max_pinned):
    T, NL = 6, 3
    say(f"case: k3gc_moe tiny layer, {NL} layers x 2 passes, {T} tokens, 18 HBM slots for "
        f"{NL * 16} experts (evictions), router and given routing, pinned layers "
        f"{'all' if max_pinned < 0 else max_pinned} (the rest through the staging buffers)")
    layers = _layers(NL, "tiled")
    bank = k3moe.Bank(NL, 16, 256, 128, k3moe.K3G_EXPERT_MXFP4_TILED,
                      max_pinned_layers=max_pinned)
    if max_pinned >= 0:
        assert bank.pinned_layers == max_pinned
    for l, lay in enumerate(layers):
        bank.fill_from_layer(lay, l)
    slot = (bank.expert_bytes + 65535) // 65536 * 65536
    cache = k3moe.Cache(bank, topk=4, budget_bytes=18 * slot)
    ctx = k3moe.Ctx(layers[0].dev_tiled, max_tokens=T)
    d, k = 256, 4
    dout, didx, dwt = k3moe.DevBuf(T * d * 4), k3moe.DevBuf(T * k * 4), k3moe.DevBuf(T * k * 4)
    requests = 0
    for p in range(2):
        for l, lay in enumerate(layers):
            x = lay.tokens(T, stream_base=300 + 10 * p + l)
            dx = k3moe.DevBuf.from_array(x)
            # reference: the same grouped kernels on the layer's resident experts
            ctx.moe(lay.dev_tiled, dx.ptr, T, dout.ptr, didx.ptr, dwt.ptr)
            ctx.sync()
            ref = dout.download(np.float32, T * d)
            ridx = didx.download(np.int32, T * k)
            rwt = dwt.download(np.float32, T * k)
            dout.zero()
            L = lay.dev_tiled
            cache.moe(ctx, L, l, dx.ptr, T, dout.ptr, didx.ptr, dwt.ptr)
            ctx.sync()
            got = dout.download(np.float32, T * d)
            assert np.array_equal(didx.download(np.int32, T * k), ridx), (p, l)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (p, l)
            requests += len(np.unique(ridx))
            # the same routing handed in
            dout.zero()
            cache.moe(ctx, L, l, dx.ptr, T, dout.ptr, didx.ptr, dwt.ptr, ridx, rwt)
            ctx.sync()
            assert np.array_equal(dout.download(np.float32, T * d).view(np.uint32),
                                  ref.view(np.uint32)), (p, l)
            requests += len(np.unique(ridx))
    st = cache.stats()
    say(f"  requests {st.requests} hits {st.hits} misses {st.misses} prefetch {st.prefetch_reads} "
        f"evictions {st.evictions} copied {st.bytes_read / 1e6:.1f} MB")
    assert st.requests == requests
    assert st.hits + st.misses == st.requests
    assert st.evictions > 0 and st.prefetch_reads > 0
    assert st.bytes_read == (st.misses + st.prefetch_reads) * bank.expert_bytes
    if max_pinned >= 0:
        assert st.staged > 0
    # every call brings its experts in with the batch prefetch first: get() then hits
    assert st.misses == 0
    ctx.destroy()
    cache.free()


@pytest.mark.parametrize("prefill,T", [(False, 5), (True, 70)])
def test_dropin_through_the_hbm_cache(gpu, prefill, T):
    say(f"case: {'k3_moe_prefill' if prefill else 'k3_moe'} tiny layer T={T} with K3MoeW.src = "
        "the HBM cache (checkpoint-layout bank, 17 slots)")
    layer = k3moe.SynthLayer(k3moe.TINY, seed=99, layout="engine")
    x = layer.tokens(T)
    experts = list(range(16))
    w, cfg, keep = O.k2_weights(layer, experts)
    f = k3moe.lib().k3_moe_prefill if prefill else k3moe.lib().k3_moe
    ref = np.zeros_like(x)
    idx = np.zeros(cfg.topk, np.int32)
    wt = np.zeros(cfg.topk, np.float32)
    f(ref.ctypes.data, x.ctypes.data, C.byref(w), C.byref(cfg), T, idx.ctypes.data,
      wt.ctypes.data, None)
    bank = k3moe.Bank(1, 16, 256, 128, k3moe.K3G_EXPERT_MXFP4)
    bank.fill_from_layer(layer, 0)
    slot = (bank.expert_bytes + 65535) // 65536 * 65536
    # a cache that holds the call's whole union runs it as one group, as the host source
    # does, so the two give the same bits
    cache = k3moe.Cache(bank, topk=4, budget_bytes=17 * slot)
    w.src = cache.src_ptr
    w.layer = 0
    out = np.zeros_like(x)
    drops0 = C.c_long.in_dll(k3moe.lib(), "k3_expert_drops").value
    f(out.ctypes.data, x.ctypes.data, C.byref(w), C.byref(cfg), T, idx.ctypes.data,
      wt.ctypes.data, None)
    assert C.c_long.in_dll(k3moe.lib(), "k3_expert_drops").value == drops0
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    st = cache.stats()
    say(f"  requests {st.requests} hits {st.hits} misses {st.misses} prefetch {st.prefetch_reads}")
    assert st.requests > 0 and st.hits + st.misses == st.requests
    cache.free()
