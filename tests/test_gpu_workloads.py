"""GPU parity at the workloads' own shapes that the other tests reach only in part:

* the streamed decode (16 stacked K2 layers behind a capped HBM cache) at K2 shape: 3 K2
  layers in a pinned host bank of which one layer is pinned and the rest pageable (copied
  through the staging buffers), batch 8, the routing of the benchmark's expert trace, a
  cache smaller than the working set (evictions): sampled rows against the oracle's
  composition for that routing, and the whole output bit-identical to the same layers
  run with every expert resident;
* the 4096-token Zipf(0.8) prefill on the FP4 x FP8 matrix cores: sampled rows against the
  quantisation-aware oracle (bar 5e-3), with the unquantised engine's rel-L2 reported.

Each test prints its case before touching the GPU."""
import numpy as np
import pytest

import bench
import k3moe
import oracle as O
from test_gpu_parity import _pair_rows, oracle_tokens, rel_l2, run_layer, say

pytestmark = pytest.mark.gpu
GEMM_REL = 1e-4


def _routed_plus_shared(layer, x, idx, wt, tokens):
    """The oracle's layer output of the given tokens for a given routing: the per-pair
    rows combined in slot order (float multiply, then add), then + the shared expert."""
    k, s = O.oracle(), layer.shape
    cap = k3moe.SWIGLU_CAP
    pairs = [(t, j) for t in tokens for j in range(s.topk)]
    rows = _pair_rows(layer, x, idx, pairs).reshape(len(tokens), s.topk, s.hidden)
    out = []
    for n, t in enumerate(tokens):
        acc = np.zeros(s.hidden, np.float32)
        for j in range(s.topk):
            acc = (acc + np.float32(wt[t, j]) * rows[n, j].astype(np.float32)).astype(np.float32)
        gu = np.concatenate([k.matmul_bf16(x[t], layer.sh1, layer.SI),
                             k.matmul_bf16(x[t], layer.sh3, layer.SI)])
        sh = k.matmul_bf16(k.situ(gu.astype(np.float32), cap, cap), layer.sh2, s.hidden)
        out.append((acc + sh.astype(np.float32)).astype(np.float32))
    return np.stack(out)


def test_streamed_k2_layers_against_the_oracle(gpu):
    NL, T, steps = 3, 8, 3
    D, E, K = 7168, 384, 8
    say(f"case: k3gc_moe, {NL} K2 layers in a host bank with 1 layer pinned (the rest through "
        f"the staging buffers), batch {T}, {steps} steps of the benchmark's expert trace, "
        f"64-slot HBM cache (evictions) vs the oracle and vs every expert resident")
    bank = k3moe.Bank(NL, E, D, 2048, k3moe.K3G_EXPERT_MXFP4_TILED, max_pinned_layers=1)
    assert bank.pinned_layers == 1
    layers = []
    for l in range(NL):
        lay = k3moe.SynthLayer(k3moe.K2, seed=2024, layer=l, layout="tiled")
        bank.fill_from_layer(lay, l)
        lay.release_experts()
        layers.append(lay)
    idx, wt = bench.expert_trace(steps, NL, T, seed=2035)
    xs = {(s, l): layers[l].tokens(T, stream_base=1000 + 10 * s + l)
          for s in range(steps) for l in range(NL)}
    slot = (bank.expert_bytes + 65535) // 65536 * 65536

    def run(budget_slots):
        cache = k3moe.Cache(bank, topk=K, budget_bytes=budget_slots * slot)
        ctx = k3moe.Ctx(layers[0].dev_tiled, max_tokens=T)
        dout, didx, dwt = k3moe.DevBuf(T * D * 4), k3moe.DevBuf(T * K * 4), k3moe.DevBuf(T * K * 4)
        outs = {}
        for s in range(steps):
            for l in range(NL):
                dx = k3moe.DevBuf.from_array(xs[s, l])
                cache.moe(ctx, layers[l].dev_tiled, l, dx.ptr, T, dout.ptr, didx.ptr, dwt.ptr,
                          idx[s, l], wt[s, l])
                ctx.sync()
                outs[s, l] = dout.download(np.float32, T * D).reshape(T, D)
                assert np.array_equal(didx.download(np.int32, T * K).reshape(T, K), idx[s, l])
        st = cache.stats()
        ctx.destroy()
        cache.free()
        return outs, st

    small, st = run(64)
    say(f"  64 slots: requests {st.requests}, misses+prefetch {st.misses + st.prefetch_reads}, "
        f"evictions {st.evictions}, staged {st.staged}")
    assert st.evictions > 0 and st.staged > 0
    full, st_full = run(NL * E)
    assert st_full.evictions == 0
    for key in small:
        assert np.array_equal(small[key].view(np.uint32), full[key].view(np.uint32)), key
    for (s, l, tokens) in ((0, 0, [0, 7]), (1, 2, [3]), (2, 1, [5]), (2, 2, [1])):
        ref = _routed_plus_shared(layers[l], xs[s, l], idx[s, l], wt[s, l], tokens)
        r = rel_l2(small[s, l][tokens], ref)
        say(f"  step {s} layer {l} tokens {tokens}: rel-L2 {r:.3e}")
        assert r <= GEMM_REL
    bank.free()


def test_k2_prefill_fp4xfp8_full_size(gpu):
    T = 4096
    say(f"case: k3g_moe K2_PREFILL ({T} tokens, Zipf(0.8)), routed experts on the FP4 x FP8 "
        f"matrix cores, sampled rows vs the quantisation-aware oracle")
    layer = k3moe.SynthLayer(k3moe.K2_PREFILL, seed=2024, layout="tiled")
    x = layer.tokens(T, stream_base=900)
    ctx = k3moe.Ctx(layer.dev_tiled, max_tokens=T)
    ctx.set_fp8(True)
    out, idx, _ = run_layer(layer, x, ctx=ctx, tiled=True)
    ctx.destroy()
    counts = np.bincount(idx.reshape(-1), minlength=layer.shape.n_experts)
    hot = int(np.argmax(counts))
    t_hot = int(np.nonzero((idx == hot).any(axis=1))[0][0])
    rng = np.random.default_rng(11)
    st = np.unique(np.concatenate([[0, T - 1, t_hot], rng.choice(T, size=5, replace=False)]))
    q = O.k2_forward_mxfp8(layer, x[st])
    ro, ri, _ = oracle_tokens(layer, x[st])
    assert np.array_equal(idx[st], ri)
    r_q, r_u = rel_l2(out[st], q), rel_l2(out[st], ro)
    say(f"  {len(st)} sampled rows: rel-L2 vs the quantisation-aware oracle {r_q:.3e}, vs the "
        f"unquantised engine {r_u:.3e}")
    assert r_q <= 5e-3
    assert r_u <= 0.1
