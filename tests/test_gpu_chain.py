"""GPU parity of k3gc_chain: the MoE half of consecutive decoder layers on a hidden state
that stays in HBM (hin = RMSNorm(h) x post_norm, h += MoE(hin); src/core/k3_ops.c:1015-1036
per layer, walked as src/cli/k3_run.c:582-618 does). Against the oracle composed layer
by layer: each layer's increment from the GPU's own h of the layer before (so a routing
near-tie cannot carry a difference from one layer into the next), routing bit-exact, and
the whole chain from x. The resident path (every expert in the cache, no host sync
between layers) gives the same bits as the fetching path when both run the same kernels.
Each test prints its case."""
import numpy as np
import pytest

import k3moe
import oracle as O
from test_gpu_parity import rel_l2, say

pytestmark = pytest.mark.gpu
REL = 1e-4


def _norm_weights(NL, d):
    return [k3moe.host_normal(d, 77, 900 + l, 1.0, 0.1) for l in range(NL)]


def _oracle_layer(layer, h, w_norm):
    """One layer of the chain on the CPU: h + MoE(RMSNorm(h) x w) per token."""
    k = O.oracle()
    out, idxs = [], []
    for t in range(h.shape[0]):
        hin = np.zeros(h.shape[1], np.float32)
        k.f_rms(O._p(hin), O._p(np.ascontiguousarray(h[t])), O._p(w_norm), h.shape[1], 1e-5)
        o, i, _ = O.k2_forward(layer, hin[None, :])
        out.append((h[t] + o[0]).astype(np.float32))
        idxs.append(i)
    return np.stack(out), np.stack(idxs)


@pytest.mark.parametrize("T", [2, 6])
def test_chain_of_three_layers(gpu, T):
    NL, d = 3, 256
    say(f"case: k3gc_chain, {NL} tiny layers with post-norm weights, T={T}, through a "
        f"7-slot cache (fetching path) and a 48-slot cache (resident path)")
    layers = [k3moe.SynthLayer(k3moe.TINY, seed=77, layer=l, layout="tiled") for l in range(NL)]
    bank = k3moe.Bank(NL, 16, d, 128, k3moe.K3G_EXPERT_MXFP4_TILED)
    for l, lay in enumerate(layers):
        bank.fill_from_layer(lay, l)
    slot = (bank.expert_bytes + 65535) // 65536 * 65536
    norms = _norm_weights(NL, d)
    dnorm = [k3moe.DevBuf.from_array(w) for w in norms]
    x = layers[0].tokens(T, stream_base=123)
    ctx = k3moe.Ctx(layers[0].dev_tiled, max_tokens=T)
    Ls = [lay.dev_tiled for lay in layers]

    def run(cache, n):
        dh = k3moe.DevBuf.from_array(x)
        cache.chain(ctx, Ls[:n], [b.ptr for b in dnorm[:n]], 0, dh.ptr, T)
        ctx.sync()
        return dh.download(np.float32, T * d).reshape(T, d)

    small = k3moe.Cache(bank, topk=4, budget_bytes=7 * slot)
    hs = [x] + [run(small, n) for n in range(1, NL + 1)]
    assert small.stats().evictions > 0
    for l in range(NL):
        ref, ridx = _oracle_layer(layers[l], hs[l], norms[l])
        r = rel_l2(hs[l + 1] - hs[l], ref - hs[l])
        say(f"  layer {l}: MoE increment rel-L2 {r:.3e}")
        assert r <= REL
    # the whole chain from x on the CPU
    h = x
    for l in range(NL):
        h, _ = _oracle_layer(layers[l], h, norms[l])
    r_all = rel_l2(hs[NL], h)
    say(f"  three layers from x: rel-L2 {r_all:.3e}")
    assert r_all <= 1e-3
    big = k3moe.Cache(bank, topk=4, budget_bytes=48 * slot)
    for l in range(NL):
        for e in range(16):
            assert big.prefetch(l, e) == 0
    big.reset_stats()
    h_res = run(big, NL)
    st = big.stats()
    say(f"  resident path: requests {st.requests}, hits {st.hits}")
    assert st.misses == 0 and st.requests > 0 and st.hits == st.requests
    # the fetching path runs a small cache's tokens in groups (here on the fused decode
    # kernel, up to 4 tokens), the resident path all T at once (the grouped GEMMs beyond
    # 4): the same bits when the kernels are the same, within both kernels' tolerance
    # otherwise
    r_res = rel_l2(h_res, hs[NL])
    say(f"  resident vs fetching path: rel-L2 {r_res:.3e}; resident vs the CPU chain "
        f"{rel_l2(h_res, h):.3e}")
    if T <= 4:
        assert np.array_equal(h_res.view(np.uint32), hs[NL].view(np.uint32))
    assert r_res <= 2 * REL and rel_l2(h_res, h) <= 1e-3
    ctx.destroy()
    small.free()
    big.free()
    bank.free()
