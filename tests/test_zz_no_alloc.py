"""k3g_moe_noalloc (the decode layer with every buffer in a fixed device array, for callers
that cannot allocate) against k3g_moe on a context (the existing entry point, same fused
kernel): outputs, routing indices and weights bit-identical, on two calls in a row, the
second with fewer tokens, on the tiny layer and on the Kimi-K2 layer, and a shape that
exceeds the array rejected with -1. Called through the C ABI."""
import ctypes as C

import numpy as np
import pytest

import k3moe
import oracle as O

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def _noalloc(L, x):
    T, d, k = x.shape[0], L.hidden, L.topk
    dx = k3moe.DevBuf.from_array(x)
    dout, didx, dwt = k3moe.DevBuf(T * d * 4), k3moe.DevBuf(T * k * 4), k3moe.DevBuf(T * k * 4)
    derr = k3moe.DevBuf(4)
    derr.zero()
    rc = k3moe.lib().k3g_moe_noalloc(C.byref(L), C.c_void_p(dx.ptr), T, C.c_void_p(dout.ptr),
                                     C.c_void_p(didx.ptr), C.c_void_p(dwt.ptr),
                                     C.c_void_p(derr.ptr), None)
    assert rc == 0
    k3moe.sync()
    assert derr.download(np.int32, 1)[0] == 0
    return (dout.download(np.float32, T * d).reshape(T, d),
            didx.download(np.int32, T * k).reshape(T, k),
            dwt.download(np.float32, T * k).reshape(T, k))


def _ctx(L, x):
    T, d, k = x.shape[0], L.hidden, L.topk
    ctx = k3moe.Ctx(L, max_tokens=4)
    dx = k3moe.DevBuf.from_array(x)
    dout, didx, dwt = k3moe.DevBuf(T * d * 4), k3moe.DevBuf(T * k * 4), k3moe.DevBuf(T * k * 4)
    ctx.moe(L, dx.ptr, T, dout.ptr, didx.ptr, dwt.ptr)
    ctx.sync()
    res = (dout.download(np.float32, T * d).reshape(T, d),
           didx.download(np.int32, T * k).reshape(T, k),
           dwt.download(np.float32, T * k).reshape(T, k))
    ctx.destroy()
    return res


@pytest.mark.parametrize("shape", ["tiny", "k2"])
def test_noalloc_matches_the_context_entry_point(gpu, shape):
    sh = k3moe.TINY if shape == "tiny" else k3moe.K2
    say(f"case: k3g_moe_noalloc vs k3g_moe, {sh.name}, T=4 then T=2")
    layer = k3moe.SynthLayer(sh, seed=31, layout="tiled")
    L = layer.dev_tiled
    x4 = layer.tokens(4)
    x2 = layer.tokens(2, stream_base=7)
    for x in (x4, x2):
        got = _noalloc(L, x)
        ref = _ctx(L, x)
        for g, r in zip(got, ref):
            assert np.array_equal(g.view(np.uint32), r.view(np.uint32))
    # and against the oracle on the smaller call (routing bit-exact)
    for t in range(2):
        _, ridx, _ = O.k2_forward(layer, x2[t:t + 1])
        assert np.array_equal(got[1][t], ridx)


def test_noalloc_rejects_what_does_not_fit(gpu):
    say("case: k3g_moe_noalloc rejects T=5 and a top-64 K2 layer (beyond the array)")
    layer = k3moe.SynthLayer(k3moe.TINY, seed=32, layout="tiled")
    L = layer.dev_tiled
    x = k3moe.DevBuf(5 * L.hidden * 4)
    out = k3moe.DevBuf(5 * L.hidden * 4)
    lib = k3moe.lib()
    assert lib.k3g_moe_noalloc(C.byref(L), C.c_void_p(x.ptr), 5, C.c_void_p(out.ptr), None,
                               None, None, None) == -1
    big = k3moe.K3gLayer.from_buffer_copy(L)
    big.hidden, big.latent, big.n_experts, big.topk, big.inter = 7168, 7168, 384, 64, 2048
    big.shared_inter = 2048
    assert lib.k3g_moe_noalloc(C.byref(big), C.c_void_p(x.ptr), 4, C.c_void_p(out.ptr), None,
                               None, None, None) == -1
