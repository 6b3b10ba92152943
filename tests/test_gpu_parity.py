"""GPU parity: the HIP path against the CPU oracle on identical seeded inputs.

Bars: routing indices bit-exact (in order); MXFP4 dequantisation bit-exact; layer
outputs within rel-L2 1e-3 (fp32 accumulation). Each test prints the case it runs
before touching the GPU.
"""
import ctypes as C
import json
import os

import numpy as np
import pytest

import k3moe
import oracle as O

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
REL_L2 = 1e-3
# the grouped bf16 GEMMs: x and the weights exact in bf16, h as bf16 plus its MXFP8
# remainder (about 12 significant bits), fp32 accumulation: rel-L2 about 4e-5
GEMM_REL = 1e-4


def rel_l2(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - np.asarray(b, np.float64)) /
                 max(np.linalg.norm(np.asarray(b, np.float64)), 1e-30))


def say(msg):
    print(msg, flush=True)


def run_layer(layer, x, ctx=None, force=0, fused=True, tiled=None):
    """tiled (default: fused and T <= 4): the tiled copy of the layer, which runs the
    fused decode kernel up to 4 tokens and the grouped GEMMs beyond; otherwise the staged
    kernels on the checkpoint layout."""
    T, d, k = x.shape[0], layer.shape.hidden, layer.shape.topk
    if tiled is None:
        tiled = fused and T <= 4
    L = layer.dev_tiled if tiled else layer.dev
    own = ctx is None
    ctx = ctx or k3moe.Ctx(L, max_tokens=T)
    ctx.force_exact(force)
    ctx.set_fused(fused)
    dx = k3moe.DevBuf.from_array(x)
    dout, didx, dwt = k3moe.DevBuf(T * d * 4), k3moe.DevBuf(T * k * 4), k3moe.DevBuf(T * k * 4)
    ctx.moe(L, dx.ptr, T, dout.ptr, didx.ptr, dwt.ptr)
    ctx.sync()
    res = (dout.download(np.float32, T * d).reshape(T, d),
           didx.download(np.int32, T * k).reshape(T, k),
           dwt.download(np.float32, T * k).reshape(T, k))
    ctx.force_exact(0)
    if own:
        ctx.destroy()
    return res


def oracle_tokens(layer, x):
    outs, idxs, wts = [], [], []
    for t in range(x.shape[0]):
        o, i, w = O.k2_forward(layer, x[t:t + 1])
        outs.append(o[0]); idxs.append(i); wts.append(w)
    return np.stack(outs), np.stack(idxs), np.stack(wts)


# ------------------------------------------------------------------ synthetic data ----

def test_device_fill_matches_host(gpu):
    say("case: k3g_fill_bytes / k3g_fill_scales vs host fills, 3 streams, odd offsets")
    L = k3moe.lib()
    for stream, first, n in [(11, 0, 4096), (12, 5, 1000), (1_000_007, 123457, 77777)]:
        buf = k3moe.DevBuf(n)
        assert L.k3g_fill_bytes(C.c_void_p(buf.ptr), n, 99, stream, first, None) == 0
        k3moe.sync()
        assert np.array_equal(buf.download(np.uint8, n), k3moe.host_bytes(n, 99, stream, first))
        assert L.k3g_fill_scales(C.c_void_p(buf.ptr), n, 99, stream, first, -4, 2, None) == 0
        k3moe.sync()
        dev = buf.download(np.uint8, n)
        assert np.array_equal(dev, k3moe.host_scales(n, 99, stream, -4, 2, first))
        assert dev.min() >= 123 and dev.max() <= 129


# ------------------------------------------------------------------ MXFP4 kernels ----

def test_dequant_real_checkpoint_bytes(gpu):
    say("case: k3_mxfp4_dequant on tests/fixtures/mxfp4.json (64 x 3584), exact")
    m = np.load(os.path.join(GOLDEN, "mxfp4.npz"))
    rows, pc = int(m["rows"]), int(m["packed_cols"])
    packed = np.ascontiguousarray(m["packed"])
    scales = np.ascontiguousarray(m["scales"])
    expected = np.ascontiguousarray(m["expected"], np.float32).ravel()
    out = np.zeros(rows * pc * 2, np.float32)
    k3moe.lib().k3_mxfp4_dequant(out.ctypes.data, packed.ctypes.data, scales.ctypes.data,
                                 rows, pc, 32)
    assert np.array_equal(out.view(np.uint32), expected.view(np.uint32))
    assert not np.array_equal(out[:64], m["swapped_first64"])


def test_matmul_mxfp4_kat(gpu):
    say("case: k3_matmul_mxfp4 3072x3584 on the bench_kernels known-answer inputs")
    pk = O.kat_b(3072 * 1792, 777)
    sc = np.full(3072 * 112, 127, np.uint8)
    x = O.kat_f(3584, 4242)
    y = np.zeros(3072, np.float32)
    k3moe.lib().k3_matmul_mxfp4(y.ctypes.data, x.ctypes.data, pk.ctypes.data, sc.ctypes.data,
                                3584, 3072, 32)
    ref = O.oracle().matmul_mxfp4(x, pk, sc, 3072)
    assert O.fnv1a(ref) == "a231061237b5579d"
    assert rel_l2(y, ref) < 1e-6
    # fp32 accumulation: every row within 1e-5 of the output's RMS
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.sqrt(np.mean(ref.astype(np.float64) ** 2))


@pytest.mark.parametrize("rows,inn,lo,hi", [(129, 48, -4, 2), (70, 40, -20, 20), (33, 2048, -4, 2),
                                           (17, 7168, 100, 110)])
def test_matmul_mxfp4_shapes(gpu, rows, inn, lo, hi):
    say(f"case: k3_matmul_mxfp4 rows={rows} in={inn} scales 127+[{lo},{hi}] incl. byte 255")
    ng = (inn + 31) // 32
    pk = k3moe.host_bytes(rows * inn // 2, 5, 900 + inn)
    sc = k3moe.host_scales(rows * ng, 5, 901 + inn, lo, hi)
    sc[3] = 255
    x = k3moe.host_normal(inn, 5, 902 + inn)
    y = np.zeros(rows, np.float32)
    k3moe.lib().k3_matmul_mxfp4(y.ctypes.data, x.ctypes.data, pk.ctypes.data, sc.ctypes.data,
                                inn, rows, 32)
    ref = O.oracle().matmul_mxfp4(x, pk, sc, rows)
    assert rel_l2(y, ref) < 1e-6


@pytest.mark.parametrize("rows,inn,group", [(40, 512, 16), (33, 1000, 64), (21, 90, 10),
                                           (9, 64, 1), (12, 100, 9)])
def test_matmul_mxfp4_other_groups(gpu, rows, inn, group):
    """group != 32 (the engine's grouped path: ceil(in / group) scale bytes per row,
    group g read from byte g * (group / 2) on, which for the odd groups 1 and 9 is not the
    plain packing), against the oracle's restatement of it (bit-identical to the
    engine's compiled kernel in the CPU tests)."""
    say(f"case: k3_matmul_mxfp4 rows={rows} in={inn} group={group}")
    ng = (inn + group - 1) // group
    pk = k3moe.host_bytes(rows * inn // 2, 6, 950 + inn)
    sc = k3moe.host_scales(rows * ng, 6, 951 + inn, -4, 2)
    x = k3moe.host_normal(inn, 6, 952 + inn)
    y = np.zeros(rows, np.float32)
    k3moe.lib().k3_matmul_mxfp4(y.ctypes.data, x.ctypes.data, pk.ctypes.data, sc.ctypes.data,
                                inn, rows, group)
    ref = O.oracle().matmul_mxfp4(x, pk, sc, rows, group)
    assert rel_l2(y, ref) < 1e-6
    # a kernel that kept 32-element scale blocks reads other bytes
    sc32 = np.ascontiguousarray(np.resize(sc, rows * ((inn + 31) // 32)))
    wrong = O.oracle().matmul_mxfp4(x, pk, sc32, rows, 32)
    assert rel_l2(wrong, ref) > 1e-3


# ------------------------------------------------------------------------ router ----

def test_router_golden(gpu):
    say("case: k3_router on tests/fixtures/ops/router.json (d=128, 8 experts, top-2, 6 rows)")
    d = np.load(os.path.join(GOLDEN, "router.npz"))
    tol = json.load(open(os.path.join(GOLDEN, "tolerance.json")))["tolerance"]
    E, K = int(d["n_experts"]), int(d["top_k"])
    W = np.ascontiguousarray(d["gate_weight"].reshape(E, -1))
    x = d["x"].reshape(-1, W.shape[1])
    bias = np.ascontiguousarray(d["bias"])
    for r in range(x.shape[0]):
        idx = np.zeros(K, np.int32)
        w = np.zeros(K, np.float32)
        xr = np.ascontiguousarray(x[r])
        k3moe.lib().k3_router(idx.ctypes.data, w.ctypes.data, xr.ctypes.data, W.ctypes.data,
                              bias.ctypes.data, W.shape[1], E, K, 1, 1.0)
        oi, ow = O.oracle().router(xr, W, bias, E, K, 1, 1.0)
        assert np.array_equal(idx, oi), (r, idx, oi)
        exp_i = d["topk_idx"].reshape(-1, K)[r]
        exp_w = d["topk_weight"].reshape(-1, K)[r]
        assert set(idx.tolist()) == set(exp_i.tolist())
        for a in range(K):
            b = list(exp_i).index(idx[a])
            assert abs(w[a] - exp_w[b]) <= tol["fp32_abs"] + tol["fp32_rel"] * abs(exp_w[b])


@pytest.fixture(scope="module")
def k2_layer(gpu):
    say("setup: Kimi-K2-scale layer (d=7168, 384 experts, top-8, I=2048), seed 2024, 9 GB bank "
        "in the checkpoint layout and 9 GB tiled")
    layer = k3moe.SynthLayer(k3moe.K2, seed=2024, layout="both")
    yield layer


@pytest.mark.parametrize("force", [0, 1, 2, 3])
def test_router_k2_bitexact(k2_layer, force):
    """force 1: every token's candidates through the exact path; 2: every expert's float
    logit from the bounded any-order sum (the serial chain where it is unsettled); 3: the
    serial chain for every logit. The exact path's scores, hence weights, are bit-exact."""
    T = 24 if force < 2 else 3
    say(f"case: k3g_router d=7168 E=384 k=8, {T} tokens, force_exact={force}")
    layer = k2_layer
    x = layer.tokens(T, stream_base=7)
    ctx = k3moe.Ctx(layer.dev, max_tokens=T)
    ctx.force_exact(force)
    dx = k3moe.DevBuf.from_array(x)
    didx, dwt = k3moe.DevBuf(T * 8 * 4), k3moe.DevBuf(T * 8 * 4)
    ctx.router(layer.dev, dx.ptr, T, didx.ptr, dwt.ptr)
    ctx.sync()
    idx = didx.download(np.int32, T * 8).reshape(T, 8)
    wt = dwt.download(np.float32, T * 8).reshape(T, 8)
    for t in range(T):
        oi, ow = O.oracle().router(x[t], layer.gate, layer.bias, 384, 8, 1, 2.5)
        assert np.array_equal(idx[t], oi), (t, idx[t], oi)
        np.testing.assert_allclose(wt[t], ow, rtol=1e-6, atol=0)
        if force:
            assert np.array_equal(wt[t].view(np.uint32), ow.view(np.uint32)), t
    if force:
        assert ctx.stats()[0] >= T
    ctx.destroy()


def test_router_ties_and_degenerate(gpu):
    say("case: router with exact ties (zero input, equal biases) and k > distinct values")
    E, d, k = 16, 64, 4
    W = np.ascontiguousarray(k3moe.host_normal(E * d, 3, 77, 0, 0.02).reshape(E, d))
    bias = np.zeros(E, np.float32)
    bias[5] = bias[9] = 0.25
    x = np.zeros(d, np.float32)
    idx = np.zeros(k, np.int32)
    w = np.zeros(k, np.float32)
    k3moe.lib().k3_router(idx.ctypes.data, w.ctypes.data, x.ctypes.data, W.ctypes.data,
                          bias.ctypes.data, d, E, k, 1, 2.5)
    oi, ow = O.oracle().router(x, W, bias, E, k, 1, 2.5)
    assert np.array_equal(idx, oi), (idx, oi)
    np.testing.assert_array_equal(w, ow)


@pytest.mark.parametrize("T,force", [(3, 0), (24, 0), (24, 1), (600, 0)])
def test_router_k3_shape(gpu, T, force):
    """The real K3 router shape: 896 experts (14 per lane in the selection), top-16,
    d = 7168, routed scale 1.0; the per-expert kernel (3 tokens), the sliced matrix-core
    logits (24), the forced exact re-routing and the unsliced matrix-core logits (600)."""
    E, d, k = 896, 7168, 16
    say(f"case: k3g_router K3 shape E={E} k={k} d={d}, {T} tokens, force_exact={force}")
    W = np.ascontiguousarray(k3moe.host_normal(E * d, 11, 501, 0, 0.02).reshape(E, d))
    bias = k3moe.host_normal(E, 11, 502, 0, 0.01)
    x = np.ascontiguousarray(k3moe.host_normal(T * d, 11, 503, 0, 1.0).reshape(T, d))
    L = k3moe.K3gLayer()
    L.hidden, L.n_experts, L.topk, L.inter, L.latent = d, E, k, 128, d
    L.renorm, L.routed_scale = 1, 1.0
    dW, db, dx = (k3moe.DevBuf.from_array(a) for a in (W, bias, x))
    L.gate, L.bias = dW.ptr, db.ptr
    ctx = k3moe.Ctx(L, max_tokens=T)
    ctx.force_exact(force)
    didx, dwt = k3moe.DevBuf(T * k * 4), k3moe.DevBuf(T * k * 4)
    ctx.router(L, dx.ptr, T, didx.ptr, dwt.ptr)
    ctx.sync()
    idx = didx.download(np.int32, T * k).reshape(T, k)
    wt = dwt.download(np.float32, T * k).reshape(T, k)
    for t in (range(T) if T <= 24 else np.random.default_rng(T).choice(T, 24, replace=False)):
        oi, ow = O.oracle().router(x[t], W, bias, E, k, 1, 1.0)
        assert np.array_equal(idx[t], oi), (t, idx[t], oi)
        np.testing.assert_allclose(wt[t], ow, rtol=1e-6, atol=0)
        if force:
            assert np.array_equal(wt[t].view(np.uint32), ow.view(np.uint32)), t
    ctx.destroy()


def test_decode_certificate_ordinary_tokens(k2_layer):
    """The decode kernel's top-k (384 experts, top-8) certifies ordinary tokens on its own:
    eight seeded single-token decodes never enter the exact path (stats[0] counts the
    tokens that do), and routing and weights are the engine's bit for bit."""
    T, d = 8, 7168
    say(f"case: fused decode d=7168 E=384 k=8, {T} single-token calls: certificate without "
        "the exact path")
    layer = k2_layer
    x = layer.tokens(T, stream_base=4242)
    ctx = k3moe.Ctx(layer.dev_tiled, max_tokens=1)
    dx = k3moe.DevBuf.from_array(x)
    dout = k3moe.DevBuf(T * d * 4)
    didx, dwt = k3moe.DevBuf(T * 8 * 4), k3moe.DevBuf(T * 8 * 4)
    for t in range(T):
        ctx.moe(layer.dev_tiled, dx.ptr + t * d * 4, 1, dout.ptr + t * d * 4,
                didx.ptr + t * 32, dwt.ptr + t * 32)
    ctx.sync()
    extra = ctx.stats()[0]
    idx = didx.download(np.int32, T * 8).reshape(T, 8)
    wt = dwt.download(np.float32, T * 8).reshape(T, 8)
    ctx.destroy()
    say(f"  tokens through the exact path: {extra}")
    assert extra == 0
    for t in range(T):
        oi, ow = O.oracle().router(x[t], layer.gate, layer.bias, 384, 8, 1, 2.5)
        assert np.array_equal(idx[t], oi), (t, idx[t], oi)
        assert np.array_equal(wt[t].view(np.uint32), ow.view(np.uint32)), t


@pytest.mark.parametrize("T,force", [(1200, 0), (512, 2)])
def test_router_bounded_logits_k2(k2_layer, T, force):
    """From 512 tokens the logits are formed on the bf16 matrix cores with a rigorous bound
    and only the experts whose bounded score can reach a token's top-k get an fp64 logit
    (force 2: every expert, so the bound is checked on every (token, expert) pair). The
    selection and weights are the engine's bit for bit on sampled tokens, and no fp64 logit
    lies outside its bounded interval (stats[2])."""
    say(f"case: k3g_router bounded bf16 logits d=7168 E=384 k=8, {T} tokens, force_exact={force}")
    layer = k2_layer
    x = layer.tokens(T, stream_base=900)
    ctx = k3moe.Ctx(layer.dev, max_tokens=T)
    ctx.force_exact(force)
    dx = k3moe.DevBuf.from_array(x)
    didx, dwt = k3moe.DevBuf(T * 8 * 4), k3moe.DevBuf(T * 8 * 4)
    ctx.router(layer.dev, dx.ptr, T, didx.ptr, dwt.ptr)
    ctx.sync()
    extra, opened, viol = ctx.stats()[:3]
    say(f"  tokens with extra candidates {extra}, open logits {opened}, bound violations {viol}")
    assert viol == 0
    if force:
        assert extra == T
    else:
        assert extra < T // 2
    idx = didx.download(np.int32, T * 8).reshape(T, 8)
    wt = dwt.download(np.float32, T * 8).reshape(T, 8)
    rng = np.random.default_rng(T + force)
    for t in np.unique(np.concatenate([[0, T - 1], rng.choice(T, 24, replace=False)])):
        oi, ow = O.oracle().router(x[t], layer.gate, layer.bias, 384, 8, 1, 2.5)
        assert np.array_equal(idx[t], oi), (t, idx[t], oi)
        assert np.array_equal(wt[t].view(np.uint32), ow.view(np.uint32)), t
    ctx.destroy()


@pytest.mark.parametrize("E,k", [(64, 4), (16, 4), (144, 9)])
def test_router_bounded_logits_ties(gpu, E, k):
    """The bounded-logit path on exact ties and odd inputs, every token against the
    engine: duplicated router rows with equal biases (tied choices, lowest index wins),
    zero tokens (every logit 0), a token of tiny values and one of huge values, expert
    counts below and not a multiple of the 128-expert tile, a ragged last token tile."""
    d, T = 256, 520
    say(f"case: k3g_router bounded bf16 logits with ties E={E} k={k} d={d}, {T} tokens")
    W = np.ascontiguousarray(k3moe.host_normal(E * d, 13, 601, 0, 0.02).reshape(E, d))
    bias = k3moe.host_normal(E, 13, 602, 0, 0.01)
    for a, b in ((3, 10), (3, E - 6), (0, E - 1)):
        W[b] = W[a]
        bias[b] = bias[a]
    x = np.ascontiguousarray(k3moe.host_normal(T * d, 13, 603, 0, 1.0).reshape(T, d))
    x[5] = 0.0
    x[100] = 0.0
    x[200] *= np.float32(2.0 ** -60)
    x[300] *= np.float32(2.0 ** 40)
    x[301] = x[302]
    L = k3moe.K3gLayer()
    L.hidden, L.n_experts, L.topk, L.inter, L.latent = d, E, k, 128, d
    L.renorm, L.routed_scale = 1, 2.5
    dW, db, dx = (k3moe.DevBuf.from_array(a) for a in (W, bias, x))
    L.gate, L.bias = dW.ptr, db.ptr
    ctx = k3moe.Ctx(L, max_tokens=T)
    didx, dwt = k3moe.DevBuf(T * k * 4), k3moe.DevBuf(T * k * 4)
    ctx.router(L, dx.ptr, T, didx.ptr, dwt.ptr)
    ctx.sync()
    assert ctx.stats()[2] == 0
    idx = didx.download(np.int32, T * k).reshape(T, k)
    wt = dwt.download(np.float32, T * k).reshape(T, k)
    for t in range(T):
        oi, ow = O.oracle().router(x[t], W, bias, E, k, 1, 2.5)
        assert np.array_equal(idx[t], oi), (t, idx[t], oi)
        assert np.array_equal(wt[t].view(np.uint32), ow.view(np.uint32)), t
    ctx.destroy()


# ------------------------------------------------------------------- tiled layouts ----

def _tile_mxfp4_host(packed, scales, rows, cols):
    """The tiled MXFP4 layout, written out block by block on the host."""
    nq = (cols + 511) // 512
    out = np.zeros((rows // 16) * nq * 4352, np.uint8)
    for r in range(rows):
        for b in range(nq * 16):
            rb, Q, j, g = r // 16, b // 16, (b % 16) // 4, b % 4
            L = 16 * g + r % 16
            base = (rb * nq + Q) * 4352
            live = 32 * b < cols and scales[r, b] != 255
            out[base + 1024 * j + 16 * L: base + 1024 * j + 16 * L + 16] = (
                packed[r, 16 * b:16 * b + 16] if live else 0)
            out[base + 4096 + 4 * L + j] = scales[r, b] if live else 127
    return out


@pytest.mark.parametrize("rows,cols", [(32, 96), (16, 512), (48, 1056)])
def test_tile_mxfp4_layout(gpu, rows, cols):
    say(f"case: k3g_tile_mxfp4 rows={rows} cols={cols} (scale 255 blocks included)")
    packed = k3moe.host_bytes(rows * cols // 2, 11, 1).reshape(rows, cols // 2)
    scales = k3moe.host_scales(rows * cols // 32, 11, 2, -3, 3).reshape(rows, cols // 32)
    scales[0, 0] = 255
    scales[rows - 1, cols // 32 - 1] = 255
    n = k3moe.lib().k3g_tiled_mxfp4_bytes(rows, cols)
    dp, ds, dt = k3moe.DevBuf.from_array(packed), k3moe.DevBuf.from_array(scales), k3moe.DevBuf(n)
    assert k3moe.lib().k3g_tile_mxfp4(dt.ptr, dp.ptr, ds.ptr, rows, cols, None) == 0
    k3moe.sync()
    got = dt.download(np.uint8, n)
    assert np.array_equal(got, _tile_mxfp4_host(packed, scales, rows, cols))


def test_tile_bf16_layout(gpu):
    rows, cols = 48, 96
    say(f"case: k3g_tile_bf16 rows={rows} cols={cols}")
    src = k3moe.host_bytes(rows * cols * 2, 12, 1).view(np.uint16).reshape(rows, cols)
    n = k3moe.lib().k3g_tiled_bf16_bytes(rows, cols)
    ds, dt = k3moe.DevBuf.from_array(src), k3moe.DevBuf(n)
    assert k3moe.lib().k3g_tile_bf16(dt.ptr, ds.ptr, rows, cols, None) == 0
    k3moe.sync()
    got = dt.download(np.uint16, rows * cols)
    exp = np.zeros(rows * cols, np.uint16)
    for rb in range(rows // 16):
        for c in range(cols // 32):
            for L in range(64):
                o = ((rb * (cols // 32) + c) * 64 + L) * 8
                exp[o:o + 8] = src[16 * rb + L % 16, 32 * c + 8 * (L // 16): 32 * c + 8 * (L // 16) + 8]
    assert np.array_equal(got, exp)
    assert k3moe.lib().k3g_tiled_bf16_bytes(40, 96) == 0


# ------------------------------------------------------------------------- layer ----

@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("T", [1, 2, 3, 4, 7])
def test_layer_tiny_decode(gpu, T, fused):
    say(f"case: k3g_moe tiny layer (d=256, E=16, k=4, I=128), {T} tokens, fused={fused}")
    layer = k3moe.SynthLayer(k3moe.TINY, seed=1234, layout="both")
    x = layer.tokens(T)
    out, idx, wt = run_layer(layer, x, fused=fused)
    ro, ri, rw = oracle_tokens(layer, x)
    assert np.array_equal(idx, ri)
    np.testing.assert_allclose(wt, rw, rtol=1e-6)
    assert rel_l2(out, ro) <= REL_L2


@pytest.mark.parametrize("fused", [False, True])
def test_layer_k2_decode_one_token(k2_layer, fused):
    say(f"case: k3g_moe K2 layer, 1-token decode, 3 different tokens, fused={fused}")
    layer = k2_layer
    for s in range(3):
        x = layer.tokens(1, stream_base=20 + s)
        out, idx, _ = run_layer(layer, x, fused=fused)
        ro, ri, _ = oracle_tokens(layer, x)
        assert np.array_equal(idx, ri)
        r = rel_l2(out, ro)
        say(f"  token {s}: rel-L2 {r:.3e}")
        assert r <= REL_L2
        # the staged kernels accumulate in fp32 on the vector ALUs; the fused kernel's
        # matrix cores see activations split into pieces (residual below 2^-24 of each
        # block's maximum) and accumulate in their own order
        assert r <= (1e-4 if fused else 1e-5)


def test_layer_k2_fused_repeat_and_force(k2_layer):
    say("case: fused K2 decode: 4 tokens in one call, 6 repeated launches, the exact "
        "re-routing forced in modes 1, 2 and 3 on three of them")
    layer = k2_layer
    x = layer.tokens(4, stream_base=60)
    ro, ri, rw = oracle_tokens(layer, x)
    ctx = k3moe.Ctx(layer.dev, max_tokens=4)
    for rep, force in enumerate([0, 1, 0, 2, 3, 0]):
        out, idx, wt = run_layer(layer, x, ctx=ctx, force=force)
        assert np.array_equal(idx, ri), rep
        assert rel_l2(out, ro) <= REL_L2, rep
        if force:
            assert np.array_equal(wt.view(np.uint32), rw.astype(np.float32).view(np.uint32)), rep
    ctx.destroy()


def test_layer_k2_fused_consecutive_tokens(k2_layer):
    say("case: fused K2 decode, 6 consecutive launches on one context, a new token each")
    layer = k2_layer
    ctx = k3moe.Ctx(layer.dev_tiled, max_tokens=2)
    for i in range(6):
        T = 1 + i % 2
        x = layer.tokens(T, stream_base=80 + 3 * i)
        out, idx, _ = run_layer(layer, x, ctx=ctx)
        ro, ri, _ = oracle_tokens(layer, x)
        assert np.array_equal(idx, ri), i
        r = rel_l2(out, ro)
        say(f"  launch {i} ({T} tokens): rel-L2 {r:.3e}")
        assert r <= 1e-4, i
    ctx.destroy()


@pytest.mark.parametrize("T,xkind", [(5, "fp32"), (16, "fp32"), (37, "fp32"), (200, "fp32"),
                                     (37, "bf16"), (200, "bf16")])
def test_layer_tiny_grouped_gemm(gpu, T, xkind):
    say(f"case: k3g_moe tiny layer on the grouped bf16 MFMA GEMMs, {T} tokens, x {xkind} "
        "(fp32: two activation pieces on 8-wave workgroups; bf16: one piece, 4-wave)")
    layer = k3moe.SynthLayer(k3moe.TINY, seed=4321, layout="both")
    x = layer.tokens(T)
    if xkind == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        x = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)
        assert not np.any(x.view(np.uint32) & 0xFFFF)
    out, idx, wt = run_layer(layer, x, tiled=True)
    ro, ri, rw = oracle_tokens(layer, x)
    assert np.array_equal(idx, ri)
    np.testing.assert_allclose(wt, rw, rtol=1e-6)
    r = rel_l2(out, ro)
    say(f"  rel-L2 {r:.3e}")
    assert r <= GEMM_REL


@pytest.mark.parametrize("T,xkind", [(40, "bf16"), (24, "fp32")])
def test_layer_k2_grouped_gemm(k2_layer, T, xkind):
    say(f"case: k3g_moe K2 layer on the grouped bf16 MFMA GEMMs, {T} tokens, x {xkind}")
    layer = k2_layer
    x = layer.tokens(T, stream_base=140)
    if xkind == "fp32":
        # values that are not bf16: the gate/up products need both activation pieces
        x = (x * np.float32(1.0 + 2.0 ** -12)).astype(np.float32)
        assert np.any(x.view(np.uint32) & 0xFFFF)
    out, idx, _ = run_layer(layer, x, tiled=True)
    ro, ri, _ = oracle_tokens(layer, x)
    assert np.array_equal(idx, ri)
    r = rel_l2(out, ro)
    say(f"  rel-L2 {r:.3e}")
    assert r <= GEMM_REL


@pytest.mark.parametrize("shape,T,nsample", [("K2_BATCH", 64, 6), ("K2_PREFILL", 4096, 6)])
def test_layer_k2_skewed_full_size(gpu, shape, T, nsample):
    """The batched-decode (64 tokens, Zipf(1.1)) and prefill (4096 tokens, Zipf(0.8))
    workloads at full size: routing bit-exact for a sample of tokens, sampled output rows
    against the oracle, and the size-independent property that a token's output does not
    depend on where it sits in the batch (the same tokens reversed give the same bits)."""
    say(f"case: k3g_moe {shape} ({T} tokens, skewed routing, grouped bf16 GEMMs): sampled "
        f"rows vs the oracle, reversed batch bit-identical")
    layer = k3moe.SynthLayer(getattr(k3moe, shape), seed=2024, layout="tiled")
    s = layer.shape
    x = layer.tokens(T, stream_base=500)
    ctx = k3moe.Ctx(layer.dev_tiled, max_tokens=T)
    out, idx, wt = run_layer(layer, x, ctx=ctx, tiled=True)
    out_r, idx_r, _ = run_layer(layer, np.ascontiguousarray(x[::-1]), ctx=ctx, tiled=True)
    ctx.destroy()
    assert np.array_equal(out_r[::-1].view(np.uint32), out.view(np.uint32))
    assert np.array_equal(idx_r[::-1], idx)
    counts = np.bincount(idx.reshape(-1), minlength=s.n_experts)
    say(f"  experts used {int((counts > 0).sum())}, most popular {int(counts.max())} pairs")
    rng = np.random.default_rng(T)
    rt = np.unique(np.concatenate([[0, T - 1], rng.choice(T, size=min(T, 64), replace=False)]))
    k = O.oracle()
    for t in rt:
        oi, ow = k.router(x[t], layer.gate, layer.bias, s.n_experts, s.topk, s.renorm,
                          s.routed_scale)
        assert np.array_equal(idx[t], oi), t
        np.testing.assert_allclose(wt[t], ow, rtol=1e-6, atol=0)
    # sampled rows: one token of the most popular expert among them
    hot = int(np.argmax(counts))
    t_hot = int(np.nonzero((idx == hot).any(axis=1))[0][0])
    st = np.unique(np.concatenate([[0, T - 1, t_hot], rng.choice(T, size=nsample, replace=False)]))
    ro, ri, _ = oracle_tokens(layer, x[st])
    assert np.array_equal(idx[st], ri)
    r = rel_l2(out[st], ro)
    say(f"  {len(st)} sampled rows: rel-L2 {r:.3e}")
    assert r <= GEMM_REL


def test_layer_k2_batch(k2_layer):
    say("case: k3g_moe K2 layer, 12 tokens in one call")
    layer = k2_layer
    x = layer.tokens(12, stream_base=40)
    out, idx, _ = run_layer(layer, x)
    ro, ri, _ = oracle_tokens(layer, x)
    assert np.array_equal(idx, ri)
    assert rel_l2(out, ro) <= REL_L2


# ------------------------------------------------------ the layer's steps one at a time ----

SENTINEL = np.uint32(0x7FC0DEAD)   # a NaN the kernels never write


def _shape_only_layer(hidden, E, topk, inter):
    L = k3moe.K3gLayer()
    L.hidden, L.n_experts, L.topk, L.inter, L.latent = hidden, E, topk, inter, hidden
    return L


def _random_routing(T, E, k, seed, drop=0.05):
    """k distinct experts per token, skewed towards low ids, a fraction dropped (-1)."""
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, E + 1) ** 0.9
    p /= p.sum()
    idx = np.stack([rng.choice(E, size=k, replace=False, p=p) for _ in range(T)])
    idx[rng.random((T, k)) < drop] = -1
    return idx.astype(np.int32)


def _dispatch_expected(idx, E):
    """Stable sort of the pair numbers by expert id, ids < 0 left out."""
    flat = idx.reshape(-1)
    keep = np.nonzero(flat >= 0)[0]
    perm = keep[np.argsort(flat[keep], kind="stable")].astype(np.int32)
    cnt = np.bincount(flat[keep], minlength=E)
    off = np.concatenate([[0], np.cumsum(cnt)]).astype(np.int32)
    return perm, off


@pytest.mark.parametrize("T,E,k", [(1, 384, 8), (20, 384, 8), (32, 384, 8), (33, 384, 8),
                                   (300, 384, 8), (512, 384, 8), (4096, 384, 8), (50, 16, 4),
                                   (600, 896, 16), (1537, 1024, 4), (4100, 64, 2),
                                   (4096, 896, 16)])
def test_dispatch_is_a_stable_sort(gpu, T, E, k):
    P = T * k
    path = "one block" if P <= 256 else "one 1024-thread block" if P <= 4096 else "three passes"
    say(f"case: k3g_dispatch, {T} tokens x top-{k} over {E} experts ({P} pairs, {path})")
    ctx = k3moe.Ctx(_shape_only_layer(128, E, k, 128), max_tokens=T)
    idx = _random_routing(T, E, k, seed=T * 7 + E)
    perm_e, off_e = _dispatch_expected(idx, E)
    didx = k3moe.DevBuf.from_array(idx)
    dperm, doff = k3moe.DevBuf(P * 4), k3moe.DevBuf((E + 1) * 4)
    ctx.dispatch(didx.ptr, T, k, E, dperm.ptr, doff.ptr)
    ctx.sync()
    off = doff.download(np.int32, E + 1)
    perm = dperm.download(np.int32, P)
    assert np.array_equal(off, off_e)
    assert np.array_equal(perm[:off[E]], perm_e)
    ctx.destroy()


@pytest.mark.parametrize("T", [8, 2000])
def test_dispatch_all_dropped(gpu, T):
    say(f"case: k3g_dispatch, every slot of {T} tokens dropped (idx -1)")
    ctx = k3moe.Ctx(_shape_only_layer(128, 64, 4, 128), max_tokens=T)
    didx = k3moe.DevBuf.from_array(np.full((T, 4), -1, np.int32))
    dperm, doff = k3moe.DevBuf(T * 4 * 4), k3moe.DevBuf(65 * 4)
    ctx.dispatch(didx.ptr, T, 4, 64, dperm.ptr, doff.ptr)
    ctx.sync()
    assert not np.any(doff.download(np.int32, 65))
    ctx.destroy()


@pytest.mark.parametrize("T,k,n,with_add", [(7, 8, 260, True), (3, 4, 7168, False),
                                            (64, 8, 1024, True)])
def test_combine_bit_exact(gpu, T, k, n, with_add):
    say(f"case: k3g_combine, {T} tokens x top-{k}, width {n}, shared add {with_add}")
    rng = np.random.default_rng(n + T)
    contrib = rng.standard_normal((T * k, n)).astype(np.float32)
    idx = _random_routing(T, 64, k, seed=T, drop=0.2)
    wt = rng.random((T, k)).astype(np.float32)
    add = rng.standard_normal((T, n)).astype(np.float32) if with_add else None
    # slot order, multiply and add rounded separately, dropped slots skipped
    exp = np.zeros((T, n), np.float32)
    c3 = contrib.reshape(T, k, n)
    for j in range(k):
        m = idx[:, j] >= 0
        exp[m] = exp[m] + wt[m, j:j + 1] * c3[m, j]
    if with_add:
        exp = exp + add
    ctx = k3moe.Ctx(_shape_only_layer(n, 64, k, 128), max_tokens=T)
    dc, di, dw = (k3moe.DevBuf.from_array(a) for a in (contrib, idx, wt))
    da = k3moe.DevBuf.from_array(add) if with_add else None
    dout = k3moe.DevBuf(T * n * 4)
    ctx.combine(dc.ptr, di.ptr, dw.ptr, T, k, n, da.ptr if da else None, dout.ptr)
    ctx.sync()
    out = dout.download(np.float32, T * n).reshape(T, n)
    assert np.array_equal(out.view(np.uint32), exp.view(np.uint32))
    ctx.destroy()


def _pair_rows(layer, x, idx, pairs, quant=False):
    """Oracle rows w2 . SwiGLU(w1 . x_t, w3 . x_t) of the given (t, j) pairs; quant: x and
    h through MXFP8 first (the FP4 x FP8 variant's inputs)."""
    k, g, s = O.oracle(), layer.geo, layer.shape
    cap = k3moe.SWIGLU_CAP
    runs, out = {}, []
    for t, j in pairs:
        e = int(idx[t, j])
        if e not in runs:
            runs[e] = layer.expert_host(e)
        r = runs[e]
        xt = O.quant_mxfp8(x[t]) if quant else np.ascontiguousarray(x[t])
        gu = np.concatenate([k.matmul_mxfp4(xt, r[g.p1_off:g.s1_off], r[g.s1_off:g.p2_off],
                                            s.inter),
                             k.matmul_mxfp4(xt, r[g.p3_off:g.s3_off], r[g.s3_off:g.nbytes],
                                            s.inter)])
        h = k.situ(gu.astype(np.float32), cap, cap)
        if quant:
            h = O.quant_mxfp8(h)
        out.append(k.matmul_mxfp4(h, r[g.p2_off:g.s2_off], r[g.s2_off:g.p3_off], s.hidden))
    return np.stack(out)


def _run_experts(layer, kind, x, idx):
    T, k, d = x.shape[0], layer.shape.topk, layer.shape.hidden
    L = layer.dev if kind == "gemv" else layer.dev_tiled
    ctx = k3moe.Ctx(L, max_tokens=T)
    dx, di = k3moe.DevBuf.from_array(x), k3moe.DevBuf.from_array(idx)
    dc = k3moe.DevBuf.from_array(np.full((T * k, d), SENTINEL, np.uint32))
    ctx.experts(kind, L, dx.ptr, T, di.ptr, dc.ptr)
    ctx.sync()
    ctx.destroy()
    return dc.download(np.float32, T * k * d).reshape(T, k, d)


def test_grouped_remainder_extremes(gpu):
    """h's MXFP8 remainder at its edges: tokens of zeros (every remainder block zero, scale
    byte 0) give rows of exact zeros; tokens scaled by 2^-20 and 2^12 (remainder blocks far
    from 1, activation caps reached) stay within the grouped tolerance of the oracle."""
    T = 24
    say(f"case: grouped bf16 experts, tiny layer, {T} tokens: zero rows, tiny and large rows")
    layer = k3moe.SynthLayer(k3moe.TINY, seed=4242, layout="both")
    x = layer.tokens(T).copy()
    x[0:4] = 0.0
    x[4:10] *= np.float32(2.0 ** -20)
    x[10:16] *= np.float32(2.0 ** 12)
    idx = _random_routing(T, layer.shape.n_experts, layer.shape.topk, seed=5, drop=0.0)
    rows = _run_experts(layer, "bf16", x, idx)
    assert np.all(rows[0:4] == 0.0), "zero tokens must give exact zeros"
    kept = [(t, j) for t in range(4, T) for j in range(layer.shape.topk)]
    exp = _pair_rows(layer, x, idx, kept)
    got = np.stack([rows[t, j] for t, j in kept])
    assert np.all(np.isfinite(got))
    for lo, hi in ((4, 10), (10, 16), (16, T)):
        sel = [i for i, (t, _) in enumerate(kept) if lo <= t < hi]
        r = rel_l2(got[sel], exp[sel])
        say(f"  tokens {lo}..{hi - 1}: rel-L2 {r:.3e}")
        assert r <= GEMM_REL


@pytest.mark.parametrize("kind,T", [("gemv", 3), ("gemv", 37), ("bf16", 5), ("bf16", 37),
                                    ("bf16", 200), ("f8f6f4", 37)])
def test_expert_products_per_pair(gpu, kind, T):
    say(f"case: routed expert products alone ({kind}), tiny layer, {T} tokens, 10% slots "
        "dropped: every kept pair's row vs the oracle, dropped rows untouched")
    layer = k3moe.SynthLayer(k3moe.TINY, seed=777, layout="both")
    x = layer.tokens(T)
    idx = _random_routing(T, layer.shape.n_experts, layer.shape.topk, seed=T, drop=0.1)
    rows = _run_experts(layer, kind, x, idx)
    kept = [(t, j) for t in range(T) for j in range(layer.shape.topk) if idx[t, j] >= 0]
    dropped = [(t, j) for t in range(T) for j in range(layer.shape.topk) if idx[t, j] < 0]
    exp = _pair_rows(layer, x, idx, kept, quant=kind == "f8f6f4")
    got = np.stack([rows[t, j] for t, j in kept])
    r = rel_l2(got, exp)
    worst = max(rel_l2(a, b) for a, b in zip(got, exp))
    say(f"  rel-L2 {r:.3e}, worst row {worst:.3e}")
    assert r <= (5e-3 if kind == "f8f6f4" else GEMM_REL if kind == "bf16" else 1e-5)
    assert worst <= (1e-2 if kind == "f8f6f4" else 4 * GEMM_REL if kind == "bf16" else 1e-4)
    for t, j in dropped:
        assert np.all(rows[t, j].view(np.uint32) == SENTINEL)


@pytest.mark.parametrize("kind,T", [("gemv", 2), ("bf16", 24)])
def test_expert_products_k2(k2_layer, kind, T):
    say(f"case: routed expert products alone ({kind}), K2 layer, {T} tokens, the routing the "
        "router picks; the first 24 pairs against the oracle")
    layer = k2_layer
    x = layer.tokens(T, stream_base=190)
    _, idx, _ = oracle_tokens(layer, x)
    idx = idx.astype(np.int32)
    rows = _run_experts(layer, kind, x, idx)
    pairs = [(t, j) for t in range(T) for j in range(layer.shape.topk)][:24]
    exp = _pair_rows(layer, x, idx, pairs)
    r = rel_l2(np.stack([rows[t, j] for t, j in pairs]), exp)
    say(f"  rel-L2 {r:.3e}")
    assert r <= GEMM_REL


def test_steps_compose_to_the_layer(gpu):
    T = 37
    say(f"case: router -> grouped bf16 -> combine, plus the shared expert, against k3g_moe "
        f"and the oracle, tiny layer, {T} tokens")
    layer = k3moe.SynthLayer(k3moe.TINY, seed=4321, layout="tiled")
    s, k = layer.shape, O.oracle()
    x = layer.tokens(T)
    out, idx, wt = run_layer(layer, x, tiled=True)
    rows = _run_experts(layer, "bf16", x, idx)
    ctx = k3moe.Ctx(layer.dev_tiled, max_tokens=T)
    dc, di, dw = (k3moe.DevBuf.from_array(np.ascontiguousarray(a)) for a in
                  (rows.reshape(T * s.topk, s.hidden), idx, wt))
    dr = k3moe.DevBuf(T * s.hidden * 4)
    ctx.combine(dc.ptr, di.ptr, dw.ptr, T, s.topk, s.hidden, None, dr.ptr)
    ctx.sync()
    ctx.destroy()
    routed = dr.download(np.float32, T * s.hidden).reshape(T, s.hidden)
    pairs = [(t, j) for t in range(T) for j in range(s.topk)]
    exp = _pair_rows(layer, x, idx, pairs).reshape(T, s.topk, s.hidden)
    ref = np.zeros((T, s.hidden), np.float32)
    for j in range(s.topk):
        ref = ref + wt[:, j:j + 1] * exp[:, j]
    r_routed = rel_l2(routed, ref)
    cap = k3moe.SWIGLU_CAP
    shared = np.stack([
        k.matmul_bf16(k.situ(np.concatenate([k.matmul_bf16(x[t], layer.sh1, layer.SI),
                                             k.matmul_bf16(x[t], layer.sh3, layer.SI)]),
                             cap, cap), layer.sh2, s.hidden) for t in range(T)])
    r_layer = rel_l2(routed + shared, out)
    say(f"  routed sum vs oracle {r_routed:.3e}; + shared expert vs k3g_moe {r_layer:.3e}")
    assert r_routed <= GEMM_REL
    assert r_layer <= 1e-5


# --------------------------------------------------------------------- drop-in ABI ----

def _moe_json_weights():
    d = np.load(os.path.join(GOLDEN, "moe.npz"))
    cfg = k3moe.K3Cfg()
    cfg.hidden, cfg.latent, cfg.moe_inter = int(d["hidden"]), int(d["latent"]), int(d["moe_inter"])
    cfg.n_experts, cfg.topk, cfg.n_shared = int(d["n_experts"]), int(d["top_k"]), int(d["n_shared"])
    cfg.routed_scale, cfg.moe_renorm = float(d["routed_scale"]), int(d["renorm"])
    cfg.latent_norm, cfg.rms_eps = int(d["latent_norm"]), float(d["rms_eps"])
    cfg.situ_b1, cfg.situ_b2 = float(d["situ_b1"]), float(d["situ_b2"])
    keep = {k: np.ascontiguousarray(d[k], np.float32) for k in d.files
            if d[k].dtype == np.float32 and d[k].ndim > 0}
    w = k3moe.K3MoeW()
    w.gate, w.bias = keep["gate_weight"].ctypes.data, keep["e_score_correction_bias"].ctypes.data
    w.w1, w.w3, w.w2 = keep["w1"].ctypes.data, keep["w3"].ctypes.data, keep["w2"].ctypes.data
    w.latent_norm = keep["norm_weight"].ctypes.data
    w.down, w.up = keep["down_weight"].ctypes.data, keep["up_weight"].ctypes.data
    w.sh1, w.sh3 = keep["shared_w1_weight"].ctypes.data, keep["shared_w3_weight"].ctypes.data
    w.sh2 = keep["shared_w2_weight"].ctypes.data
    return w, cfg, keep


def test_dropin_moe_json(gpu):
    say("case: k3_moe on tests/fixtures/ops/moe.json (LatentMoE, SiTU(4,25), fp32 bank)")
    w, cfg, keep = _moe_json_weights()
    tol = json.load(open(os.path.join(GOLDEN, "tolerance.json")))["tolerance"]
    x = keep["in"].reshape(-1, cfg.hidden)
    T = x.shape[0]
    out = np.zeros_like(x)
    idx = np.zeros(cfg.topk, np.int32)
    wt = np.zeros(cfg.topk, np.float32)
    k3moe.lib().k3_moe(out.ctypes.data, x.ctypes.data, C.byref(w), C.byref(cfg), T,
                       idx.ctypes.data, wt.ctypes.data, None)
    exp = keep["out"].reshape(out.shape)
    worst = np.max(np.abs(out - exp) / (tol["fp32_abs"] + tol["fp32_rel"] * np.abs(exp)))
    say(f"  worst {worst:.2f}x tolerance")
    assert worst <= 1.0
    oo, oi, ow = O.oracle().moe(w, cfg, x)
    assert np.array_equal(idx, oi)
    assert rel_l2(out, oo) <= 1e-5


@pytest.mark.parametrize("prefill,T", [(False, 5), (True, 70), (True, 65)])
def test_dropin_k3_moe_host_source(gpu, prefill, T):
    say(f"case: {'k3_moe_prefill' if prefill else 'k3_moe'} tiny K2 layer, T={T}, host expert source")
    layer = k3moe.SynthLayer(k3moe.TINY, seed=99, device=False)
    x = layer.tokens(T)
    experts = list(range(layer.shape.n_experts))
    w, cfg, keep = O.k2_weights(layer, experts)
    out = np.zeros_like(x)
    idx = np.full(cfg.topk, -7, np.int32)
    wt = np.zeros(cfg.topk, np.float32)
    f = k3moe.lib().k3_moe_prefill if prefill else k3moe.lib().k3_moe
    f(out.ctypes.data, x.ctypes.data, C.byref(w), C.byref(cfg), T, idx.ctypes.data,
      wt.ctypes.data, None)
    gets_gpu = keep[1].s.gets
    w2, cfg2, keep2 = O.k2_weights(layer, experts)
    oo, oi, ow = O.oracle().moe(w2, cfg2, x, prefill=prefill)
    assert rel_l2(out, oo) <= REL_L2
    assert gets_gpu == keep2[1].s.gets, "expert source saw a different request pattern"
    if not prefill or (T - 1) % 64 == 0:
        assert np.array_equal(idx, oi)
        np.testing.assert_allclose(wt, ow, rtol=1e-6)
    else:
        assert np.all(idx == -7), "batched prefill must leave idx/wt untouched"


def test_dropin_k3_shape_latent_moe(gpu):
    """The real K3 LatentMoE shape through the drop-in k3_moe: d 7168, 896 MXFP4 experts
    top-16 at latent width 3584 (I 3072), bf16 latent down/up projections, RMSNorm of the
    aggregate, two shared experts fused (6144), SiTU(4, 25), routed scale 1.0; synthetic
    seeded weights, experts from a host source; against the oracle's k3_moe."""
    T = 2
    d, E, k, Lw, I, SI = 7168, 896, 16, 3584, 3072, 6144
    say(f"case: k3_moe K3 shape (d={d}, E={E}, top-{k}, latent {Lw}, I={I}, shared {SI}, "
        f"SiTU 4/25, latent RMSNorm), {T} tokens, host expert source")
    shape = k3moe.Shape("K3 latent experts", Lw, E, k, I, n_shared=2, routed_scale=1.0,
                        x_bf16=False)
    experts = k3moe.SynthLayer(shape, seed=31, device=False)
    gate = np.ascontiguousarray(k3moe.host_normal(E * d, 31, 601, 0.0, 0.02))
    bias = k3moe.host_normal(E, 31, 602, 0.0, 0.01)
    lnorm = k3moe.host_normal(Lw, 31, 603, 1.0, 0.1)
    bf = lambda n, s: k3moe.bf16_bits(k3moe.host_normal(n, 31, s, 0.0, 0.02, bf16=True))  # noqa: E731
    down, up = bf(Lw * d, 604), bf(d * Lw, 605)
    sh1, sh3, sh2 = bf(SI * d, 606), bf(SI * d, 607), bf(d * SI, 608)
    x = np.ascontiguousarray(k3moe.host_normal(T * d, 31, 609, 0.0, 1.0).reshape(T, d))
    kk = O.oracle()
    used = sorted({int(e) for t in range(T)
                   for e in kk.router(x[t], gate, bias, E, k, 1, 1.0)[0]})
    runs = {(0, e): experts.expert_host(e) for e in used}

    def weights():
        src = O.MemSrc(runs, 1, E, experts.geo)
        w = k3moe.K3MoeW()
        w.gate, w.bias, w.latent_norm = gate.ctypes.data, bias.ctypes.data, lnorm.ctypes.data
        w.down, w.up = down.ctypes.data, up.ctypes.data
        w.sh1, w.sh3, w.sh2 = sh1.ctypes.data, sh3.ctypes.data, sh2.ctypes.data
        w.wdt = k3moe.K3_WBF16
        w.src, w.layer = src.ptr, 0
        return w, src

    cfg = k3moe.K3Cfg()
    cfg.hidden, cfg.latent, cfg.moe_inter = d, Lw, I
    cfg.n_experts, cfg.topk, cfg.n_shared = E, k, 2
    cfg.routed_scale, cfg.moe_renorm, cfg.latent_norm = 1.0, 1, 1
    cfg.rms_eps, cfg.situ_b1, cfg.situ_b2, cfg.n_layers = 1e-6, 4.0, 25.0, 1
    w, src = weights()
    out = np.zeros_like(x)
    idx = np.zeros(k, np.int32)
    wt = np.zeros(k, np.float32)
    k3moe.lib().k3_moe(out.ctypes.data, x.ctypes.data, C.byref(w), C.byref(cfg), T,
                       idx.ctypes.data, wt.ctypes.data, None)
    paths = k3moe.lib().k3moe_last_kernels()
    k3moe.lib().k3moe_forget_weights()
    w2, src2 = weights()
    oo, oi, ow = kk.moe(w2, cfg, x)
    r = rel_l2(out, oo)
    say(f"  rel-L2 {r:.3e}, {len(used)} experts, kernels {paths}")
    assert paths == 2          # the fused decode kernel, latent tickets, routing given
    assert np.array_equal(idx, oi)
    np.testing.assert_allclose(wt, ow, rtol=1e-6)
    assert r <= REL_L2


def test_dropin_expert_drop(gpu):
    say("case: k3_moe with a source that fails one expert: drop counted, slot skipped")
    layer = k3moe.SynthLayer(k3moe.TINY, seed=5, device=False)
    x = layer.tokens(6)
    O_ = O.oracle()
    union = O.routed_union(layer, x)
    missing = union[0]
    experts = [e for e in range(layer.shape.n_experts) if e != missing]
    w, cfg, keep = O.k2_weights(layer, experts)
    drops0 = C.c_long.in_dll(k3moe.lib(), "k3_expert_drops").value
    out = np.zeros_like(x)
    idx = np.zeros(cfg.topk, np.int32)
    wt = np.zeros(cfg.topk, np.float32)
    k3moe.lib().k3_moe(out.ctypes.data, x.ctypes.data, C.byref(w), C.byref(cfg), 6,
                       idx.ctypes.data, wt.ctypes.data, None)
    drops = C.c_long.in_dll(k3moe.lib(), "k3_expert_drops").value - drops0
    w2, cfg2, keep2 = O.k2_weights(layer, experts)
    od0 = O_.drops.value
    oo, _, _ = O_.moe(w2, cfg2, x)
    assert drops == O_.drops.value - od0 and drops > 0
    assert rel_l2(out, oo) <= REL_L2


# ------------------------------------------------------- FP4 x FP8 matrix cores ----

def _e4m3_decode(b):
    b = b.astype(np.int64)
    s = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 7
    v = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (e - 7))
    return s * v


def test_mxfp8_quantiser_matches_the_oracle(gpu):
    say("case: k3k_xq8 (hardware E4M3 conversion) vs the oracle's OCP MX quantiser, "
        "incl. zero blocks, 448 clamps, E4M3 subnormals and ties")
    T, d = 6, 256
    x = k3moe.host_normal(T * d, 31, 5, 0.0, 1.0).reshape(T, d)
    x[0, :32] = 0.0                                         # zero block
    x[1, :32] = 1.0 / 256
    x[1, 0] = 1.99                                          # 1.99 * 2^8 > 448: clamped
    x[2, :32] = np.float32(1.0)
    x[2, 1:8] = np.float32(1e-5)                            # E4M3 subnormals of the block
    x[3, :32] = np.float32(1.0625) * 2.0 ** -3              # ties between 1.0 and 1.125
    x[3, 0] = 1.0
    x = np.ascontiguousarray(x, np.float32)
    L = k3moe.lib()
    L.k3k_xq8.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    dx, dq, ds = k3moe.DevBuf.from_array(x), k3moe.DevBuf(T * d), k3moe.DevBuf(T * d // 32)
    assert L.k3k_xq8(dx.ptr, T, d, d, dq.ptr, ds.ptr, None) == 0
    k3moe.sync()
    q = dq.download(np.uint8, T * d).reshape(T, d // 32, 32)
    sc = ds.download(np.uint8, T * d // 32).reshape(T, d // 32, 1).astype(np.int64)
    got = (_e4m3_decode(q) * 2.0 ** (sc - 127)).astype(np.float32).reshape(T, d)
    exp = O.quant_mxfp8(x.ravel()).reshape(T, d)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
    assert got[1, 0] == np.float32(448.0 * 2.0 ** -8)


@pytest.mark.parametrize("T", [16])
def test_layer_k2_fp4xfp8_variant(k2_layer, T):
    say(f"case: k3g_moe K2 layer, {T} tokens, routed experts on the FP4 x FP8 matrix cores "
        "(MXFP8 activations) vs the quantisation-aware oracle")
    layer = k2_layer
    x = layer.tokens(T, stream_base=170)
    ctx = k3moe.Ctx(layer.dev_tiled, max_tokens=T)
    ctx.set_fp8(True)
    out, idx, _ = run_layer(layer, x, ctx=ctx, tiled=True)
    ctx.destroy()
    q = O.k2_forward_mxfp8(layer, x)
    ro, ri, _ = oracle_tokens(layer, x)
    assert np.array_equal(idx, ri)
    r_q, r_u = rel_l2(out, q), rel_l2(out, ro)
    say(f"  rel-L2 vs quantisation-aware oracle {r_q:.3e}, vs the unquantised engine {r_u:.3e}")
    assert r_q <= 5e-3
    assert r_u <= 0.1


def test_layer_tiny_fp4xfp8_variant(gpu):
    T = 37
    say(f"case: k3g_moe tiny layer, {T} tokens, FP4 x FP8 variant vs the quantisation-aware oracle")
    layer = k3moe.SynthLayer(k3moe.TINY, seed=4321, layout="tiled")
    x = layer.tokens(T)
    ctx = k3moe.Ctx(layer.dev_tiled, max_tokens=T)
    ctx.set_fp8(True)
    out, idx, _ = run_layer(layer, x, ctx=ctx, tiled=True)
    ctx.destroy()
    q = O.k2_forward_mxfp8(layer, x)
    r = rel_l2(out, q)
    say(f"  rel-L2 {r:.3e}")
    assert r <= 5e-3
