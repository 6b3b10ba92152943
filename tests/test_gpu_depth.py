"""GPU parity at full size, checked row by row against the oracle where the other tests
sample a handful of rows:

* the 64-token Zipf(1.1) batch: every output row;
* the 4096-token Zipf(0.8) prefill, both variants: a token set that reaches every active
  expert at least once (greedy cover of the routing), plus the tokens of the first and
  last pair of every 128-pair column tile of the three most popular experts (pairs are
  grouped by expert in token order, so those rows sit at the tiles' edges);
* the same prefill with fp32-valued x (two activation pieces, 8-wave workgroups);
* the real K3 LatentMoE layer through the device API (latent down/up, latent RMSNorm, two
  shared experts, SiTU(4, 25)) at 64 and 600 tokens;
* the grouped path's router at 520 tokens with every expert a candidate (force 2), for
  bf16-valued x (the router skips the w0 x1 product) and fp32-valued x.

Pattern: the engine's own test_ops t_moe (tests/unit/test_ops.c:465-545) compares k3_moe
against a scalar composition of its kernels; here the oracle is that composition. Each
test prints its case before touching the GPU."""
import numpy as np
import pytest

import k3moe
import oracle as O
from test_gpu_parity import oracle_tokens, rel_l2, run_layer, say

pytestmark = pytest.mark.gpu
GEMM_REL = 1e-4
REL_L2 = 1e-3
FP8_REL = 5e-3
TILE = 128


def _cover_tokens(idx, n_experts):
    """Greedy set cover: tokens whose routing reaches every expert used by idx [T][k]."""
    T = idx.shape[0]
    M = np.zeros((T, n_experts), bool)
    rows = np.repeat(np.arange(T), idx.shape[1])
    keep = idx.reshape(-1) >= 0
    M[rows[keep], idx.reshape(-1)[keep]] = True
    left = M.any(axis=0)
    chosen = []
    while left.any():
        gain = (M & left).sum(axis=1)
        t = int(np.argmax(gain))
        chosen.append(t)
        left &= ~M[t]
    return chosen


def _tile_edge_tokens(idx, n_experts, nhot=3):
    """Tokens of the first and last pair of every 128-pair column tile of the nhot most
    popular experts (an expert's pairs in token order, as the stable dispatch sorts them)."""
    counts = np.bincount(idx[idx >= 0], minlength=n_experts)
    hot = np.argsort(-counts, kind="stable")[:nhot]
    out = []
    for e in hot:
        toks = np.nonzero((idx == e).any(axis=1))[0]
        n = len(toks)
        for a in range(0, n, TILE):
            out += [int(toks[a]), int(toks[min(a + TILE, n) - 1])]
    return [int(e) for e in hot], [int(c) for c in counts[hot]], out


def _oracle_rows(layer, x):
    """The oracle's layer output for tokens x and each token's routing. The outputs come
    from the oracle's k3_moe_prefill (bit-identical per token to its k3_moe, and
    expert-major, so each expert's weights are regenerated once)."""
    s = layer.shape
    out, _, _ = O.k2_forward(layer, x, prefill=True)
    k = O.oracle()
    idx = np.stack([k.router(x[t], layer.gate, layer.bias, s.n_experts, s.topk, s.renorm,
                             s.routed_scale)[0] for t in range(x.shape[0])])
    return out, idx


def test_batch64_every_row(gpu):
    T = 64
    say(f"case: k3g_moe K2_BATCH ({T} tokens, Zipf(1.1)), grouped GEMMs: every row vs the oracle")
    layer = k3moe.SynthLayer(k3moe.K2_BATCH, seed=2024, layout="tiled")
    x = layer.tokens(T, stream_base=1900)
    out, idx, wt = run_layer(layer, x, tiled=True)
    ro, ri = _oracle_rows(layer, x)
    assert np.array_equal(idx, ri)
    per_row = [rel_l2(out[t], ro[t]) for t in range(T)]
    r = rel_l2(out, ro)
    say(f"  {len(np.unique(idx))} experts; rel-L2 all rows {r:.3e}, worst row {max(per_row):.3e}")
    assert r <= GEMM_REL
    assert max(per_row) <= 2 * GEMM_REL


@pytest.fixture(scope="module")
def prefill_run(gpu):
    """The 4096-token Zipf(0.8) prefill of the bench, on both variants of the routed
    experts, from one context."""
    T = 4096
    say(f"setup: K2_PREFILL layer, {T} tokens (the bench's inputs), bf16 and FP4 x FP8 runs")
    layer = k3moe.SynthLayer(k3moe.K2_PREFILL, seed=2024, layout="tiled")
    x = layer.tokens(T, stream_base=900)
    ctx = k3moe.Ctx(layer.dev_tiled, max_tokens=T)
    out, idx, wt = run_layer(layer, x, ctx=ctx, tiled=True)
    ctx.set_fp8(True)
    out8, idx8, _ = run_layer(layer, x, ctx=ctx, tiled=True)
    ctx.set_fp8(False)
    ctx.destroy()
    assert np.array_equal(idx8, idx)
    yield layer, x, out, out8, idx, wt


def _prefill_tokens(idx, E):
    cover = _cover_tokens(idx, E)
    hot, cnt, edges = _tile_edge_tokens(idx, E)
    tokens = np.unique(np.array(cover + edges, np.int64))
    say(f"  {len(cover)} tokens cover all {len(np.unique(idx[idx >= 0]))} active experts; "
        f"hottest experts {hot} with {cnt} pairs give {len(set(edges))} tile-edge tokens")
    return tokens


def test_prefill_bf16_every_expert(prefill_run):
    layer, x, out, _, idx, wt = prefill_run
    s = layer.shape
    say("case: K2_PREFILL bf16 grouped GEMMs: every active expert and the hot experts' tile "
        "edges vs the oracle")
    tokens = _prefill_tokens(idx, s.n_experts)
    ro, ri = _oracle_rows(layer, x[tokens])
    assert np.array_equal(idx[tokens], ri)
    per_row = np.array([rel_l2(out[t], ro[n]) for n, t in enumerate(tokens)])
    r = rel_l2(out[tokens], ro)
    say(f"  {len(tokens)} rows: rel-L2 {r:.3e}, worst row {per_row.max():.3e}")
    assert r <= GEMM_REL
    assert per_row.max() <= 2 * GEMM_REL


def test_prefill_fp4xfp8_every_expert(prefill_run):
    layer, x, _, out8, idx, _ = prefill_run
    s = layer.shape
    say("case: K2_PREFILL FP4 x FP8 grouped GEMMs: every active expert and the hot experts' "
        "tile edges vs the quantisation-aware oracle")
    tokens = _prefill_tokens(idx, s.n_experts)
    q = O.k2_forward_mxfp8(layer, x[tokens])
    per_row = np.array([rel_l2(out8[t], q[n]) for n, t in enumerate(tokens)])
    r = rel_l2(out8[tokens], q)
    say(f"  {len(tokens)} rows: rel-L2 {r:.3e}, worst row {per_row.max():.3e}")
    assert r <= FP8_REL
    assert per_row.max() <= 2 * FP8_REL


def test_prefill_fp32_x(gpu):
    """The engine's decoder passes fp32 hin into k3_moe_prefill (src/core/k3_ops.c:1015-1024):
    x values that are not bf16 take two activation pieces on 8-wave workgroups and the
    router's full three products."""
    T = 4096
    say(f"case: k3g_moe K2_PREFILL {T} tokens, fp32-valued x: sampled rows + the hot experts' "
        f"tile edges vs the oracle")
    layer = k3moe.SynthLayer(k3moe.K2_PREFILL, seed=2024, layout="tiled")
    x = layer.tokens(T, stream_base=900)
    x = (x * np.float32(1.0 + 2.0 ** -12)).astype(np.float32)
    assert np.any(x.view(np.uint32) & 0xFFFF)
    ctx = k3moe.Ctx(layer.dev_tiled, max_tokens=T)
    out, idx, _ = run_layer(layer, x, ctx=ctx, tiled=True)
    viol = ctx.stats()[2]
    ctx.destroy()
    assert viol == 0
    _, _, edges = _tile_edge_tokens(idx, layer.shape.n_experts, nhot=1)
    rng = np.random.default_rng(4097)
    tokens = np.unique(np.concatenate([[0, T - 1], edges, rng.choice(T, 12, replace=False)]))
    ro, ri = _oracle_rows(layer, x[tokens])
    assert np.array_equal(idx[tokens], ri)
    r = rel_l2(out[tokens], ro)
    say(f"  {len(tokens)} rows: rel-L2 {r:.3e}")
    assert r <= GEMM_REL


@pytest.mark.parametrize("xkind", ["bf16", "fp32"])
def test_grouped_router_every_candidate(gpu, xkind):
    """k3g_moe on the grouped path at 520 tokens with every expert a candidate (force 2):
    no fp64 logit outside its bounded interval, and every token's indices and weights
    bit-exact against the engine. bf16-valued x runs the bounded logits without the w0 x1
    product (its flag is clear); fp32-valued x runs all three products."""
    T = 520
    say(f"case: k3g_moe K2 layer {T} tokens, x {xkind}, router force_exact=2: every token's "
        f"routing bit-exact, bound violations 0")
    layer = k3moe.SynthLayer(k3moe.K2, seed=2024, layout="tiled")
    x = layer.tokens(T, stream_base=2600)
    if xkind == "fp32":
        x = (x * np.float32(1.0 + 2.0 ** -12)).astype(np.float32)
        assert np.any(x.view(np.uint32) & 0xFFFF)
    else:
        assert not np.any(x.view(np.uint32) & 0xFFFF)
    ctx = k3moe.Ctx(layer.dev_tiled, max_tokens=T)
    out, idx, wt = run_layer(layer, x, ctx=ctx, force=2, tiled=True)
    extra, opened, viol = ctx.stats()[:3]
    ctx.destroy()
    say(f"  tokens with extra candidates {extra}, open logits {opened}, violations {viol}")
    assert viol == 0 and extra == T
    s = layer.shape
    k = O.oracle()
    for t in range(T):
        oi, ow = k.router(x[t], layer.gate, layer.bias, s.n_experts, s.topk, s.renorm,
                          s.routed_scale)
        assert np.array_equal(idx[t], oi), t
        assert np.array_equal(wt[t].view(np.uint32), ow.view(np.uint32)), t
    assert np.isfinite(out).all()


def test_router_beyond_512_tile_pairs(gpu):
    """More than 512 (128-expert x 128-token) tiles: the bounded bf16 logits run with one
    K slice. 896 experts, d 256, 9600 tokens (525 tiles)."""
    E, d, k, T = 896, 256, 16, 9600
    say(f"case: k3g_router bounded bf16 logits with {((E + 127) // 128) * ((T + 127) // 128)} "
        f"tiles: E={E} k={k} d={d}, {T} tokens")
    W = np.ascontiguousarray(k3moe.host_normal(E * d, 17, 701, 0, 0.02).reshape(E, d))
    bias = k3moe.host_normal(E, 17, 702, 0, 0.01)
    x = np.ascontiguousarray(k3moe.host_normal(T * d, 17, 703, 0, 1.0).reshape(T, d))
    L = k3moe.K3gLayer()
    L.hidden, L.n_experts, L.topk, L.inter, L.latent = d, E, k, 128, d
    L.renorm, L.routed_scale = 1, 1.0
    dW, db, dx = (k3moe.DevBuf.from_array(a) for a in (W, bias, x))
    L.gate, L.bias = dW.ptr, db.ptr
    ctx = k3moe.Ctx(L, max_tokens=T)
    didx, dwt = k3moe.DevBuf(T * k * 4), k3moe.DevBuf(T * k * 4)
    ctx.router(L, dx.ptr, T, didx.ptr, dwt.ptr)
    ctx.sync()
    extra, opened, viol = ctx.stats()[:3]
    ctx.destroy()
    say(f"  tokens with extra candidates {extra}, open logits {opened}, violations {viol}")
    assert viol == 0
    idx = didx.download(np.int32, T * k).reshape(T, k)
    wt = dwt.download(np.float32, T * k).reshape(T, k)
    rng = np.random.default_rng(9600)
    for t in np.unique(np.concatenate([[0, T - 1], rng.choice(T, 200, replace=False)])):
        oi, ow = O.oracle().router(x[t], W, bias, E, k, 1, 1.0)
        assert np.array_equal(idx[t], oi), (t, idx[t], oi)
        assert np.array_equal(wt[t].view(np.uint32), ow.view(np.uint32)), t


# ------------------------------------------------------------ K3 LatentMoE layer ----

class K3Layer:
    """The real Kimi-K3 LatentMoE layer with seeded synthetic weights: d 7168, 896 MXFP4
    experts top-16 at latent 3584 x I 3072, bf16 latent down/up, latent RMSNorm, two shared
    experts fused (6144), SiTU(4, 25), routed scale 1.0. Host copies for the oracle, tiled
    copies in HBM for the device API."""
    d, E, k, Lw, I, SI = 7168, 896, 16, 3584, 3072, 6144

    def __init__(self, seed=31):
        import ctypes as C
        lib = k3moe.lib()
        d, E, Lw, I, SI = self.d, self.E, self.Lw, self.I, self.SI
        shape = k3moe.Shape("K3 latent experts", Lw, E, self.k, I, n_shared=2,
                            routed_scale=1.0, x_bf16=False)
        self.experts = k3moe.SynthLayer(shape, seed=seed, layout="tiled")
        n = lambda cnt, s, m, sd, bf=False: k3moe.host_normal(cnt, seed, s, m, sd, bf16=bf)  # noqa: E731
        self.gate = np.ascontiguousarray(n(E * d, 601, 0.0, 0.02))
        self.bias = n(E, 602, 0.0, 0.01)
        self.lnorm = n(Lw, 603, 1.0, 0.1)
        bf = lambda cnt, s: k3moe.bf16_bits(n(cnt, s, 0.0, 0.02, True))  # noqa: E731
        self.down, self.up = bf(Lw * d, 604), bf(d * Lw, 605)
        self.sh1, self.sh3, self.sh2 = bf(SI * d, 606), bf(SI * d, 607), bf(d * SI, 608)
        self.keep = []

        def tiled(bits, rows, cols):
            src = k3moe.DevBuf.from_array(bits)
            t = k3moe.DevBuf(lib.k3g_tiled_bf16_bytes(rows, cols))
            k3moe._check(lib.k3g_tile_bf16(C.c_void_p(t.ptr), C.c_void_p(src.ptr), rows, cols,
                                           None), "k3g_tile_bf16")
            k3moe.sync()
            self.keep.append(t)
            return t.ptr

        g, b, ln = (k3moe.DevBuf.from_array(a) for a in (self.gate, self.bias, self.lnorm))
        self.keep += [g, b, ln]
        L = k3moe.K3gLayer()
        L.hidden, L.n_experts, L.topk, L.inter = d, E, self.k, I
        L.shared_inter, L.latent = SI, Lw
        L.renorm, L.routed_scale, L.act_b1, L.act_b2, L.rms_eps = 1, 1.0, 4.0, 25.0, 1e-6
        L.gate, L.bias, L.latent_norm = g.ptr, b.ptr, ln.ptr
        L.expert_fmt, L.experts = k3moe.K3G_EXPERT_MXFP4_TILED, self.experts.d_ttable.ptr
        L.wdt, L.shared_fmt = k3moe.K3_WBF16, 1
        L.down, L.up = tiled(self.down, Lw, d), tiled(self.up, d, Lw)
        L.sh1, L.sh3 = tiled(self.sh1, SI, d), tiled(self.sh3, SI, d)
        L.sh2 = tiled(self.sh2, d, SI)
        self.L = L

    def oracle(self, x):
        """The oracle's k3_moe_prefill over tokens x (per token bit-identical to its k3_moe),
        and each token's routing from the oracle's router."""
        kk = O.oracle()
        E, k = self.E, self.k
        idx = np.stack([kk.router(x[t], self.gate, self.bias, E, k, 1, 1.0)[0]
                        for t in range(x.shape[0])])
        used = sorted({int(e) for e in idx.reshape(-1)})
        runs = {(0, e): self.experts.expert_host(e) for e in used}
        src = O.MemSrc(runs, 1, E, self.experts.geo)
        w = k3moe.K3MoeW()
        w.gate, w.bias, w.latent_norm = self.gate.ctypes.data, self.bias.ctypes.data, \
            self.lnorm.ctypes.data
        w.down, w.up = self.down.ctypes.data, self.up.ctypes.data
        w.sh1, w.sh3, w.sh2 = self.sh1.ctypes.data, self.sh3.ctypes.data, self.sh2.ctypes.data
        w.wdt = k3moe.K3_WBF16
        w.src, w.layer = src.ptr, 0
        cfg = k3moe.K3Cfg()
        cfg.hidden, cfg.latent, cfg.moe_inter = self.d, self.Lw, self.I
        cfg.n_experts, cfg.topk, cfg.n_shared = E, k, 2
        cfg.routed_scale, cfg.moe_renorm, cfg.latent_norm = 1.0, 1, 1
        cfg.rms_eps, cfg.situ_b1, cfg.situ_b2, cfg.n_layers = 1e-6, 4.0, 25.0, 1
        out, _, _ = kk.moe(w, cfg, x, prefill=True)
        del runs, src
        return out, idx


@pytest.fixture(scope="module")
def k3_layer(gpu):
    say("setup: K3 LatentMoE layer (d 7168, 896 experts top-16, latent 3584, I 3072, shared "
        "6144), 15.7 GB tiled bank")
    lay = K3Layer()
    yield lay
    del lay


def test_k3_decode_certificate_ordinary_tokens(k3_layer):
    """The decode kernel's top-k at 896 experts, top-16 certifies ordinary tokens on its
    own: six seeded single-token decodes never enter the exact path (stats[0]), and the
    routing is the engine's."""
    lay = k3_layer
    T = 6
    say(f"case: fused decode K3 E=896 k=16, {T} single-token calls: certificate without the "
        "exact path")
    x = np.ascontiguousarray(k3moe.host_normal(T * lay.d, 31, 4343, 0.0, 1.0).reshape(T, lay.d))
    ctx = k3moe.Ctx(lay.L, max_tokens=1)
    dx = k3moe.DevBuf.from_array(x)
    dout = k3moe.DevBuf(T * lay.d * 4)
    didx, dwt = k3moe.DevBuf(T * lay.k * 4), k3moe.DevBuf(T * lay.k * 4)
    for t in range(T):
        ctx.moe(lay.L, dx.ptr + t * lay.d * 4, 1, dout.ptr + t * lay.d * 4,
                didx.ptr + t * lay.k * 4, dwt.ptr + t * lay.k * 4)
    ctx.sync()
    extra = ctx.stats()[0]
    idx = didx.download(np.int32, T * lay.k).reshape(T, lay.k)
    ctx.destroy()
    say(f"  tokens through the exact path: {extra}")
    assert extra == 0
    kk = O.oracle()
    for t in range(T):
        oi, _ = kk.router(x[t], lay.gate, lay.bias, lay.E, lay.k, 1, 1.0)
        assert np.array_equal(idx[t], oi), t


@pytest.mark.parametrize("T,nsample", [(1, 1), (2, 2), (4, 4), (64, 10), (600, 8)])
def test_k3_latent_moe_device(k3_layer, T, nsample):
    """Up to 4 tokens: the fused decode kernel with its latent tickets (z = down x, the
    routed experts on z, the slot-order aggregate, its RMSNorm, up, + shared); more: the
    grouped GEMMs with the latent projections."""
    lay = k3_layer
    kind = "fused decode kernel" if T <= 4 else "grouped GEMMs"
    say(f"case: k3g_moe K3 LatentMoE, {T} tokens, {kind} with latent projections: "
        f"routing bit-exact for every token, {nsample} sampled rows vs the oracle")
    x = np.ascontiguousarray(k3moe.host_normal(T * lay.d, 31, 609 + T, 0.0, 1.0).reshape(T, lay.d))
    ctx = k3moe.Ctx(lay.L, max_tokens=T)
    dx = k3moe.DevBuf.from_array(x)
    dout = k3moe.DevBuf(T * lay.d * 4)
    didx, dwt = k3moe.DevBuf(T * lay.k * 4), k3moe.DevBuf(T * lay.k * 4)
    ctx.paths()
    ctx.moe(lay.L, dx.ptr, T, dout.ptr, didx.ptr, dwt.ptr)
    ctx.sync()
    paths = ctx.paths()
    out = dout.download(np.float32, T * lay.d).reshape(T, lay.d)
    idx = didx.download(np.int32, T * lay.k).reshape(T, lay.k)
    wt = dwt.download(np.float32, T * lay.k).reshape(T, lay.k)
    ctx.destroy()
    assert paths == (2 if T <= 4 else 4), paths
    kk = O.oracle()
    for t in range(T):
        oi, ow = kk.router(x[t], lay.gate, lay.bias, lay.E, lay.k, 1, 1.0)
        assert np.array_equal(idx[t], oi), t
        np.testing.assert_allclose(wt[t], ow, rtol=1e-6, atol=0)
    rng = np.random.default_rng(T)
    st = np.unique(np.concatenate([[0, T - 1], rng.choice(T, nsample, replace=False)]))
    ro, ri = lay.oracle(x[st])
    assert np.array_equal(idx[st], ri)
    r = rel_l2(out[st], ro)
    say(f"  {len(np.unique(idx))} experts used; {len(st)} rows: rel-L2 {r:.3e}")
    assert r <= REL_L2
