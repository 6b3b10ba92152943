#!/usr/bin/env python3
"""Benchmark: one Kimi-K2-scale routed-expert MoE layer on one MI355X.

Workload (the step): single-token decode through one MoE layer with d=7168, 384 routed
MXFP4 experts (top-8, intermediate 2048, SwiGLU), one bf16 shared expert, fp32 router
with selection bias, routed scale 2.5. Synthetic seeded weights and bf16-valued N(0,1)
activations, every tensor resident in HBM before timing starts. Each step runs a new
token through the next of --layers distinct layers (round robin), so consecutive steps
stream different experts and different shared/router weights, as a decode pass over a
stack of layers does, instead of re-reading what the 256 MB last-level cache holds.

Prints one JSON line. value = tokens/s (1 token per step); ms_per_step is the layer
latency per token. roofline: the dominant kernel (the fused decode kernel), timed with HIP
events bracketing the timed region on the stream it runs on (every step is one launch, so
the average includes the gap between back-to-back launches), against HBM peak. prefill: a 4096-token prefill of the
same layer with Zipf(0.8) expert popularity (tokens/s, fraction of the bf16 MFMA peak,
its own roofline entry for the dominant GEMM). cpu_baseline: the engine's own CPU
kernels on this host's cores on a bounded sample of the decode workload.
"""
import argparse
import json
import os
import platform
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "kimi-k3-in-rust_amd"))

METRIC = ("MoE layer decode µs/token + HBM GB/s; prefill tokens/s + MFMA util")
HBM_PEAK_GBS = 8000.0

# algorithmic bytes (one token, c1 shapes)
D, E, K, I = 7168, 384, 8, 2048
B_EXPERT = 3 * I * D * 17 // 32            # 23,396,352: packed nibbles + E8M0 scales
B_SHARED = 6 * I * D                       # 88,080,384: three bf16 matrices
B_ROUTER = 4 * E * D + 4 * E               # 11,011,584: fp32 gate + bias
B_TOKEN = D * 2 + D * 4                    # bf16-valued input, fp32 output
B_GATEUP_EXPERT = 2 * (I * D // 2 + I * D // 32)   # w1 + w3 of one expert

# HBM bytes per launch of the fused decode kernel on this workload, from two rocprofv3
# --pmc runs (FETCH_SIZE x 1.9997 + WRITE_SIZE x 1.0, the factors that make a 256 MiB
# device-to-device copy read 256 MiB); the run and the numbers are in
# profiles/k_decode_fused_k2_decode.md. Re-measured whenever the kernel changes.
TRAFFIC_FUSED = 302055321
# HBM bytes per launch of the routed gate/up GEMM (k_gemm<0, 4>) of the 4096-token
# Zipf(0.8) prefill, the same way (FETCH_SIZE x 1.9997 + WRITE_SIZE, mean of 3 launches):
# 7.666 GB read + 0.204 GB written; profiles/k_gemm_k2_prefill4096.md.
TRAFFIC_GATEUP_PREFILL = 7869400121
# the same for the fp32-x sub-leg's routed gate/up (k_gemm<0, 8>: x in two bf16 pieces),
# mean of its last 6 launches: 8.059 GB read + 0.203 GB written;
# profiles/k_gemm_k2_prefill4096.md.
TRAFFIC_GATEUP_PREFILL_FP32 = 8261930315


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def host_cpu():
    """CPU model, sockets and physical cores of this host (lscpu)."""
    info = {"model": platform.processor() or "cpu", "sockets": None, "physical_cores": None,
            "logical_cpus": os.cpu_count()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        f = {}
        for line in out.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                f[k.strip()] = v.strip()
        info["model"] = f.get("Model name", info["model"])
        if f.get("Socket(s)", "").isdigit():
            info["sockets"] = int(f["Socket(s)"])
        if f.get("Core(s) per socket", "").isdigit() and info["sockets"]:
            info["physical_cores"] = int(f["Core(s) per socket"]) * info["sockets"]
    except OSError:
        pass
    return info


def cpu_baseline(seconds: float, max_tokens: int, seed: int,
                 legs=("decode", "identity", "batch", "prefill", "streamed")):
    """The engine's CPU kernels (k3_router, k3_matmul_mxfp4, k3_situ_glu, k3_matmul_bf16,
    compiled from the engine's src/core/k3_ops.c with its flags: kind "reference"; the C
    restatement when that library is absent: kind "port") composed as k3_moe /
    k3_moe_prefill (src/core/k3_ops.c:556-808) for the same K2 layers. Expert
    regeneration on the host is outside the timed regions; every routed expert the timed
    call reads is in host RAM.
      decode: median over a bounded sample of 1-token calls (the c1 workload), without
        the latent projections (down = up = NULL);
      identity_latent: the same tokens through the full k3_moe with bf16 identity latent
        matrices (7168 x 7168, as the engine must express a K2 layer);
      batch: one 64-token k3_moe_prefill call (64-token chunk) on the Zipf(1.1) layer;
      prefill: 128 tokens (two 64-token chunks) of the Zipf(0.8) 4096-token prefill, three
        calls;
      streamed: the 16-layer x batch-8 workload, one 8-token k3_moe_prefill call per
        layer, as many of the 16 layers as a bounded sample allows."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import k3moe
    import oracle as O
    ref = O.ref()
    kind = "reference" if ref else "port"
    if ref:
        O.set_kernels(ref)
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count()
    cpu = host_cpu()
    what = ("the engine's own kernels compiled from src/core/k3_ops.c" if ref else
            "the C restatement of the engine's kernels")
    res = {"cores": threads, "kind": kind, "cpu": cpu,
           "omp": {v: os.environ.get(v, "unset") for v in
                   ("OMP_NUM_THREADS", "OMP_PROC_BIND", "OMP_PLACES")}}
    if "decode" in legs:
        layer = k3moe.SynthLayer(k3moe.K2, seed=seed, layer=0, device=False)
        times = []
        for i in range(max_tokens):
            x = layer.tokens(1, stream_base=5000 + i)
            experts = O.routed_union(layer, x)
            w, cfg, keep = O.k2_weights(layer, experts)
            t0 = time.perf_counter()
            O.oracle().moe(w, cfg, x)
            times.append(time.perf_counter() - t0)
            del keep
            if sum(times) >= seconds and len(times) >= 3:
                break
        med = float(np.median(times))
        res.update({"value": round(1e6 * med, 1), "unit": "us/token",
                    "sample": f"{len(times)} decode tokens through the same K2 layer (median), "
                              f"{what} composed as k3_moe without identity latent, OpenMP "
                              f"{threads} threads on {cpu['model']}",
                    "tokens_per_s": round(1.0 / med, 2),
                    "GBps": round((K * B_EXPERT + B_SHARED + B_ROUTER + B_TOKEN) / med / 1e9, 2)})
        del layer
    if "identity" in legs:
        # the full k3_moe as the engine runs a K2 layer: bf16 identity latent down and up
        layer = k3moe.SynthLayer(k3moe.K2, seed=seed, layer=0, device=False)
        times = []
        for i in range(max_tokens):
            x = layer.tokens(1, stream_base=5000 + i)
            experts = O.routed_union(layer, x)
            w, cfg, keep = O.k2_weights(layer, experts, identity=True)
            t0 = time.perf_counter()
            O.oracle().moe(w, cfg, x)
            times.append(time.perf_counter() - t0)
            del keep
            if sum(times) >= seconds / 2 and len(times) >= 3:
                break
        med = float(np.median(times))
        res["identity_latent"] = {
            "value": round(1e6 * med, 1), "unit": "us/token",
            "tokens_per_s": round(1.0 / med, 2),
            "sample": f"{len(times)} decode tokens (the decode sample's first ones, median) "
                      f"through the full k3_moe with bf16 identity latent matrices "
                      f"(7168 x 7168 down and up), {what}, OpenMP {threads} threads"}
        del layer
    for leg, shape, T, base, reps in (("batch", k3moe.K2_BATCH, 64, 1900, 1),
                                      ("prefill", k3moe.K2_PREFILL, 128, 900, 3)):
        if leg not in legs:
            continue
        layer = k3moe.SynthLayer(shape, seed=seed, layer=0, device=False)
        x = layer.tokens(T, stream_base=base)
        experts = O.routed_union(layer, x)
        w, cfg, keep = O.k2_weights(layer, experts)
        runs = []
        for _ in range(reps):
            t0 = time.perf_counter()
            O.oracle().moe(w, cfg, x, prefill=True)
            runs.append(time.perf_counter() - t0)
        dt = float(np.median(runs))
        del keep, layer
        res[leg] = {"tokens": T, "seconds": round(dt, 3), "tokens_per_s": round(T / dt, 2),
                    "us_per_token": round(1e6 * dt / T, 1), "experts": len(experts),
                    "sample": f"{T} tokens of the {shape.name} workload through one "
                              f"k3_moe_prefill call (64-token chunks, first-seen unique "
                              f"experts), {what}, OpenMP {threads} threads"
                              + (f"; median of {reps} calls" if reps > 1 else "")}
        if reps > 1:
            res[leg]["runs_seconds"] = [round(r, 3) for r in runs]
    if "streamed" in legs:
        # 16 K2 layers x batch 8, one 8-token k3_moe_prefill call per layer with every
        # routed expert in host RAM; bounded: the layers that fit the sample
        times, nexp = [], []
        for l in range(16):
            layer = k3moe.SynthLayer(k3moe.K2, seed=seed, layer=l, device=False)
            x = layer.tokens(8, stream_base=2950)
            experts = O.routed_union(layer, x)
            w, cfg, keep = O.k2_weights(layer, experts)
            t0 = time.perf_counter()
            O.oracle().moe(w, cfg, x, prefill=True)
            times.append(time.perf_counter() - t0)
            nexp.append(len(experts))
            del keep, layer
            if sum(times) >= seconds / 2 and len(times) >= 2:
                break
        per_layer = float(np.mean(times))
        res["streamed"] = {
            "layers_timed": len(times), "batch": 8,
            "seconds_per_layer": round(per_layer, 4),
            "experts_per_layer": round(float(np.mean(nexp)), 1),
            "ms_per_step_16_layers": round(16e3 * per_layer, 1),
            "tokens_per_s": round(8 / (16 * per_layer), 2),
            "sample": f"the 16-layer x batch-8 streamed workload: {len(times)} of the 16 K2 "
                      f"layers, one 8-token k3_moe_prefill call each with every routed "
                      f"expert in host RAM, {what}, OpenMP {threads} threads; the step "
                      f"time is 16 x the mean layer time"}
    O.set_kernels(None)
    return res


# algorithmic flops of a T-token prefill step (routed gate/up + down, shared, router)
def prefill_flops(T):
    routed = 2 * T * K * 3 * I * D
    shared = 6 * T * I * D
    router = 2 * T * E * D
    return routed, shared, router


BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0


def batch_decode(a):
    """64-token batched decode through the same K2 layer with Zipf(1.1) expert popularity
    (~200 distinct experts per step): the grouped expert GEMMs with per-expert column
    lists, the sort-based dispatch and the slot-ordered combine. HBM-bound: bytes per step
    = U expert runs + shared + router + activations, U measured from the routing."""
    import numpy as np
    import k3moe
    T = a.batch_tokens
    log(f"bench: batched decode {T} tokens, Zipf(1.1) routing skew")
    layers = [k3moe.SynthLayer(k3moe.K2_BATCH, seed=a.seed, layer=l, layout="tiled")
              for l in range(2)]
    n = a.batch_warmup + a.batch_steps
    xs = layers[0].tokens(T * n, stream_base=1900)
    ctx = k3moe.Ctx(layers[0].dev, max_tokens=T)
    dx = k3moe.DevBuf.from_array(xs)
    dout = k3moe.DevBuf(T * n * D * 4)
    didx, dwt = k3moe.DevBuf(T * n * K * 4), k3moe.DevBuf(T * n * K * 4)

    def step(i):
        ctx.moe(layers[i % 2].dev, dx.ptr + i * T * D * 4, T, dout.ptr + i * T * D * 4,
                didx.ptr + i * T * K * 4, dwt.ptr + i * T * K * 4)

    for i in range(a.batch_warmup):
        step(i)
    ctx.sync()
    k3moe.sync()
    t0 = time.perf_counter()
    for i in range(a.batch_warmup, n):
        step(i)
    k3moe.sync()
    t1 = time.perf_counter()
    ctx.sync()
    idx = didx.download(np.int32, T * n * K).reshape(n, T * K)
    U = [len(np.unique(r[r >= 0])) for r in idx[a.batch_warmup:]]
    out = dout.download(np.float32, T * n * D)
    assert np.isfinite(out).all()
    ctx.destroy()
    del layers
    ms = (t1 - t0) * 1e3 / a.batch_steps
    u = float(np.mean(U))
    step_bytes = u * B_EXPERT + B_SHARED + B_ROUTER + T * B_TOKEN
    return {"tokens": T, "ms_per_step": round(ms, 4), "tokens_per_s": round(T / (ms * 1e-3), 1),
            "us_per_token": round(1e3 * ms / T, 2), "experts_per_step": round(u, 1),
            "bytes_per_step": int(step_bytes),
            "hbm_GBps": round(step_bytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "steps": a.batch_steps, "warmup": a.batch_warmup,
            "workload": "64-token batched decode, same K2 layer, Zipf(1.1) selection-bias "
                        "skew (alpha 0.025), 2 layers round-robin; grouped bf16 MFMA GEMMs, "
                        "h's MXFP8 remainder on scaled FP8 MFMA"}


def expert_trace(n_steps, n_layers, T, seed, reuse=0.7, zipf_s=1.0, per_step=40):
    """Routing of a streamed decode, per (step, layer): the step's `per_step` distinct
    experts, of which `reuse` are carried over from the previous step's and the rest drawn
    by Zipf(s) popularity over a seeded per-layer permutation of the experts, dealt to the
    tokens so every one of them is used (token t takes the K consecutive entries from 8 t,
    wrapping, of a shuffled list: distinct within a token). Returns idx
    [steps][layers][T][K] int32 and the routed weights (uniform routed_scale / K)."""
    import numpy as np
    rng = np.random.default_rng(seed)
    pop = []
    for _ in range(n_layers):
        perm = rng.permutation(E)
        p = np.empty(E)
        p[perm] = np.arange(1, E + 1, dtype=np.float64) ** (-zipf_s)
        pop.append(p / p.sum())
    idx = np.empty((n_steps, n_layers, T, K), np.int32)
    prev = [None] * n_layers
    for s in range(n_steps):
        for l in range(n_layers):
            keep = [] if prev[l] is None else list(rng.choice(prev[l], int(round(reuse * per_step)),
                                                            replace=False))
            p = pop[l].copy()
            p[keep] = 0.0
            p /= p.sum()
            fresh = rng.choice(E, per_step - len(keep), replace=False, p=p)
            cur = np.array(keep + list(fresh), np.int64)
            prev[l] = cur
            deal = rng.permutation(cur)
            for t in range(T):
                idx[s, l, t] = deal[(K * t + np.arange(K)) % deal.size]
    wt = np.full(idx.shape, 2.5 / K, np.float32)
    return idx, wt


def streamed_decode(a):
    """16 stacked K2 layers whose ~144 GB of routed MXFP4 experts live in a pinned host
    bank, with the HBM expert cache capped at 48 GB: batch-8 decode steps through all
    layers, per-layer Zipf(1.0) routing with 70% of each step's experts reused from the
    previous step (trace-driven). Misses are copied on the cache's stream; the shared
    expert runs while they copy. The trace runs as a previous segment (--cache-steps
    steps, untimed) and the measured segment (--cache-steps steps): first with LRU, then
    with the hottest half of the slots pinned from the previous segment's request
    histogram (k3gc_pin_hottest), warmed on the previous segment's last --cache-warmup
    steps."""
    import numpy as np
    import k3moe
    NL, T = a.cache_layers, a.cache_tokens
    log(f"bench: streamed decode, {NL} layers in a pinned host bank, {a.cache_gb} GB HBM cache")
    bank = k3moe.Bank(NL, E, D, I, k3moe.K3G_EXPERT_MXFP4_TILED)
    layers = []
    for l in range(NL):
        lay = k3moe.SynthLayer(k3moe.K2, seed=a.seed, layer=l, layout="tiled")
        bank.fill_from_layer(lay, l)
        lay.release_experts()
        layers.append(lay)
    S = a.cache_steps
    idx, wt = expert_trace(2 * S, NL, T, a.seed + 11)
    ctx = k3moe.Ctx(layers[0].dev_tiled, max_tokens=T)
    x = layers[0].tokens(T, stream_base=2900)
    dx = k3moe.DevBuf.from_array(x)
    dout, didx, dwt = k3moe.DevBuf(T * D * 4), k3moe.DevBuf(T * K * 4), k3moe.DevBuf(T * K * 4)

    def step(cache, s):
        for l in range(NL):
            cache.moe(ctx, layers[l].dev_tiled, l, dx.ptr, T, dout.ptr, didx.ptr, dwt.ptr,
                      idx[s, l], wt[s, l])

    def measured(cache, label, extra):
        cache.reset_stats()
        t0 = time.perf_counter()
        for s in range(S, 2 * S):
            step(cache, s)
        ctx.sync()
        t1 = time.perf_counter()
        st = cache.stats()
        assert np.isfinite(dout.download(np.float32, T * D)).all()
        ms = (t1 - t0) * 1e3 / S
        served = max(st.hits - st.prefetch_reads, 0)
        r = {"policy": label, "ms_per_step": round(ms, 3), "ms_per_token_latency": round(ms, 3),
             "tokens_per_s": round(T / (ms * 1e-3), 2), "requests": st.requests,
             "true_hit_rate": round(served / max(st.requests, 1), 4),
             "misses_copied": st.prefetch_reads + st.misses,
             "pcie_GB": round(st.bytes_read / 1e9, 2),
             "pcie_GBps_while_copying": round(st.bytes_read / 1e9 / max(st.load_seconds, 1e-9), 1),
             "pcie_GBps_over_run": round(st.bytes_read / 1e9 / (t1 - t0), 1),
             "copy_stream_busy_frac": round(st.load_seconds / (t1 - t0), 3)}
        r.update(extra)
        return r, st

    lru_cache = k3moe.Cache(bank, topk=K, budget_bytes=int(a.cache_gb * 1e9))
    for s in range(S):                      # the previous segment
        step(lru_cache, s)
    ctx.sync()
    hist = lru_cache.hist()
    lru, st = measured(lru_cache, "LRU", {})
    nslot = st.nslot
    lru_cache.free()
    pin_cache = k3moe.Cache(bank, topk=K, budget_bytes=int(a.cache_gb * 1e9))
    npin = pin_cache.pin_hottest(hist, nslot // 2)
    for s in range(S - a.cache_warmup, S):
        step(pin_cache, s)
    ctx.sync()
    pinned, _ = measured(pin_cache, "pinned hottest + LRU",
                         {"pinned_slots": npin,
                          "pins_from": f"request histogram of the previous {S} steps"})
    pin_cache.free()
    # the 16 layers chained with the hidden state in HBM (k3gc_chain: RMSNorm x post-norm,
    # MoE, residual add per layer), every expert resident: per-token latency of the stack
    slot = (bank.expert_bytes + 65535) // 65536 * 65536
    full = k3moe.Cache(bank, topk=K, budget_bytes=NL * E * slot)
    for l in range(NL):
        for e in range(E):
            full.prefetch(l, e)
    full.reset_stats()
    norms = [k3moe.DevBuf.from_array(k3moe.host_normal(D, a.seed, 950 + l, 1.0, 0.1))
             for l in range(NL)]
    Ls = [lay.dev_tiled for lay in layers]
    chain = {}
    for Tc in (1, T):
        h = k3moe.DevBuf.from_array(layers[0].tokens(Tc, stream_base=2950))
        # the call's argument arrays formed once, as the engine's C caller holds them
        run = full.chain_call(ctx, Ls, [b.ptr for b in norms], 0, h.ptr, Tc)
        for _ in range(2):
            run()
        ctx.sync()
        reps = 10
        t0 = time.perf_counter()
        for _ in range(reps):
            run()
        ctx.sync()
        ms = (time.perf_counter() - t0) * 1e3 / reps
        assert np.isfinite(h.download(np.float32, Tc * D)).all()
        chain[f"T{Tc}"] = {"ms_per_step": round(ms, 3), "ms_per_token": round(ms / Tc, 3),
                           "us_per_layer": round(1e3 * ms / NL, 1)}
    fst = full.stats()
    chain.update({"layers": NL, "all_experts_resident": True,
                  "cache_hit_rate": round(fst.hits / max(fst.requests, 1), 4),
                  "what": "k3gc_chain over the 16 layers, h [T][7168] kept in HBM, one host "
                          "synchronisation per chain call"})
    full.free()
    # the same request stream (each step's unique experts per layer, in first-seen order,
    # as k3gc_moe asks for them) replayed offline at the cache's capacity
    req = []
    for s_ in range(2 * S):
        for l in range(NL):
            seen = []
            for e in idx[s_, l].reshape(-1):
                if int(e) not in seen:
                    seen.append(int(e))
            req.extend((l, e) for e in seen)
    req = np.array(req, np.int32)
    n_req = len(req)
    replays = {p: round(k3moe.replay(p, req, nslot, nslot // 2) / n_req, 4)
               for p in ("lru", "belady", "pinned_lru")}
    res = dict(lru)
    res.update({"layers": NL, "tokens_per_step": T, "steps": S, "warmup": S,
                "hbm_cache_GB": a.cache_gb, "slots": nslot,
                "host_bank_GB": round(NL * E * bank.expert_bytes / 1e9, 1),
                "bank_layers_pinned": bank.pinned_layers,
                "histogram_pinning": pinned,
                "chained_layers": chain,
                "offline_replay_hit_rates": dict(replays, what=f"both segments' {n_req} "
                                                 f"requests from cold at {nslot} slots; "
                                                 f"belady and pinned_lru see the future"),
                "workload": "16 stacked K2 layers, experts in a pinned host bank, HBM cache "
                            "48 GB, batch 8, per-layer Zipf(1.0) routing with 70% step-to-step "
                            "reuse (trace-driven); LRU, then the hottest half of the slots "
                            "pinned from the previous segment's histogram"})
    ctx.destroy()
    bank.free()
    del layers
    return res


def prefill(a):
    """4096-token prefill through the same K2 layer with Zipf(0.8) expert popularity
    (selection-bias skew), experts in the tiled layout in HBM, x resident: router +
    dispatch + grouped bf16 MFMA GEMMs + combine. Reported against the bf16 dense peak."""
    import numpy as np
    import k3moe
    T = a.prefill_tokens
    log(f"bench: prefill {T} tokens, Zipf(0.8) routing skew")
    layer = k3moe.SynthLayer(k3moe.K2_PREFILL, seed=a.seed, layer=0, layout="tiled")
    x = layer.tokens(T, stream_base=900)
    ctx = k3moe.Ctx(layer.dev, max_tokens=T)
    dx = k3moe.DevBuf.from_array(x)
    dout, didx, dwt = k3moe.DevBuf(T * D * 4), k3moe.DevBuf(T * K * 4), k3moe.DevBuf(T * K * 4)

    def run():
        ctx.moe(layer.dev, dx.ptr, T, dout.ptr, didx.ptr, dwt.ptr)

    for _ in range(a.prefill_warmup):
        run()
    ctx.sync()
    idx = didx.download(np.int32, T * K)
    cnt = np.bincount(idx[idx >= 0], minlength=E)
    act = cnt[cnt > 0]
    k3moe.sync()
    t0 = time.perf_counter()
    for _ in range(a.prefill_steps):
        run()
    k3moe.sync()
    t1 = time.perf_counter()
    ctx.sync()
    # per-stage times: HIP events around each stage, in a separate pass so that those
    # events do not sit in the timed region
    nprof = min(a.prefill_steps, 3)
    ctx.profile(True)
    for _ in range(nprof):
        run()
    ctx.sync()
    ms_stage, n_stage = ctx.stage_ms()
    ctx.profile(False)
    out = dout.download(np.float32, T * D)
    assert np.isfinite(out).all()
    # the router's counters over the warmup, timed and profiled calls (bounded bf16
    # logits, then the candidates' fp64 logits): tokens with more candidates than k,
    # candidate logits the any-order bound left open, candidates outside their interval
    extra, opened, violations = ctx.stats()[:3]
    ncalls = a.prefill_warmup + a.prefill_steps + nprof
    # the FP4 x FP8 variant of the routed experts, reported separately
    ctx.set_fp8(True)
    for _ in range(a.prefill_warmup):
        run()
    ctx.sync()
    k3moe.sync()
    f0 = time.perf_counter()
    for _ in range(a.prefill_steps):
        run()
    k3moe.sync()
    f1 = time.perf_counter()
    ctx.sync()
    ctx.profile(True)
    for _ in range(nprof):
        run()
    ctx.sync()
    ms8_stage, n8_stage = ctx.stage_ms()
    ctx.profile(False)
    ctx.set_fp8(False)
    assert np.isfinite(dout.download(np.float32, T * D)).all()
    # the engine's real prefill input: k3_decoder_layer_inc hands k3_moe_prefill the fp32
    # hidden state (src/core/k3_ops.c:1015-1024); the same draws, not rounded to bf16, so x
    # takes two bf16 pieces and the router's second-piece product runs
    x32 = layer.tokens(T, stream_base=900, bf16=False)
    dx32 = k3moe.DevBuf.from_array(x32)

    def run32():
        ctx.moe(layer.dev, dx32.ptr, T, dout.ptr, didx.ptr, dwt.ptr)

    for _ in range(a.prefill_warmup):
        run32()
    ctx.sync()
    idx32 = didx.download(np.int32, T * K)
    k3moe.sync()
    g0 = time.perf_counter()
    for _ in range(a.prefill_steps):
        run32()
    k3moe.sync()
    g1 = time.perf_counter()
    ctx.sync()
    ctx.profile(True)
    for _ in range(nprof):
        run32()
    ctx.sync()
    ms32_stage, n32_stage = ctx.stage_ms()
    ctx.profile(False)
    assert np.isfinite(dout.download(np.float32, T * D)).all()
    del dx32
    ctx.destroy()
    del layer
    ms = (t1 - t0) * 1e3 / a.prefill_steps
    ms8 = (f1 - f0) * 1e3 / a.prefill_steps
    routed, shared, router = prefill_flops(T)
    flops = routed + shared + router
    names = ["router", "dispatch", "routed_gateup", "routed_down", "shared_gateup",
             "shared_down", "combine", "latent", "fused_layer", "activation_pieces"]
    stage_us = {names[s]: round(1e3 * ms_stage[s] / max(n_stage[s], 1), 1)
                for s in range(len(names)) if n_stage[s]}
    gu_us = 1e3 * ms_stage[2] / max(n_stage[2], 1)
    gu_flops = 2 * T * K * 2 * I * D
    gu_tf = gu_flops / (gu_us * 1e-6) / 1e12
    ms32 = (g1 - g0) * 1e3 / a.prefill_steps
    gu32_us = 1e3 * ms32_stage[2] / max(n32_stage[2], 1)
    gu32_tf = gu_flops / (gu32_us * 1e-6) / 1e12
    same = float(np.mean(np.sort(idx32.reshape(T, K), axis=1) == np.sort(idx.reshape(T, K), axis=1)))
    return {
        "tokens": T,
        "ms_per_step": round(ms, 4),
        "tokens_per_s": round(T / (ms * 1e-3), 1),
        "mfma_frac": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
        "algorithmic_flop": flops,
        "achieved_TFLOPs": round(flops / (ms * 1e-3) / 1e12, 1),
        "steps": a.prefill_steps, "warmup": a.prefill_warmup,
        "workload": "4096-token prefill, same K2 layer, Zipf(0.8) selection-bias skew "
                    "(alpha 0.02), bf16-valued x; bf16 MFMA grouped GEMMs, h's MXFP8 "
                    "remainder on scaled FP8 MFMA",
        "routing": {"experts_used": int(len(act)), "max_tokens": int(cnt.max()),
                    "min_tokens": int(act.min()),
                    "p90_over_p10": round(float(np.percentile(act, 90) / max(np.percentile(act, 10), 1)), 2),
                    "tokens_with_extra_candidates_per_call": round(extra / ncalls, 1),
                    "open_candidate_logits_per_call": round(opened / ncalls, 1),
                    "bound_violations": int(violations)},
        "stage_us": stage_us,
        "fp4xfp8_variant": {
            "ms_per_step": round(ms8, 4), "tokens_per_s": round(T / (ms8 * 1e-3), 1),
            "frac_of_bf16_peak": round(flops / (ms8 * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "frac_of_fp8_peak": round(flops / (ms8 * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4),
            "routed_gateup_us": round(1e3 * ms8_stage[2] / max(n8_stage[2], 1), 1),
            "routed_down_us": round(1e3 * ms8_stage[3] / max(n8_stage[3], 1), 1),
            "routed_gateup_frac_of_fp8_peak": round(
                gu_flops / (1e-3 * ms8_stage[2] / max(n8_stage[2], 1)) / 1e12 / FP8_PEAK_TFLOPS, 4),
            "what": "routed experts on v_mfma_scale_f32_16x16x128_f8f6f4: MXFP4 weights as "
                    "stored, x and h quantised to MXFP8 (E4M3, E8M0 per 32); shared expert "
                    "bf16; rel-L2 vs the unquantised engine ~5e-2 (tests)"},
        "fp32_x": {
            "ms_per_step": round(ms32, 4), "tokens_per_s": round(T / (ms32 * 1e-3), 1),
            "mfma_frac": round(flops / (ms32 * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "achieved_TFLOPs": round(flops / (ms32 * 1e-3) / 1e12, 1),
            "stage_us": {names[s]: round(1e3 * ms32_stage[s] / max(n32_stage[s], 1), 1)
                         for s in range(len(names)) if n32_stage[s]},
            "routing_slots_same_as_bf16_x": round(same, 4),
            "what": "the same 4096 tokens as fp32 values (the engine's k3_decoder_layer_inc "
                    "input, not rounded to bf16): x is two bf16 pieces, so the router adds "
                    "the second piece's product and the routed and shared gate/up GEMMs "
                    "multiply both pieces (8-wave workgroups); same layer, same Zipf(0.8) "
                    "skew",
            "roofline": {"kernel": "k_gemm<0, 8> routed gate/up on x's two bf16 pieces "
                                   "(8-wave workgroups)",
                         "bound": "mfma", "achieved": round(gu32_tf, 1),
                         "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(gu32_tf / BF16_PEAK_TFLOPS, 4),
                         "traffic": TRAFFIC_GATEUP_PREFILL_FP32,
                         "flop_per_launch": gu_flops, "avg_launch_us": round(gu32_us, 1)}},
        "roofline": {"kernel": "k_gemm<0> routed gate/up (MXFP4 dequantised to bf16 in "
                               "registers, bf16 MFMA, SwiGLU epilogue)",
                     "bound": "mfma", "achieved": round(gu_tf, 1), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(gu_tf / BF16_PEAK_TFLOPS, 4),
                     "traffic": TRAFFIC_GATEUP_PREFILL, "flop_per_launch": gu_flops,
                     "avg_launch_us": round(gu_us, 1)},
    }


def dropin(a):
    """The engine's own entry point k3_moe on the c1 workload: host x and out (the PCIe
    round trip of 28 KB each way is inside the measured time), router/shared weights from
    host pointers mirrored in HBM once, experts from an HBM expert cache (tiled bank)
    holding all of the --layers layers' experts: per call the router, the engine's
    getmany + get per slot, then the fused decode kernel with the routing given. Then
    64-token calls (the grouped GEMMs) on the Zipf(1.1) batch workload."""
    import ctypes as C
    import numpy as np
    import k3moe
    NL = a.layers
    log(f"bench: drop-in k3_moe, {NL} K2 layers with every expert in a tiled HBM cache")
    L = k3moe.lib()

    def build(shape, nl, base_layer=0):
        bank = k3moe.Bank(nl, E, D, I, k3moe.K3G_EXPERT_MXFP4_TILED)
        layers = []
        for l in range(nl):
            lay = k3moe.SynthLayer(shape, seed=a.seed, layer=l, layout="tiled")
            bank.fill_from_layer(lay, l)
            lay.release_experts()
            layers.append(lay)
        slot = (bank.expert_bytes + 65535) // 65536 * 65536
        cache = k3moe.Cache(bank, topk=K, budget_bytes=nl * E * slot)
        for l in range(nl):
            for e in range(E):
                cache.prefetch(l, e)
        cache.reset_stats()
        ws = []
        for lay in layers:
            w = k3moe.K3MoeW()
            w.gate, w.bias = lay.gate.ctypes.data, lay.bias.ctypes.data
            w.sh1, w.sh3, w.sh2 = lay.sh1.ctypes.data, lay.sh3.ctypes.data, lay.sh2.ctypes.data
            w.wdt = k3moe.K3_WBF16
            w.src, w.layer = cache.src_ptr, lay.layer
            ws.append(w)
        return bank, cache, layers, ws

    def timed(ws, cfg, xs, T, warm, steps, fn):
        n = warm + steps
        # every call's output kept for the check below; filled (NaN) beforehand so its
        # pages are mapped, as the engine's reused output buffer is: a fresh page's first
        # write is a page fault (7 per token here) that the engine never pays
        out = np.full((n * T, D), np.nan, np.float32)
        idx = np.zeros(K, np.int32)
        wt = np.zeros(K, np.float32)

        # the call's pointers formed before the timed loop: the engine calls k3_moe from C,
        # so per-call Python work (slicing, ctypes conversions) is not part of the leg
        optr, xptr = out.ctypes.data, xs.ctypes.data
        wrefs = [C.byref(w) for w in ws]
        cref, iptr, wptr = C.byref(cfg), C.c_void_p(idx.ctypes.data), C.c_void_p(wt.ctypes.data)
        ob, xb = T * D * 4, T * xs.shape[1] * 4
        args = [(C.c_void_p(optr + i * ob), C.c_void_p(xptr + i * xb), wrefs[i % len(ws)])
                for i in range(n)]

        def call(i):
            o, xq, w = args[i]
            fn(o, xq, w, cref, T, iptr, wptr, None)

        for i in range(warm):
            call(i)
        t0 = time.perf_counter()
        for i in range(warm, n):
            call(i)
        dt = time.perf_counter() - t0
        assert np.isfinite(out).all()
        return dt / steps, L.k3moe_last_kernels()

    bank, cache, layers, ws = build(k3moe.K2, NL)
    cfg = layers[0].cfg()
    xs = np.ascontiguousarray(layers[0].tokens(a.warmup + a.steps, stream_base=900))
    d0 = C.c_long.in_dll(L, "k3_expert_drops").value
    sec, kern = timed(ws, cfg, xs, 1, a.warmup, a.steps, L.k3_moe)
    st = cache.stats()
    assert C.c_long.in_dll(L, "k3_expert_drops").value == d0
    res = {"us_per_token": round(1e6 * sec, 2), "tokens_per_s": round(1.0 / sec, 1),
           "hbm_GBps": round((K * B_EXPERT + B_SHARED + B_ROUTER + B_TOKEN) / sec / 1e9, 1),
           "kernels": {1: "staged", 2: "fused decode kernel",
                       4: "grouped GEMMs"}.get(kern, str(kern)),
           "steps": a.steps, "warmup": a.warmup, "cache_hit_rate": round(st.hits / max(st.requests, 1), 4),
           "workload": "k3_moe (host x/out, host weight pointers, K3ExpertSrc = HBM expert "
                       "cache with every expert of %d K2 layers resident), 1 token per call, "
                       "layers round-robin" % NL}
    cache.free()
    bank.free()
    del layers, ws
    if a.batch_tokens > 0:
        T = a.batch_tokens
        bank, cache, layers, ws = build(k3moe.K2_BATCH, 2)
        cfg = layers[0].cfg()
        xs = np.ascontiguousarray(layers[0].tokens(T * (a.batch_warmup + a.batch_steps),
                                                   stream_base=1900))
        sec, kern = timed(ws, cfg, xs, T, a.batch_warmup, a.batch_steps, L.k3_moe)
        res["batch"] = {"tokens": T, "ms_per_step": round(1e3 * sec, 3),
                        "us_per_token": round(1e6 * sec / T, 2),
                        "kernels": {4: "grouped GEMMs"}.get(kern, str(kern)),
                        "workload": f"k3_moe on {T} tokens per call, Zipf(1.1) batch layers, "
                                    f"experts resident in the HBM cache"}
        cache.free()
        bank.free()
        del layers, ws
    return res


def k3_shape(a):
    """The real Kimi-K3 LatentMoE layer on the device API: d 7168, 896 MXFP4 experts top-16
    at latent 3584 x I 3072, bf16 latent down/up projections, RMSNorm of the aggregate, two
    shared experts fused (6144), SiTU(4, 25), routed scale 1.0; synthetic seeded weights.
    Decode (1 token, 2 layers round-robin) on the fused decode kernel and a
    --k3-prefill-tokens prefill on the grouped matrix-core GEMMs."""
    import ctypes as C
    import numpy as np
    import k3moe
    d, E3, k3, Lw, I3, SI3 = 7168, 896, 16, 3584, 3072, 6144
    log(f"bench: K3 LatentMoE layer (E={E3}, top-{k3}, latent {Lw}, I={I3}, shared {SI3})")
    lib = k3moe.lib()
    shape = k3moe.Shape("K3 latent experts", Lw, E3, k3, I3, n_shared=2, routed_scale=1.0,
                        x_bf16=False)
    keep = []

    def tiled_bf16(v, rows, cols):
        src = k3moe.DevBuf.from_array(k3moe.bf16_bits(v))
        t = k3moe.DevBuf(lib.k3g_tiled_bf16_bytes(rows, cols))
        k3moe._check(lib.k3g_tile_bf16(C.c_void_p(t.ptr), C.c_void_p(src.ptr), rows, cols, None),
                     "k3g_tile_bf16")
        k3moe.sync()
        keep.append(t)
        return t.ptr

    def layer(l):
        ex = k3moe.SynthLayer(shape, seed=a.seed, layer=l, layout="tiled")
        keep.append(ex)
        n = lambda cnt, s, m, sd, bf=False: k3moe.host_normal(cnt, a.seed, 700 + 20 * l + s, m, sd, bf16=bf)  # noqa: E731
        g = k3moe.DevBuf.from_array(n(E3 * d, 1, 0.0, 0.02))
        b = k3moe.DevBuf.from_array(n(E3, 2, 0.0, 0.01))
        ln = k3moe.DevBuf.from_array(n(Lw, 3, 1.0, 0.1))
        keep.extend([g, b, ln])
        Lk = k3moe.K3gLayer()
        Lk.hidden, Lk.n_experts, Lk.topk, Lk.inter = d, E3, k3, I3
        Lk.shared_inter, Lk.latent = SI3, Lw
        Lk.renorm, Lk.routed_scale, Lk.act_b1, Lk.act_b2, Lk.rms_eps = 1, 1.0, 4.0, 25.0, 1e-6
        Lk.gate, Lk.bias, Lk.latent_norm = g.ptr, b.ptr, ln.ptr
        Lk.expert_fmt, Lk.experts = k3moe.K3G_EXPERT_MXFP4_TILED, ex.d_ttable.ptr
        Lk.wdt, Lk.shared_fmt = k3moe.K3_WBF16, 1
        Lk.down = tiled_bf16(n(Lw * d, 4, 0.0, 0.02, True), Lw, d)
        Lk.up = tiled_bf16(n(d * Lw, 5, 0.0, 0.02, True), d, Lw)
        Lk.sh1 = tiled_bf16(n(SI3 * d, 6, 0.0, 0.02, True), SI3, d)
        Lk.sh3 = tiled_bf16(n(SI3 * d, 7, 0.0, 0.02, True), SI3, d)
        Lk.sh2 = tiled_bf16(n(d * SI3, 8, 0.0, 0.02, True), d, SI3)
        return Lk

    Ls = [layer(0), layer(1)]
    Tp = a.k3_prefill_tokens
    ctx = k3moe.Ctx(Ls[0], max_tokens=max(Tp, 1))
    n = a.warmup + a.steps
    xs = k3moe.host_normal(max(n, Tp) * d, a.seed, 790, 0.0, 1.0).reshape(-1, d)
    dx = k3moe.DevBuf.from_array(xs)
    dout = k3moe.DevBuf(max(n, Tp) * d * 4)
    didx, dwt = k3moe.DevBuf(max(n, Tp) * k3 * 4), k3moe.DevBuf(max(n, Tp) * k3 * 4)

    def step(i):
        ctx.moe(Ls[i % 2], dx.ptr + i * d * 4, 1, dout.ptr + i * d * 4, didx.ptr + i * k3 * 4,
                dwt.ptr + i * k3 * 4)

    for i in range(a.warmup):
        step(i)
    ctx.sync()
    tm = k3moe.Timer(ctx.stream)
    tm.start()
    for i in range(a.warmup, n):
        step(i)
    us = 1e3 * tm.stop() / a.steps
    ctx.sync()
    assert np.isfinite(dout.download(np.float32, n * d)).all()
    B_e3 = 3 * I3 * Lw * 17 // 32
    dense = 6 * SI3 * d + 4 * E3 * d + 4 * E3 + 2 * 2 * Lw * d + d * 8
    tok_bytes = k3 * B_e3 + dense
    res = {"decode": {"us_per_token": round(us, 2), "bytes_per_token": tok_bytes,
                      "hbm_GBps": round(tok_bytes / (us * 1e-6) / 1e9, 1),
                      "hbm_frac": round(tok_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                      "steps": a.steps,
                      "kernels": "fused decode kernel: router, top-k, latent down, routed "
                                 "experts on z, aggregate + RMSNorm, latent up, shared"}}
    if Tp > 0:
        def run():
            ctx.moe(Ls[0], dx.ptr, Tp, dout.ptr, didx.ptr, dwt.ptr)
        run()
        ctx.sync()
        tm.start()
        for _ in range(a.prefill_steps):
            run()
        ms = tm.stop() / a.prefill_steps
        ctx.sync()
        assert np.isfinite(dout.download(np.float32, Tp * d)).all()
        flops = (2 * Tp * k3 * 3 * I3 * Lw + 6 * Tp * SI3 * d + 2 * 2 * Tp * Lw * d +
                 2 * Tp * E3 * d)
        res["prefill"] = {"tokens": Tp, "ms_per_step": round(ms, 3),
                          "tokens_per_s": round(Tp / (ms * 1e-3), 1), "algorithmic_flop": flops,
                          "achieved_TFLOPs": round(flops / (ms * 1e-3) / 1e12, 1),
                          "mfma_frac": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                          "steps": a.prefill_steps}
    res["workload"] = ("Kimi-K3 LatentMoE layer: d 7168, 896 MXFP4 experts top-16, latent "
                       "3584, I 3072, bf16 latent down/up, latent RMSNorm, 2 shared experts "
                       "(6144), SiTU(4,25); x N(0,1) fp32; decode 2 layers round-robin")
    ctx.destroy()
    del Ls, keep
    return res


def decode(a):
    """The headline: 1-token decode through the fused decode kernel, --layers K2 layers
    round-robin. Returns the JSON line's fields."""
    import numpy as np
    import k3moe
    log(f"bench: building {a.layers} K2 layers (d={D}, E={E}, top-{K}, I={I}) in HBM")
    layers = [k3moe.SynthLayer(k3moe.K2, seed=a.seed, layer=l, layout="tiled")
              for l in range(a.layers)]
    n_tok = a.warmup + a.steps
    xs = layers[0].tokens(n_tok, stream_base=900)
    ctx = k3moe.Ctx(layers[0].dev, max_tokens=1)
    dx = k3moe.DevBuf.from_array(xs)
    dout = k3moe.DevBuf(n_tok * D * 4)
    didx = k3moe.DevBuf(n_tok * K * 4)
    dwt = k3moe.DevBuf(n_tok * K * 4)

    def step(i):
        ctx.moe(layers[i % a.layers].dev, dx.ptr + i * D * 4, 1, dout.ptr + i * D * 4,
                didx.ptr + i * K * 4, dwt.ptr + i * K * 4)

    log(f"bench: warmup {a.warmup} steps")
    for i in range(a.warmup):
        step(i)
    ctx.sync()
    log(f"bench: timing {a.steps} steps")
    # HIP events bracket the timed region on the context's stream (every step is one
    # launch of the fused layer kernel, back to back)
    region = k3moe.Timer(ctx.stream)
    k3moe.sync()
    t0 = time.perf_counter()
    region.start()
    for i in range(a.warmup, n_tok):
        step(i)
    region_ms = region.stop()
    k3moe.sync()
    t1 = time.perf_counter()
    ctx.sync()
    # per-stage times: HIP events around each stage on the context's stream, in a separate
    # pass over the same steps so those events do not sit in the timed region
    ctx.profile(True)
    for i in range(a.warmup, n_tok):
        step(i)
    ctx.sync()
    ms_stage, n_stage = ctx.stage_ms()
    ctx.profile(False)
    out = dout.download(np.float32, n_tok * D)
    assert np.isfinite(out).all()

    ms_step = (t1 - t0) * 1e3 / a.steps
    us_tok = ms_step * 1e3
    layer_bytes = K * B_EXPERT + B_SHARED + B_ROUTER + B_TOKEN
    names = ["router", "dispatch", "routed_gateup", "routed_down", "shared_gateup",
             "shared_down", "combine", "latent", "fused_layer"]
    stage_us = {names[s]: round(1e3 * ms_stage[s] / max(n_stage[s], 1), 2)
                for s in range(len(names)) if n_stage[s]}
    if n_stage[8]:
        kern = "k_decode_fused (whole layer: router, top-k, shared + routed MXFP4 GEMVs, combine)"
        k_us = 1e3 * region_ms / a.steps
        k_bytes = layer_bytes
        traffic = TRAFFIC_FUSED
    else:
        kern = "k_routed_gateup (MXFP4 gate+up GEMV, SwiGLU epilogue)"
        k_us = 1e3 * ms_stage[2] / max(n_stage[2], 1)
        k_bytes = K * B_GATEUP_EXPERT
        traffic = None
    achieved = k_bytes / (k_us * 1e-6) / 1e9
    res = {
        "metric": METRIC,
        "value": round(1e6 / us_tok, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "1-token decode, one Kimi-K2-scale MoE layer: d=7168, 384 "
                               "MXFP4 routed experts top-8 (I=2048, SwiGLU), 1 bf16 shared "
                               "expert, fp32 router; %d layers round-robin" % a.layers,
                   "tokens_per_step": 1, "layers": a.layers, "seed": a.seed},
        "us_per_token": round(us_tok, 2),
        "hbm_GBps": round(layer_bytes / (us_tok * 1e-6) / 1e9, 1),
        "hbm_frac": round(layer_bytes / (us_tok * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "bytes_per_token": layer_bytes,
        "stage_us": stage_us,
        "roofline": {"kernel": kern, "bound": "hbm", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "bytes_per_launch": k_bytes,
                     "avg_launch_us": round(k_us, 2)},
    }
    ctx.destroy()
    del layers, dx, dout, didx, dwt
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--seed", type=int, default=2024)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-tokens", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--batch-tokens", type=int, default=64,
                    help="tokens of the batched-decode measurement (0: skip it)")
    ap.add_argument("--batch-steps", type=int, default=20)
    ap.add_argument("--batch-warmup", type=int, default=4)
    ap.add_argument("--prefill-tokens", type=int, default=4096,
                    help="tokens of the prefill measurement (0: skip it)")
    ap.add_argument("--prefill-steps", type=int, default=5)
    ap.add_argument("--prefill-warmup", type=int, default=2)
    ap.add_argument("--cache-layers", type=int, default=16,
                    help="layers of the streamed-decode measurement (0: skip it)")
    ap.add_argument("--cache-gb", type=float, default=48.0)
    ap.add_argument("--cache-tokens", type=int, default=8)
    ap.add_argument("--cache-steps", type=int, default=12)
    ap.add_argument("--cache-warmup", type=int, default=6)
    ap.add_argument("--legs", default="decode,batch,prefill,stream,dropin,k3,cpu",
                    help="comma list of the measurements to run (decode is the headline)")
    ap.add_argument("--k3-prefill-tokens", type=int, default=4096)
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run one 256 MiB device-to-device copy (a counter calibration "
                         "point for rocprofv3 --pmc runs), outside the timed region")
    a = ap.parse_args()
    legs = set(a.legs.split(","))
    if a.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {a.gpus} is not supported (the layer runs "
              f"on a single MI355X; sharding across GPUs is design-only)",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import __graft_entry__ as g
    g._ensure_built()
    import k3moe

    if a.calib_copy:
        n = 256 << 20
        src, dst = k3moe.DevBuf(n), k3moe.DevBuf(n)
        k3moe._check(k3moe.hip().hipMemcpy(k3moe.C.c_void_p(dst.ptr), k3moe.C.c_void_p(src.ptr),
                                           n, k3moe.D2D), "calibration copy")
        k3moe.sync()
        del src, dst
    if "decode" in legs:
        res = decode(a)
    else:
        res = {"metric": METRIC, "value": None, "unit": "tokens/s", "n_gpus": 1,
               "steps": 0, "warmup": 0, "ms_per_step": None, "higher_is_better": True,
               "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
               "config": {"workload": "decode leg skipped (--legs)"}}
    if a.batch_tokens > 0 and "batch" in legs:
        res["batch_decode"] = batch_decode(a)
    if a.prefill_tokens > 0 and "prefill" in legs:
        res["prefill"] = prefill(a)
    if "dropin" in legs:
        res["dropin_decode"] = dropin(a)
    if "k3" in legs:
        res["k3_latent_moe"] = k3_shape(a)
    if a.cache_layers > 0 and "stream" in legs:
        res["streamed_decode"] = streamed_decode(a)
    if not a.no_cpu and "cpu" in legs:
        log("bench: CPU baseline")
        res["cpu_baseline"] = cpu_baseline(a.cpu_seconds, a.cpu_tokens, a.seed)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
