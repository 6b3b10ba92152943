"""ctypes wrapper of the CPU oracle (liboracle.so, the C restatement) and of the
engine's own compiled kernels (_ref/libk3ref.so, built from the reference sources when
they are present).

TEST INFRASTRUCTURE: only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg
use this module, and only as the reference of a test or the CPU baseline, never as the
product.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libk3ref.so")

sys.path.insert(0, os.path.join(os.path.dirname(HERE), "kimi-k3-in-rust_amd"))
import k3moe  # noqa: E402  (struct layouts shared with the product binding)

vp, i32, f32 = C.c_void_p, C.c_int, C.c_float


def build(quiet: bool = True) -> None:
    """make -C oracle (liboracle.so, and _ref when the reference sources exist)."""
    r = subprocess.run(["make", "-C", HERE], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + r.stdout + r.stderr)
    if not quiet:
        print(r.stdout)


class OrMemSrc(C.Structure):
    _fields_ = [("src", k3moe.K3ExpertSrc), ("bases", C.POINTER(C.c_void_p)),
                ("p1_off", C.c_int64), ("s1_off", C.c_int64), ("p2_off", C.c_int64),
                ("s2_off", C.c_int64), ("p3_off", C.c_int64), ("s3_off", C.c_int64),
                ("n_layers", C.c_int), ("n_experts", C.c_int),
                ("gets", C.c_int64), ("getmanys", C.c_int64), ("residents", C.c_int64)]


class OrKernels(C.Structure):
    _fields_ = [("router", vp), ("matmul_mxfp4", vp), ("matmul_bf16", vp), ("matmul", vp),
                ("situ_glu", vp), ("rmsnorm", vp), ("matmul_q8", vp)]


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(vp)


class Kernels:
    """One set of kernels with the engine's signatures: the restatement (prefix ork3_)
    or the engine's compiled code (prefix k3_)."""

    def __init__(self, path: str, prefix: str):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.path, self.prefix = path, prefix
        L = C.CDLL(path)
        self.L = L
        g = lambda n: getattr(L, prefix + n)  # noqa: E731
        self.f_router = g("router")
        self.f_router.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, f32]
        self.f_mx = g("matmul_mxfp4")
        self.f_mx.argtypes = [vp, vp, vp, vp, i32, i32, i32]
        self.f_deq = g("mxfp4_dequant")
        self.f_deq.argtypes = [vp, vp, vp, i32, i32, i32]
        self.f_bf16 = g("matmul_bf16")
        self.f_bf16.argtypes = [vp, vp, vp, i32, i32]
        self.f_mm = g("matmul")
        self.f_mm.argtypes = [vp, vp, vp, i32, i32]
        self.f_q8 = g("matmul_q8")
        self.f_q8.argtypes = [vp, vp, vp, i32, i32]
        self.f_situ = g("situ_glu")
        self.f_situ.argtypes = [vp, vp, i32, f32, f32]
        self.f_rms = g("rmsnorm")
        self.f_rms.argtypes = [vp, vp, vp, i32, f32]
        self.f_moe = g("moe")
        self.f_moe.argtypes = [vp, vp, C.POINTER(k3moe.K3MoeW), C.POINTER(k3moe.K3Cfg), i32,
                               vp, vp, vp]
        self.f_moe_prefill = g("moe_prefill")
        self.f_moe_prefill.argtypes = self.f_moe.argtypes
        self.f_scratch = g("moe_scratch")
        self.f_scratch.argtypes = [C.POINTER(k3moe.K3Cfg)]
        self.f_scratch.restype = C.c_size_t
        self.drops = C.c_long.in_dll(L, prefix + "expert_drops")

    def addr(self, f) -> int:
        return C.cast(f, vp).value

    # -- kernels ---------------------------------------------------------------------
    def router(self, x, W, bias, E, k, renorm=1, scale=1.0):
        x = np.ascontiguousarray(x, np.float32)
        idx = np.zeros(k, np.int32)
        w = np.zeros(k, np.float32)
        self.f_router(_p(idx), _p(w), _p(x), _p(np.ascontiguousarray(W, np.float32)),
                      _p(None if bias is None else np.ascontiguousarray(bias, np.float32)),
                      x.size, E, k, renorm, scale)
        return idx, w

    def matmul_mxfp4(self, x, packed, scales, rows, group=32):
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(rows, np.float32)
        self.f_mx(_p(y), _p(x), _p(np.ascontiguousarray(packed, np.uint8)),
                  _p(np.ascontiguousarray(scales, np.uint8)), x.size, rows, group)
        return y

    def dequant(self, packed, scales, rows, pcols, group=32):
        out = np.zeros(rows * pcols * 2, np.float32)
        self.f_deq(_p(out), _p(np.ascontiguousarray(packed, np.uint8)),
                   _p(np.ascontiguousarray(scales, np.uint8)), rows, pcols, group)
        return out.reshape(rows, pcols * 2)

    def matmul_bf16(self, x, Wbits, out_rows):
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(out_rows, np.float32)
        self.f_bf16(_p(y), _p(x), _p(np.ascontiguousarray(Wbits, np.uint16)), x.size, out_rows)
        return y

    def matmul(self, x, W, out_rows):
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(out_rows, np.float32)
        self.f_mm(_p(y), _p(x), _p(np.ascontiguousarray(W, np.float32)), x.size, out_rows)
        return y

    def matmul_q8(self, x, Wrows, out_rows):
        """Wrows: uint8 [out_rows][4 + in], each row an f32 scale then int8 weights."""
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(out_rows, np.float32)
        self.f_q8(_p(y), _p(x), _p(np.ascontiguousarray(Wrows, np.uint8)), x.size, out_rows)
        return y

    def situ(self, gu, b1, b2):
        gu = np.ascontiguousarray(gu, np.float32)
        n = gu.size // 2
        y = np.zeros(n, np.float32)
        self.f_situ(_p(y), _p(gu), n, b1, b2)
        return y

    def moe(self, w: k3moe.K3MoeW, cfg: k3moe.K3Cfg, x: np.ndarray, prefill=False):
        x = np.ascontiguousarray(x, np.float32)
        T = x.shape[0]
        out = np.zeros_like(x)
        idx = np.zeros(cfg.topk, np.int32)
        wt = np.zeros(cfg.topk, np.float32)
        sc = np.zeros(self.f_scratch(C.byref(cfg)) + 2 * cfg.moe_inter * cfg.n_shared + 16,
                      np.float32)
        f = self.f_moe_prefill if prefill else self.f_moe
        f(_p(out), _p(x), C.byref(w), C.byref(cfg), T, _p(idx), _p(wt), _p(sc))
        return out, idx, wt


_oracle = None
_ref = None


def oracle() -> Kernels:
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_SO):
            build()
        _oracle = Kernels(ORACLE_SO, "ork3_")
        L = _oracle.L
        L.ork3_set_kernels.argtypes = [C.POINTER(OrKernels)]
        L.ork3_memsrc_init.argtypes = [C.POINTER(OrMemSrc), C.POINTER(C.c_void_p), i32, i32,
                                       C.POINTER(C.c_int64)]
        L.ork3_lru_hits.argtypes = [vp, C.c_int64, C.c_int64, C.c_int64]
        L.ork3_lru_hits.restype = C.c_int64
        L.ork3_quant_mxfp8.argtypes = [vp, i32]
        L.ork3_kat_fillf.argtypes = [vp, C.c_size_t, C.c_uint]
        L.ork3_kat_fillb.argtypes = [vp, C.c_size_t, C.c_uint]
        L.ork3_kat_fillbf16.argtypes = [vp, C.c_size_t, C.c_uint]
        L.ork3_fnv1a.argtypes = [vp, i32]
        L.ork3_fnv1a.restype = C.c_ulonglong
    return _oracle


def ref() -> Kernels | None:
    """The engine's compiled kernels, or None when _ref was not built (no reference
    sources on this machine and no prebuilt library carried over)."""
    global _ref
    if _ref is None and os.path.exists(REF_SO):
        _ref = Kernels(REF_SO, "k3_")
    return _ref


def set_kernels(k: Kernels | None) -> None:
    """Make ork3_moe compose kernel set k (None: the restatement)."""
    O = oracle()
    if k is None:
        O.L.ork3_set_kernels(None)
        return
    t = OrKernels(k.addr(k.f_router), k.addr(k.f_mx), k.addr(k.f_bf16), k.addr(k.f_mm),
                  k.addr(k.f_situ), k.addr(k.f_rms), k.addr(k.f_q8))
    O.L.ork3_set_kernels(C.byref(t))


class MemSrc:
    """An OrMemSrc over host expert runs {(layer, expert): uint8 array}."""

    def __init__(self, runs: dict, n_layers: int, n_experts: int, geo):
        self.runs = runs
        self.bases = (C.c_void_p * (n_layers * n_experts))()
        for (l, e), a in runs.items():
            self.bases[l * n_experts + e] = a.ctypes.data
        offs = (C.c_int64 * 6)(geo.p1_off, geo.s1_off, geo.p2_off, geo.s2_off, geo.p3_off,
                               geo.s3_off)
        self.s = OrMemSrc()
        oracle().L.ork3_memsrc_init(C.byref(self.s), self.bases, n_layers, n_experts, offs)

    @property
    def ptr(self) -> int:
        return C.addressof(self.s)


def lru_hits(keys: np.ndarray, nkeys: int, capacity: int) -> int:
    keys = np.ascontiguousarray(keys, np.int32)
    return int(oracle().L.ork3_lru_hits(_p(keys), keys.size, nkeys, capacity))


def kat_f(n: int, seed: int) -> np.ndarray:
    a = np.empty(n, np.float32)
    oracle().L.ork3_kat_fillf(_p(a), n, seed)
    return a


def kat_b(n: int, seed: int) -> np.ndarray:
    a = np.empty(n, np.uint8)
    oracle().L.ork3_kat_fillb(_p(a), n, seed)
    return a


def kat_bf16(n: int, seed: int) -> np.ndarray:
    a = np.empty(n, np.uint16)
    oracle().L.ork3_kat_fillbf16(_p(a), n, seed)
    return a


def fnv1a(v: np.ndarray) -> str:
    v = np.ascontiguousarray(v, np.float32)
    return "%016x" % oracle().L.ork3_fnv1a(_p(v), v.size)


def quant_mxfp8(x: np.ndarray) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True)
    oracle().L.ork3_quant_mxfp8(_p(y), y.size)
    return y


# ------------------------------------------------------------ K2-shaped layers ----

def routed_union(layer: "k3moe.SynthLayer", x: np.ndarray, k: Kernels | None = None) -> list:
    """Experts the engine's router picks for any of the tokens (runs the router)."""
    k = k or oracle()
    s = layer.shape
    seen = []
    for t in range(x.shape[0]):
        idx, _ = k.router(x[t], layer.gate, layer.bias, s.n_experts, s.topk, s.renorm,
                          s.routed_scale)
        for e in idx:
            if int(e) not in seen:
                seen.append(int(e))
    return seen


def k2_weights(layer: "k3moe.SynthLayer", experts: list, identity: bool = False):
    """K3MoeW + K3Cfg for a synthetic K2 layer, the routed experts regenerated on the
    host and served by an in-memory source. identity=True expresses the layer the way
    the engine must (bf16 identity latent matrices) instead of with down = up = NULL."""
    s = layer.shape
    runs = {(layer.layer, e): layer.expert_host(e) for e in experts}
    src = MemSrc(runs, layer.layer + 1, s.n_experts, layer.geo)
    w = k3moe.K3MoeW()
    keep = [runs, src]
    w.gate = layer.gate.ctypes.data
    w.bias = layer.bias.ctypes.data
    if layer.SI:
        w.sh1, w.sh3, w.sh2 = layer.sh1.ctypes.data, layer.sh3.ctypes.data, layer.sh2.ctypes.data
    w.wdt = k3moe.K3_WBF16
    if identity:
        eye = np.zeros((s.hidden, s.hidden), np.uint16)
        eye[np.arange(s.hidden), np.arange(s.hidden)] = 0x3F80
        keep.append(eye)
        w.down = w.up = eye.ctypes.data
    w.src = src.ptr
    w.layer = layer.layer
    cfg = layer.cfg()
    return w, cfg, keep


def k2_forward(layer: "k3moe.SynthLayer", x: np.ndarray, k: Kernels | None = None,
               prefill: bool = False, identity: bool = False):
    """Oracle output of the synthetic layer for tokens x [T][hidden]."""
    k = k or oracle()
    experts = routed_union(layer, x, k)
    w, cfg, keep = k2_weights(layer, experts, identity)
    out, idx, wt = k.moe(w, cfg, x, prefill=prefill)
    del keep
    return out, idx, wt


def k2_forward_mxfp8(layer: "k3moe.SynthLayer", x: np.ndarray):
    """Quantisation-aware oracle of the FP4 x FP8 variant: the engine's layer with the
    routed experts' inputs quantised to MXFP8 (OCP MX, 32-element blocks) -- x before
    gate/up, the activation h before down -- and everything else the engine's own
    arithmetic (router, exact MXFP4 GEMVs in double, SwiGLU, slot-ordered combine, the
    bf16 shared expert unquantised)."""
    k = oracle()
    s = layer.shape
    d, I, E = s.hidden, s.inter, s.n_experts
    g = layer.geo
    cap = float(2.0 ** 100)
    runs = {}
    out = np.zeros((x.shape[0], d), np.float32)
    for t in range(x.shape[0]):
        xt = np.ascontiguousarray(x[t], np.float32)
        idx, w = k.router(xt, layer.gate, layer.bias, E, s.topk, s.renorm, s.routed_scale)
        xq = quant_mxfp8(xt)
        acc = np.zeros(d, np.float32)
        for j in range(s.topk):
            e = int(idx[j])
            if e not in runs:
                runs[e] = layer.expert_host(e)
            r = runs[e]
            p1 = r[g.p1_off:g.s1_off]; s1 = r[g.s1_off:g.p2_off]
            p2 = r[g.p2_off:g.s2_off]; s2 = r[g.s2_off:g.p3_off]
            p3 = r[g.p3_off:g.s3_off]; s3 = r[g.s3_off:g.nbytes]
            gu = np.concatenate([k.matmul_mxfp4(xq, p1, s1, I), k.matmul_mxfp4(xq, p3, s3, I)])
            h = quant_mxfp8(k.situ(gu.astype(np.float32), cap, cap))
            y = k.matmul_mxfp4(h, p2, s2, d)
            acc = (acc + np.float32(w[j]) * y.astype(np.float32)).astype(np.float32)
        if layer.SI:
            SI = layer.SI
            gu = np.concatenate([k.matmul_bf16(xt, layer.sh1, SI), k.matmul_bf16(xt, layer.sh3, SI)])
            hs = k.situ(gu.astype(np.float32), cap, cap)
            acc = (acc + k.matmul_bf16(hs, layer.sh2, d).astype(np.float32)).astype(np.float32)
        out[t] = acc
    return out


# --------------------------------------------------- cache policies (offline replays) ----
# The engine's tools/sim_cache.py, restated for small traces (pure Python): the product's
# k3gc_replay_* must give the same hits. keys: any hashable request keys in trace order.

def sim_lru(keys, cap):
    """tools/sim_cache.py:36-49"""
    from collections import OrderedDict
    seen, hits = OrderedDict(), 0
    for k in keys:
        if k in seen:
            seen.move_to_end(k)
            hits += 1
        else:
            if len(seen) >= cap:
                seen.popitem(last=False)
            seen[k] = 1
    return hits


def sim_belady(keys, cap):
    """tools/sim_cache.py:52-76: evict the resident key used furthest in the future; a
    request used later than every resident key is not cached."""
    n = len(keys)
    nxt, last = [n] * n, {}
    for i in range(n - 1, -1, -1):
        nxt[i] = last.get(keys[i], n)
        last[keys[i]] = i
    resident, hits = {}, 0
    for i, k in enumerate(keys):
        if k in resident:
            hits += 1
            resident[k] = nxt[i]
            continue
        if len(resident) >= cap:
            victim = max(resident, key=resident.get)
            if resident[victim] < nxt[i]:
                continue
            del resident[victim]
        resident[k] = nxt[i]
    return hits


def sim_pinned_lru(keys, cap, npin, hot=None, preloaded=False):
    """tools/sim_cache.py:79-110: the npin most requested keys (ties to the first seen)
    held once read, LRU in the remaining room. hot: an explicit hot set instead;
    preloaded: the hot keys are resident before the first request (a cache pinned from a
    previous workload's histogram), so their first touch is a hit too."""
    from collections import Counter, OrderedDict
    if npin >= cap:
        npin = cap - 1
    if hot is None:
        hot = {k for k, _ in Counter(keys).most_common(npin)}
    loaded = set(hot) if preloaded else set()
    seen, hits = OrderedDict(), 0
    room = max(cap - len(hot), 1)
    for k in keys:
        if k in hot:
            if k in loaded:
                hits += 1
            else:
                loaded.add(k)
            continue
        if k in seen:
            seen.move_to_end(k)
            hits += 1
        else:
            if len(seen) >= room:
                seen.popitem(last=False)
            seen[k] = 1
    return hits



class EngineIO:
    """The engine's own safetensors index and expert resolution (src/io/k3_st.c,
    src/io/k3_load.c) from _ref/libk3ref.so: k3_st_open fills a K3St exactly as the
    engine's main() would before it calls k3_cache_init, and k3_expert_ref /
    k3_expert_load give the engine's geometry and bytes of an expert."""

    def __init__(self, path):
        L = C.CDLL(path)
        vp = C.c_void_p
        L.k3_st_open.argtypes = [vp, C.c_char_p]
        L.k3_st_open.restype = C.c_int
        L.k3_st_close.argtypes = [vp]
        L.k3_st_close.restype = None
        L.k3_expert_ref.argtypes = [vp, C.c_int, C.c_int, vp]
        L.k3_expert_ref.restype = C.c_int
        L.k3_expert_load.argtypes = [vp, vp, vp]
        L.k3_expert_load.restype = C.c_int64
        self.L = L


_engine_io = None


def engine_io() -> "EngineIO | None":
    """EngineIO, or None when _ref was not built."""
    global _engine_io
    if _engine_io is None and os.path.exists(REF_SO):
        lib = C.CDLL(REF_SO)
        if hasattr(lib, "k3_st_open") and hasattr(lib, "k3_expert_load"):
            _engine_io = EngineIO(REF_SO)
    return _engine_io
