"""ctypes binding of libk3moe.so: the C ABI in include/k3moe.h, plus the seeded
synthetic layers the tests and the benchmark drive it with.

The binding mirrors the engine's own interface (include/k3/k3.h): K3Cfg, K3MoeW,
K3ExpertQ and K3ExpertSrc are the engine's struct layouts, and k3_router / k3_moe /
k3_moe_prefill / k3_matmul_mxfp4 / k3_mxfp4_dequant keep the engine's argument meaning.
Device memory and timing go straight through the HIP runtime (libamdhip64); nothing here
computes a result on the CPU.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libk3moe.so")

# ----------------------------------------------------------------- struct layouts ----


class K3Cfg(C.Structure):
    """include/k3/k3.h:73-120, field for field."""
    _fields_ = [
        ("hidden", C.c_int), ("n_layers", C.c_int), ("vocab", C.c_int), ("rms_eps", C.c_float),
        ("kda_heads", C.c_int), ("kda_head_dim", C.c_int), ("conv_k", C.c_int),
        ("gate_lb", C.c_float),
        ("n_heads", C.c_int), ("q_lora", C.c_int), ("kv_lora", C.c_int), ("qk_nope", C.c_int),
        ("qk_rope", C.c_int), ("v_head", C.c_int), ("mla_out_gate", C.c_int),
        ("n_experts", C.c_int), ("topk", C.c_int), ("n_shared", C.c_int), ("latent", C.c_int),
        ("moe_inter", C.c_int), ("routed_scale", C.c_float), ("moe_renorm", C.c_int),
        ("latent_norm", C.c_int),
        ("first_dense", C.c_int), ("dense_inter", C.c_int),
        ("attn_res_block", C.c_int),
        ("situ_b1", C.c_float), ("situ_b2", C.c_float),
        ("n_full_attn", C.c_int), ("full_attn", C.POINTER(C.c_int)),
    ]


class K3ExpertQ(C.Structure):
    """include/k3/k3.h:323-327."""
    _fields_ = [("p1", C.c_void_p), ("s1", C.c_void_p), ("p3", C.c_void_p),
                ("s3", C.c_void_p), ("p2", C.c_void_p), ("s2", C.c_void_p)]


class K3ExpertSrc(C.Structure):
    """include/k3/k3.h:332-355."""
    _fields_ = [("get", C.c_void_p), ("getmany", C.c_void_p), ("resident", C.c_void_p),
                ("ctx", C.c_void_p)]


class K3gcStats(C.Structure):
    """include/k3moe.h K3gcStats"""
    _fields_ = [("requests", C.c_int64), ("hits", C.c_int64), ("misses", C.c_int64),
                ("evictions", C.c_int64), ("prefetch_reads", C.c_int64),
                ("bytes_read", C.c_int64), ("load_seconds", C.c_double), ("nslot", C.c_int),
                ("resident", C.c_int), ("pinned", C.c_int), ("slot_bytes", C.c_int64),
                ("staged", C.c_int64)]


class K3St(C.Structure):
    """src/io/k3_st.h:56-70: the engine's checkpoint index (filled by its k3_st_open)."""
    _fields_ = [("fd", C.c_void_p), ("dfd", C.c_void_p), ("path", C.c_void_p),
                ("nshard", C.c_int), ("t", C.c_void_p), ("nt", C.c_int),
                ("bucket", C.c_void_p), ("nbucket", C.c_int), ("strpool", C.c_void_p),
                ("strcap", C.c_size_t), ("strlen_", C.c_size_t)]


class K3QMat(C.Structure):
    """src/io/k3_load.h:29-35."""
    _fields_ = [("p_off", C.c_int64), ("p_bytes", C.c_int64), ("s_off", C.c_int64),
                ("s_bytes", C.c_int64), ("rows", C.c_int), ("pcols", C.c_int),
                ("scols", C.c_int)]


class K3ExpertRef(C.Structure):
    """src/io/k3_load.h:37-43."""
    _fields_ = [("layer", C.c_int), ("expert", C.c_int), ("shard", C.c_int),
                ("off", C.c_int64), ("nbytes", C.c_int64), ("contiguous", C.c_int),
                ("m", K3QMat * 3)]


class K3Cache(C.Structure):
    """src/cache/k3_cache.h:47-96: the engine's expert cache, here on HBM slots
    (k3_cache_init of this library)."""
    _fields_ = [("src", K3ExpertSrc), ("st", C.c_void_p), ("n_layers", C.c_int),
                ("n_experts", C.c_int), ("arena", C.c_void_p), ("slot_bytes", C.c_int64),
                ("nslot", C.c_int), ("slot_of", C.POINTER(C.c_int32)),
                ("key_of", C.POINTER(C.c_int32)), ("used_at", C.POINTER(C.c_uint64)),
                ("pinned", C.POINTER(C.c_uint8)), ("ref", C.POINTER(K3ExpertRef)),
                ("pad", C.POINTER(C.c_int32)), ("clock", C.c_uint64), ("hits", C.c_uint64),
                ("misses", C.c_uint64), ("evictions", C.c_uint64), ("bytes_read", C.c_uint64),
                ("prefetch_reads", C.c_uint64), ("load_seconds", C.c_double),
                ("hist", C.POINTER(C.c_uint32)), ("trace", C.POINTER(C.c_int32)),
                ("ntrace", C.c_int64), ("captrace", C.c_int64)]


# the K3ExpertSrc entry points, called through the vtable as the engine does
SRC_GET = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p)
SRC_GETMANY = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int)
SRC_RESIDENT = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p)


class K3MoeW(C.Structure):
    """include/k3/k3.h:357-380."""
    _fields_ = [
        ("gate", C.c_void_p), ("bias", C.c_void_p),
        ("w1", C.c_void_p), ("w3", C.c_void_p), ("w2", C.c_void_p),
        ("latent_norm", C.c_void_p),
        ("down", C.c_void_p), ("up", C.c_void_p),
        ("sh1", C.c_void_p), ("sh3", C.c_void_p), ("sh2", C.c_void_p),
        ("wdt", C.c_int),
        ("src", C.c_void_p), ("layer", C.c_int), ("cache_only", C.c_int),
    ]


class K3gcExpertRun(C.Structure):
    """include/k3moe.h K3gcExpertRun"""
    _fields_ = [("shard", C.c_int), ("off", C.c_int64), ("nbytes", C.c_int64),
                ("contiguous", C.c_int), ("rows", C.c_int * 3), ("pcols", C.c_int * 3),
                ("p_bytes", C.c_int64 * 3), ("s_bytes", C.c_int64 * 3),
                ("p_file", C.c_int64 * 3), ("s_file", C.c_int64 * 3)]


class K3gExpertLayout(C.Structure):
    _fields_ = [("p1_off", C.c_int64), ("s1_off", C.c_int64), ("p2_off", C.c_int64),
                ("s2_off", C.c_int64), ("p3_off", C.c_int64), ("s3_off", C.c_int64),
                ("nbytes", C.c_int64)]


class K3gLayer(C.Structure):
    _fields_ = [
        ("hidden", C.c_int), ("n_experts", C.c_int), ("topk", C.c_int), ("inter", C.c_int),
        ("shared_inter", C.c_int), ("latent", C.c_int),
        ("renorm", C.c_int), ("routed_scale", C.c_float),
        ("act_b1", C.c_float), ("act_b2", C.c_float), ("rms_eps", C.c_float),
        ("gate", C.c_void_p), ("bias", C.c_void_p),
        ("expert_fmt", C.c_int),
        ("experts", C.c_void_p),
        ("w1", C.c_void_p), ("w3", C.c_void_p), ("w2", C.c_void_p),
        ("wdt", C.c_int),
        ("sh1", C.c_void_p), ("sh3", C.c_void_p), ("sh2", C.c_void_p),
        ("down", C.c_void_p), ("up", C.c_void_p),
        ("latent_norm", C.c_void_p),
        ("shared_fmt", C.c_int),
    ]


K3G_EXPERT_MXFP4, K3G_EXPERT_F32, K3G_EXPERT_MXFP4_TILED = 0, 1, 2
K3_WF32, K3_WBF16, K3_WI8 = 0, 1, 2
SWIGLU_CAP = float(2.0 ** 100)   # the engine's SwiGLU setting of the SiTU caps

# -------------------------------------------------------------------- libraries ----

_lib = None
_hip = None


def lib() -> C.CDLL:
    """libk3moe.so, loaded once. Raises when it has not been built: there is no CPU
    fallback for anything in it."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        vp, i, f, sz = C.c_void_p, C.c_int, C.c_float, C.c_size_t
        u64 = C.c_uint64
        L.k3_router.argtypes = [vp, vp, vp, vp, vp, i, i, i, i, f]
        L.k3_router.restype = None
        L.k3_moe.argtypes = [vp, vp, C.POINTER(K3MoeW), C.POINTER(K3Cfg), i, vp, vp, vp]
        L.k3_moe.restype = None
        L.k3_moe_prefill.argtypes = L.k3_moe.argtypes
        L.k3_moe_prefill.restype = None
        L.k3_moe_scratch.argtypes = [C.POINTER(K3Cfg)]
        L.k3_moe_scratch.restype = sz
        L.k3_matmul_mxfp4.argtypes = [vp, vp, vp, vp, i, i, i]
        L.k3_matmul_mxfp4.restype = None
        L.k3_mxfp4_dequant.argtypes = [vp, vp, vp, i, i, i]
        L.k3_mxfp4_dequant.restype = None
        L.k3moe_forget_weights.argtypes = []
        L.k3moe_forget_weights.restype = None
        L.k3moe_invalidate_weights.argtypes = [vp, sz]
        L.k3moe_invalidate_weights.restype = None
        L.k3moe_last_kernels.argtypes = []
        L.k3moe_last_kernels.restype = i
        L.k3g_expert_layout.argtypes = [i, i]
        L.k3g_expert_layout.restype = K3gExpertLayout
        L.k3g_ctx_create.argtypes = [C.POINTER(vp), i, C.POINTER(K3gLayer), i]
        L.k3g_ctx_create.restype = i
        L.k3g_ctx_destroy.argtypes = [vp]
        L.k3g_ctx_destroy.restype = None
        L.k3g_ctx_stream.argtypes = [vp]
        L.k3g_ctx_stream.restype = vp
        L.k3g_ctx_stats.argtypes = [vp, C.POINTER(C.c_int64), i]
        L.k3g_ctx_stats.restype = None
        L.k3g_ctx_force_exact.argtypes = [vp, i]
        L.k3g_ctx_force_exact.restype = None
        L.k3g_ctx_set_fused.argtypes = [vp, i]
        L.k3g_ctx_set_fused.restype = None
        L.k3g_ctx_paths.argtypes = [vp, i]
        L.k3g_ctx_paths.restype = i
        L.k3g_ctx_set_fp8.argtypes = [vp, i]
        L.k3g_ctx_set_fp8.restype = None
        L.k3g_ctx_profile.argtypes = [vp, i]
        L.k3g_ctx_profile.restype = None
        L.k3g_ctx_stage_ms.argtypes = [vp, vp, vp, i]
        L.k3g_ctx_stage_ms.restype = i
        L.k3g_router.argtypes = [vp, C.POINTER(K3gLayer), vp, i, vp, vp, vp]
        L.k3g_router.restype = i
        L.k3g_moe.argtypes = [vp, C.POINTER(K3gLayer), vp, i, vp, vp, vp, vp]
        L.k3g_moe.restype = i
        L.k3g_dispatch.argtypes = [vp, vp, i, i, i, vp, vp, vp]
        L.k3g_dispatch.restype = i
        for name in ("k3g_expert_gemv", "k3g_grouped_gemm_bf16", "k3g_grouped_gemm_f8f6f4"):
            getattr(L, name).argtypes = [vp, C.POINTER(K3gLayer), vp, i, vp, vp, vp]
            getattr(L, name).restype = i
        L.k3g_combine.argtypes = [vp, vp, vp, vp, i, i, i, vp, vp, vp]
        L.k3g_combine.restype = i
        L.k3g_moe_noalloc.argtypes = [C.POINTER(K3gLayer), vp, i, vp, vp, vp, vp, vp]
        L.k3g_moe_noalloc.restype = i
        L.k3g_sync.argtypes = [vp, vp]
        L.k3g_sync.restype = i
        L.k3s_byte.argtypes = [u64, u64, u64]
        L.k3s_byte.restype = C.c_uint8
        L.k3s_fill_bytes.argtypes = [vp, sz, u64, u64, u64]
        L.k3s_fill_bytes.restype = None
        L.k3s_fill_scales.argtypes = [vp, sz, u64, u64, u64, i, i]
        L.k3s_fill_scales.restype = None
        L.k3s_fill_normal.argtypes = [vp, sz, u64, u64, u64, f, f, i]
        L.k3s_fill_normal.restype = None
        L.k3g_fill_bytes.argtypes = [vp, sz, u64, u64, u64, vp]
        L.k3g_fill_bytes.restype = i
        L.k3g_fill_scales.argtypes = [vp, sz, u64, u64, u64, i, i, vp]
        L.k3g_fill_scales.restype = i
        L.k3g_tiled_mxfp4_bytes.argtypes = [i, i]
        L.k3g_tiled_mxfp4_bytes.restype = sz
        L.k3g_tiled_bf16_bytes.argtypes = [i, i]
        L.k3g_tiled_bf16_bytes.restype = sz
        L.k3g_tile_mxfp4.argtypes = [vp, vp, vp, i, i, vp]
        L.k3g_tile_mxfp4.restype = i
        L.k3g_tile_bf16.argtypes = [vp, vp, i, i, vp]
        L.k3g_tile_bf16.restype = i
        i64 = C.c_int64
        L.k3gc_bank_create.argtypes = [C.POINTER(vp), i, i, i, i, i]
        L.k3gc_bank_create.restype = i
        L.k3gc_bank_create_ex.argtypes = [C.POINTER(vp), i, i, i, i, i, i]
        L.k3gc_bank_create_ex.restype = i
        L.k3gc_bank_geometry.argtypes = [C.POINTER(vp), i, i, i64]
        L.k3gc_bank_geometry.restype = i
        L.k3gc_bank_free.argtypes = [vp]
        L.k3gc_bank_free.restype = None
        L.k3gc_bank_expert.argtypes = [vp, i, i]
        L.k3gc_bank_expert.restype = vp
        L.k3gc_bank_expert_bytes.argtypes = [vp]
        L.k3gc_bank_expert_bytes.restype = i64
        L.k3gc_bank_pinned_layers.argtypes = [vp]
        L.k3gc_bank_pinned_layers.restype = i
        L.k3gc_init.argtypes = [C.POINTER(vp), i, vp, i, i64]
        L.k3gc_init.restype = i
        L.k3gc_free.argtypes = [vp]
        L.k3gc_free.restype = None
        L.k3gc_src.argtypes = [vp]
        L.k3gc_src.restype = vp
        L.k3gc_pin.argtypes = [vp, i, i, i]
        L.k3gc_pin.restype = i
        L.k3gc_prefetch.argtypes = [vp, i, i]
        L.k3gc_prefetch.restype = i
        L.k3gc_reset_stats.argtypes = [vp]
        L.k3gc_reset_stats.restype = None
        L.k3gc_report.argtypes = [vp, C.c_char_p]
        L.k3gc_report.restype = None
        L.k3gc_dump_hist.argtypes = [vp, C.c_char_p]
        L.k3gc_dump_hist.restype = i
        L.k3gc_dump_trace.argtypes = [vp, C.c_char_p]
        L.k3gc_dump_trace.restype = i
        L.k3_cache_init.argtypes = [C.POINTER(K3Cache), vp, C.POINTER(K3Cfg), C.c_int64]
        L.k3_cache_init.restype = i
        L.k3_cache_free.argtypes = [C.POINTER(K3Cache)]
        L.k3_cache_free.restype = None
        L.k3_cache_pin.argtypes = [C.POINTER(K3Cache), i, i, i]
        L.k3_cache_pin.restype = i
        L.k3_cache_prefetch.argtypes = [C.POINTER(K3Cache), i, i]
        L.k3_cache_prefetch.restype = i
        L.k3_cache_reset_stats.argtypes = [C.POINTER(K3Cache)]
        L.k3_cache_reset_stats.restype = None
        L.k3_cache_report.argtypes = [C.POINTER(K3Cache), C.c_char_p]
        L.k3_cache_report.restype = None
        L.k3_cache_dump_hist.argtypes = [C.POINTER(K3Cache), C.c_char_p]
        L.k3_cache_dump_hist.restype = i
        L.k3_cache_dump_trace.argtypes = [C.POINTER(K3Cache), C.c_char_p]
        L.k3_cache_dump_trace.restype = i
        L.k3gc_stats.argtypes = [vp, C.POINTER(K3gcStats)]
        L.k3gc_stats.restype = None
        L.k3gc_step_begin.argtypes = [vp]
        L.k3gc_step_begin.restype = None
        L.k3gc_step_end.argtypes = [vp, vp]
        L.k3gc_step_end.restype = None
        L.k3gc_wait.argtypes = [vp, vp]
        L.k3gc_wait.restype = None
        L.k3gc_moe.argtypes = [vp, vp, C.POINTER(K3gLayer), i, vp, i, vp, vp, vp, vp, vp, vp]
        L.k3gc_moe.restype = i
        L.k3gc_bank_create_raw.argtypes = [C.POINTER(vp), i, i, i64, i]
        L.k3gc_bank_create_raw.restype = i
        L.k3gc_st_open.argtypes = [C.POINTER(vp), C.c_char_p]
        L.k3gc_st_open.restype = i
        L.k3gc_st_close.argtypes = [vp]
        L.k3gc_st_close.restype = None
        L.k3gc_st_count.argtypes = [vp]
        L.k3gc_st_count.restype = i
        L.k3gc_st_direct.argtypes = [vp]
        L.k3gc_st_direct.restype = i
        L.k3gc_st_expert.argtypes = [vp, i, i, C.POINTER(K3gcExpertRun)]
        L.k3gc_st_expert.restype = i
        L.k3gc_st_read_run.argtypes = [vp, C.POINTER(K3gcExpertRun), vp]
        L.k3gc_st_read_run.restype = i
        L.k3gc_st_read_run_into.argtypes = [vp, C.POINTER(K3gcExpertRun), vp, C.c_int64,
                                            C.POINTER(C.c_int64)]
        L.k3gc_st_read_run_into.restype = i
        L.k3gc_st_from_engine.argtypes = [C.POINTER(vp), vp]
        L.k3gc_st_from_engine.restype = i
        L.k3gc_bank_create_disk.argtypes = [C.POINTER(vp), vp, i, i, i]
        L.k3gc_bank_create_disk.restype = i
        L.k3gc_bank_load.argtypes = [vp, vp, i, i, i]
        L.k3gc_bank_load.restype = i
        L.k3gc_tile_mxfp4_host.argtypes = [vp, vp, vp, i, i]
        L.k3gc_tile_mxfp4_host.restype = i
        L.k3gc_chain.argtypes = [vp, vp, vp, vp, i, i, vp, i, f, vp]
        L.k3gc_chain.restype = i
        L.k3gc_pin_hottest.argtypes = [vp, vp, i]
        L.k3gc_pin_hottest.restype = i
        L.k3gc_hist.argtypes = [vp]
        L.k3gc_hist.restype = vp
        for name in ("k3gc_replay_lru", "k3gc_replay_belady"):
            getattr(L, name).argtypes = [vp, i64, i64]
            getattr(L, name).restype = i64
        L.k3gc_replay_pinned_lru.argtypes = [vp, i64, i64, i64]
        L.k3gc_replay_pinned_lru.restype = i64
        _lib = L
    return _lib


def hip() -> C.CDLL:
    """The HIP runtime, for device memory, copies and events."""
    global _hip
    if _hip is None:
        H = C.CDLL("libamdhip64.so", mode=C.RTLD_GLOBAL)
        vp, sz, i = C.c_void_p, C.c_size_t, C.c_int
        H.hipMalloc.argtypes = [C.POINTER(vp), sz]
        H.hipFree.argtypes = [vp]
        H.hipMemcpy.argtypes = [vp, vp, sz, i]
        H.hipMemcpyAsync.argtypes = [vp, vp, sz, i, vp]
        H.hipMemset.argtypes = [vp, i, sz]
        H.hipDeviceSynchronize.argtypes = []
        H.hipStreamSynchronize.argtypes = [vp]
        H.hipGetDeviceCount.argtypes = [C.POINTER(i)]
        H.hipSetDevice.argtypes = [i]
        H.hipEventCreate.argtypes = [C.POINTER(vp)]
        H.hipEventRecord.argtypes = [vp, vp]
        H.hipEventSynchronize.argtypes = [vp]
        H.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), vp, vp]
        H.hipEventDestroy.argtypes = [vp]
        H.hipGetErrorString.argtypes = [i]
        H.hipGetErrorString.restype = C.c_char_p
        H.hipHostMalloc.argtypes = [C.POINTER(vp), sz, C.c_uint]
        H.hipHostFree.argtypes = [vp]
        _hip = H
    return _hip


H2D, D2H, D2D = 1, 2, 3


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = hip().hipGetErrorString(rc)
        raise RuntimeError(f"{what} failed: {msg.decode() if msg else rc}")


def gpu_count() -> int:
    n = C.c_int(0)
    if hip().hipGetDeviceCount(C.byref(n)) != 0:
        return 0
    return n.value


class DevBuf:
    """A device allocation owned by Python."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        _check(hip().hipMalloc(C.byref(p), max(self.nbytes, 1)), f"hipMalloc({nbytes})")
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DevBuf":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        _check(hip().hipMemcpy(C.c_void_p(self.ptr + offset), a.ctypes.data_as(C.c_void_p),
                               a.nbytes, H2D), "hipMemcpy H2D")

    def download(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        _check(hip().hipMemcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr + offset),
                               out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def zero(self) -> None:
        _check(hip().hipMemset(C.c_void_p(self.ptr), 0, self.nbytes), "hipMemset")

    def free(self) -> None:
        if self.ptr:
            hip().hipFree(C.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def sync() -> None:
    _check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


class Timer:
    """HIP events on a given stream (events on the stream the kernels run on)."""

    def __init__(self, stream=None):
        H = hip()
        self.stream = stream
        self.a, self.b = C.c_void_p(), C.c_void_p()
        _check(H.hipEventCreate(C.byref(self.a)), "hipEventCreate")
        _check(H.hipEventCreate(C.byref(self.b)), "hipEventCreate")

    def start(self):
        _check(hip().hipEventRecord(self.a, C.c_void_p(self.stream)), "hipEventRecord")

    def stop(self) -> float:
        H = hip()
        _check(H.hipEventRecord(self.b, C.c_void_p(self.stream)), "hipEventRecord")
        _check(H.hipEventSynchronize(self.b), "hipEventSynchronize")
        ms = C.c_float()
        _check(H.hipEventElapsedTime(C.byref(ms), self.a, self.b), "hipEventElapsedTime")
        return float(ms.value)


# ---------------------------------------------------------------- synthetic data ----

def bf16_bits(a: np.ndarray) -> np.ndarray:
    """fp32 values already rounded to bf16 -> their 16-bit patterns."""
    return (np.ascontiguousarray(a, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def host_normal(n: int, seed: int, stream: int, mean=0.0, std=1.0, bf16=False,
                first: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().k3s_fill_normal(out.ctypes.data_as(C.c_void_p), n, seed, stream, first, mean, std,
                          1 if bf16 else 0)
    return out


def host_bytes(n: int, seed: int, stream: int, first: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint8)
    lib().k3s_fill_bytes(out.ctypes.data_as(C.c_void_p), n, seed, stream, first)
    return out


def host_scales(n: int, seed: int, stream: int, lo: int, hi: int, first: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint8)
    lib().k3s_fill_scales(out.ctypes.data_as(C.c_void_p), n, seed, stream, first, lo, hi)
    return out


# stream ids: every tensor of every layer has its own hash stream
S_GATE, S_BIAS, S_X, S_SH1, S_SH3, S_SH2 = 1, 2, 3, 4, 5, 6


def expert_stream(layer: int, e: int, mat: int, scale: bool) -> int:
    """Hash stream of matrix mat (0 = w1, 1 = w2, 2 = w3) of expert e: packed or scales."""
    return 1_000_000 + ((layer * 4096 + e) * 4 + mat) * 2 + (1 if scale else 0)


@dataclass
class Shape:
    name: str
    hidden: int
    n_experts: int
    topk: int
    inter: int
    n_shared: int = 1
    routed_scale: float = 2.5
    renorm: int = 1
    x_bf16: bool = True
    scale_lo: int = -4
    scale_hi: int = 2
    zipf_s: float = 0.0        # selection-bias skew (0 = none)
    zipf_alpha: float = 0.0


# The workloads: (c0) tiny layer on the CPU-runnable path, (c1) Kimi-K2-scale layer.
TINY = Shape("tiny d=256 E=16 k=4 I=128", 256, 16, 4, 128, x_bf16=False)
K2 = Shape("K2 d=7168 E=384 k=8 I=2048", 7168, 384, 8, 2048)
# (c2) 64-token batched decode with Zipf(1.1) expert popularity: alpha 0.025 puts ~200
# distinct experts in a 64-token step; (c3) 4096-token prefill with Zipf(0.8): alpha
# 0.02 gives a 10x spread between the 90th and 10th percentile of tokens per expert.
K2_BATCH = Shape("K2 T=64 Zipf(1.1)", 7168, 384, 8, 2048, zipf_s=1.1, zipf_alpha=0.025)
K2_PREFILL = Shape("K2 T=4096 Zipf(0.8)", 7168, 384, 8, 2048, zipf_s=0.8, zipf_alpha=0.02)


class SynthLayer:
    """A seeded K2-shaped MoE layer (no latent projection, SwiGLU, one bf16 shared
    expert, MXFP4 routed experts): host copies of the small tensors, the whole layer in
    HBM, and on-demand host regeneration of any expert for a CPU check."""

    def __init__(self, shape: Shape, seed: int, layer: int = 0, device: bool = True,
                 zipf_perm_seed: int | None = None, layout: str = "engine"):
        """layout: "engine" keeps the experts and the shared expert in the checkpoint
        layout (self.dev); "tiled" only in the tiled layouts the fused decode kernel
        streams (self.dev is then that layer); "both" keeps both (self.dev engine,
        self.dev_tiled tiled)."""
        assert layout in ("engine", "tiled", "both")
        self.layout = layout
        self.shape, self.seed, self.layer = shape, seed, layer
        d, E, I = shape.hidden, shape.n_experts, shape.inter
        SI = I * shape.n_shared
        self.SI = SI
        self.geo = lib().k3g_expert_layout(d, I)
        self.gate = host_normal(E * d, seed, S_GATE + 100 * layer, 0.0, 0.02)
        self.bias = host_normal(E, seed, S_BIAS + 100 * layer, 0.0, 0.01)
        if shape.zipf_alpha:
            # selection-only skew: alpha * log p_rank(e), p_rank Zipf(s) over a seeded
            # permutation of the experts
            rng = np.random.default_rng(seed if zipf_perm_seed is None else zipf_perm_seed)
            perm = rng.permutation(E)
            ranks = np.empty(E, dtype=np.int64)
            ranks[perm] = np.arange(1, E + 1)
            p = ranks.astype(np.float64) ** (-shape.zipf_s)
            p /= p.sum()
            self.bias = (self.bias + shape.zipf_alpha * np.log(p)).astype(np.float32)
        sh = []
        for s in (S_SH1, S_SH3, S_SH2):
            v = host_normal(SI * d, seed, s + 100 * layer, 0.0, 0.02, bf16=True)
            sh.append(bf16_bits(v))
        self.sh1, self.sh3, self.sh2 = sh
        self.dev = None
        if device:
            self.to_device()

    # -- experts -------------------------------------------------------------------
    def expert_host(self, e: int) -> np.ndarray:
        """Expert e's run (w1p w1s w2p w2s w3p w3s), regenerated on the host."""
        g, d, I = self.geo, self.shape.hidden, self.shape.inter
        out = np.empty(g.nbytes, dtype=np.uint8)
        lo, hi = self.shape.scale_lo, self.shape.scale_hi
        parts = [(0, g.p1_off, I * d // 2, g.s1_off, I * ((d + 31) // 32)),
                 (1, g.p2_off, d * I // 2, g.s2_off, d * ((I + 31) // 32)),
                 (2, g.p3_off, I * d // 2, g.s3_off, I * ((d + 31) // 32))]
        for m, po, pn, so, sn in parts:
            out[po:po + pn] = host_bytes(pn, self.seed, expert_stream(self.layer, e, m, False))
            out[so:so + sn] = host_scales(sn, self.seed, expert_stream(self.layer, e, m, True),
                                          lo, hi)
        return out

    def fill_expert_device(self, base_ptr: int, e: int, stream=None) -> None:
        g, d, I = self.geo, self.shape.hidden, self.shape.inter
        lo, hi = self.shape.scale_lo, self.shape.scale_hi
        parts = [(0, g.p1_off, I * d // 2, g.s1_off, I * ((d + 31) // 32)),
                 (1, g.p2_off, d * I // 2, g.s2_off, d * ((I + 31) // 32)),
                 (2, g.p3_off, I * d // 2, g.s3_off, I * ((d + 31) // 32))]
        L = lib()
        for m, po, pn, so, sn in parts:
            _check(L.k3g_fill_bytes(C.c_void_p(base_ptr + po), pn, self.seed,
                                    expert_stream(self.layer, e, m, False), 0, stream),
                   "k3g_fill_bytes")
            _check(L.k3g_fill_scales(C.c_void_p(base_ptr + so), sn, self.seed,
                                     expert_stream(self.layer, e, m, True), 0, lo, hi, stream),
                   "k3g_fill_scales")

    def expert_table(self, bank_ptr: int) -> list:
        g = self.geo
        tab = (K3ExpertQ * self.shape.n_experts)()
        for e in range(self.shape.n_experts):
            b = bank_ptr + e * g.nbytes
            tab[e] = K3ExpertQ(b + g.p1_off, b + g.s1_off, b + g.p3_off, b + g.s3_off,
                               b + g.p2_off, b + g.s2_off)
        return tab

    def tiled_sizes(self):
        """(w1/w3 bytes, w2 bytes, expert bytes) of one expert in the tiled layout"""
        d, I = self.shape.hidden, self.shape.inter
        t13 = lib().k3g_tiled_mxfp4_bytes(I, d)
        t2 = lib().k3g_tiled_mxfp4_bytes(d, I)
        if not t13 or not t2:
            raise ValueError(f"shape d={d} I={I} has no tiled layout")
        return t13, t2, 2 * t13 + t2

    def _upload_table(self, tab) -> "DevBuf":
        buf = DevBuf(C.sizeof(tab))
        _check(hip().hipMemcpy(C.c_void_p(buf.ptr), C.cast(tab, C.c_void_p), C.sizeof(tab),
                               H2D), "table upload")
        return buf

    def to_device(self) -> None:
        E, g = self.shape.n_experts, self.geo
        d, I = self.shape.hidden, self.shape.inter
        L = lib()
        keep_engine = self.layout in ("engine", "both")
        if keep_engine:
            self.bank = DevBuf(E * g.nbytes)
            for e in range(E):
                self.fill_expert_device(self.bank.ptr + e * g.nbytes, e)
            sync()
            self.d_table = self._upload_table(self.expert_table(self.bank.ptr))
        self.d_gate = DevBuf.from_array(self.gate)
        self.d_bias = DevBuf.from_array(self.bias)
        self.d_sh1 = DevBuf.from_array(self.sh1)
        self.d_sh3 = DevBuf.from_array(self.sh3)
        self.d_sh2 = DevBuf.from_array(self.sh2)
        if self.layout in ("tiled", "both"):
            t13, t2, te = self.tiled_sizes()
            self.tbank = DevBuf(E * te)
            scratch = None if keep_engine else DevBuf(g.nbytes)
            tab = (K3ExpertQ * E)()
            for e in range(E):
                src = self.bank.ptr + e * g.nbytes if keep_engine else scratch.ptr
                if not keep_engine:
                    self.fill_expert_device(src, e)
                tb = self.tbank.ptr + e * te
                for dst, po, so, rows, cols in ((tb, g.p1_off, g.s1_off, I, d),
                                                (tb + t13, g.p3_off, g.s3_off, I, d),
                                                (tb + 2 * t13, g.p2_off, g.s2_off, d, I)):
                    _check(L.k3g_tile_mxfp4(C.c_void_p(dst), C.c_void_p(src + po),
                                            C.c_void_p(src + so), rows, cols, None),
                           "k3g_tile_mxfp4")
                tab[e] = K3ExpertQ(tb, None, tb + t13, None, tb + 2 * t13, None)
            sync()
            del scratch
            self.d_ttable = self._upload_table(tab)
            if self.SI:
                self.d_tsh = []
                for src, rows, cols in ((self.d_sh1, self.SI, d), (self.d_sh3, self.SI, d),
                                        (self.d_sh2, d, self.SI)):
                    t = DevBuf(L.k3g_tiled_bf16_bytes(rows, cols))
                    _check(L.k3g_tile_bf16(C.c_void_p(t.ptr), C.c_void_p(src.ptr), rows, cols,
                                           None), "k3g_tile_bf16")
                    self.d_tsh.append(t)
                sync()
            self.dev_tiled = self.k3g_layer(tiled=True)
        self.dev = self.k3g_layer() if keep_engine else self.dev_tiled

    def release_experts(self) -> None:
        """free the device copies of the routed experts (the HBM cache serves them from a
        host bank instead); gate, bias and the shared expert stay resident"""
        for name in ("bank", "tbank", "d_table", "d_ttable"):
            b = getattr(self, name, None)
            if b is not None:
                b.free()
                setattr(self, name, None)
        # the layer descriptors no longer name an expert table: a call that needs one is
        # refused by the library instead of reading freed memory
        for name in ("dev", "dev_tiled"):
            L = getattr(self, name, None)
            if L is not None:
                L.experts = None

    def k3g_layer(self, tiled: bool = False) -> K3gLayer:
        s = self.shape
        L = K3gLayer()
        L.hidden, L.n_experts, L.topk, L.inter = s.hidden, s.n_experts, s.topk, s.inter
        L.shared_inter, L.latent = self.SI, s.hidden
        L.renorm, L.routed_scale = s.renorm, s.routed_scale
        L.act_b1 = L.act_b2 = SWIGLU_CAP
        L.rms_eps = 1e-5
        L.gate, L.bias = self.d_gate.ptr, self.d_bias.ptr
        L.wdt = K3_WBF16
        if tiled:
            L.expert_fmt = K3G_EXPERT_MXFP4_TILED
            L.experts = self.d_ttable.ptr
            if self.SI:
                L.sh1, L.sh3, L.sh2 = (t.ptr for t in self.d_tsh)
                L.shared_fmt = 1
        else:
            L.expert_fmt = K3G_EXPERT_MXFP4
            L.experts = self.d_table.ptr
            if self.SI:
                L.sh1, L.sh3, L.sh2 = self.d_sh1.ptr, self.d_sh3.ptr, self.d_sh2.ptr
        return L

    def cfg(self) -> K3Cfg:
        s = self.shape
        c = K3Cfg()
        c.hidden, c.latent, c.moe_inter = s.hidden, s.hidden, s.inter
        c.n_experts, c.topk, c.n_shared = s.n_experts, s.topk, s.n_shared
        c.routed_scale, c.moe_renorm, c.latent_norm = s.routed_scale, s.renorm, 0
        c.rms_eps = 1e-5
        c.situ_b1 = c.situ_b2 = SWIGLU_CAP
        c.n_layers = 1
        return c

    def tokens(self, T: int, stream_base: int = 0, bf16=None) -> np.ndarray:
        """T tokens of the layer's input stream; bf16 (default: the shape's x_bf16) rounds
        the same draws to bf16 values."""
        x = host_normal(T * self.shape.hidden, self.seed, S_X + 100 * self.layer + stream_base,
                        0.0, 1.0, bf16=self.shape.x_bf16 if bf16 is None else bf16)
        return x.reshape(T, self.shape.hidden)


class Ctx:
    """A k3g context sized for a layer shape and token budget."""

    def __init__(self, layer: K3gLayer, max_tokens: int, device: int = 0):
        self.ptr = C.c_void_p()
        rc = lib().k3g_ctx_create(C.byref(self.ptr), device, C.byref(layer), max_tokens)
        if rc != 0:
            raise RuntimeError("k3g_ctx_create failed")
        self.stream = lib().k3g_ctx_stream(self.ptr)

    def moe(self, layer: K3gLayer, x_ptr: int, T: int, out_ptr: int, idx_ptr=None,
            wt_ptr=None) -> None:
        rc = lib().k3g_moe(self.ptr, C.byref(layer), C.c_void_p(x_ptr), T, C.c_void_p(out_ptr),
                           C.c_void_p(idx_ptr) if idx_ptr else None,
                           C.c_void_p(wt_ptr) if wt_ptr else None, None)
        if rc != 0:
            raise RuntimeError("k3g_moe launch failed")

    def router(self, layer: K3gLayer, x_ptr: int, T: int, idx_ptr: int, wt_ptr: int) -> None:
        rc = lib().k3g_router(self.ptr, C.byref(layer), C.c_void_p(x_ptr), T,
                              C.c_void_p(idx_ptr), C.c_void_p(wt_ptr), None)
        if rc != 0:
            raise RuntimeError("k3g_router launch failed")

    # the layer's steps one at a time (device pointers, the context's stream)
    def dispatch(self, idx_ptr: int, T: int, topk: int, n_experts: int, perm_ptr: int,
                 off_ptr: int) -> None:
        rc = lib().k3g_dispatch(self.ptr, C.c_void_p(idx_ptr), T, topk, n_experts,
                                C.c_void_p(perm_ptr), C.c_void_p(off_ptr), None)
        if rc != 0:
            raise RuntimeError("k3g_dispatch failed")

    def experts(self, kind: str, layer: K3gLayer, x_ptr: int, T: int, idx_ptr: int,
                contrib_ptr: int) -> None:
        """kind: "gemv", "bf16" or "f8f6f4" (k3g_expert_gemv / k3g_grouped_gemm_*)."""
        fn = {"gemv": lib().k3g_expert_gemv, "bf16": lib().k3g_grouped_gemm_bf16,
              "f8f6f4": lib().k3g_grouped_gemm_f8f6f4}[kind]
        rc = fn(self.ptr, C.byref(layer), C.c_void_p(x_ptr), T, C.c_void_p(idx_ptr),
                C.c_void_p(contrib_ptr), None)
        if rc != 0:
            raise RuntimeError(f"expert products ({kind}) failed")

    def combine(self, contrib_ptr: int, idx_ptr: int, wt_ptr: int, T: int, topk: int, n: int,
                add_ptr, out_ptr: int) -> None:
        rc = lib().k3g_combine(self.ptr, C.c_void_p(contrib_ptr), C.c_void_p(idx_ptr),
                               C.c_void_p(wt_ptr), T, topk, n,
                               C.c_void_p(add_ptr) if add_ptr else None, C.c_void_p(out_ptr),
                               None)
        if rc != 0:
            raise RuntimeError("k3g_combine failed")

    def sync(self) -> None:
        rc = lib().k3g_sync(self.ptr, None)
        if rc != 0:
            raise RuntimeError(f"device error {rc}")

    def force_exact(self, mode: int) -> None:
        lib().k3g_ctx_force_exact(self.ptr, mode)

    def paths(self, clear: bool = True) -> int:
        """kernels run since the last clear: 1 staged, 2 fused decode, 4 grouped GEMMs"""
        return lib().k3g_ctx_paths(self.ptr, int(clear))

    def set_fused(self, on: bool) -> None:
        lib().k3g_ctx_set_fused(self.ptr, 1 if on else 0)

    def profile(self, on: bool) -> None:
        lib().k3g_ctx_profile(self.ptr, 1 if on else 0)

    def stage_ms(self):
        ms = np.zeros(16)
        n = np.zeros(16, np.int64)
        ns = lib().k3g_ctx_stage_ms(self.ptr, ms.ctypes.data, n.ctypes.data, 16)
        return ms[:ns], n[:ns]

    def set_fp8(self, on: bool) -> None:
        lib().k3g_ctx_set_fp8(self.ptr, 1 if on else 0)

    def stats(self) -> list:
        out = (C.c_int64 * 4)()
        lib().k3g_ctx_stats(self.ptr, out, 4)
        return list(out)

    def destroy(self) -> None:
        if self.ptr:
            lib().k3g_ctx_destroy(self.ptr)
            self.ptr = C.c_void_p()


# ------------------------------------------------------------------ HBM expert cache ----

def replay(policy: str, trace_pairs: np.ndarray, capacity: int, npin: int = 0) -> int:
    """Hits of an offline replay of a (layer, expert) trace: policy "lru", "belady" or
    "pinned_lru" (k3gc_replay_*)."""
    t = np.ascontiguousarray(trace_pairs, np.int32).reshape(-1)
    n = t.size // 2
    if policy == "pinned_lru":
        return lib().k3gc_replay_pinned_lru(t.ctypes.data, n, capacity, npin)
    return getattr(lib(), "k3gc_replay_" + policy)(t.ctypes.data, n, capacity)



class Bank:
    """A pinned host bank of expert runs (k3gc_bank_create), or a geometry-only bank for
    bookkeeping replays (k3gc_bank_geometry)."""

    def __init__(self, n_layers: int, n_experts: int, hidden: int = 0, inter: int = 0,
                 layout: int = K3G_EXPERT_MXFP4_TILED, expert_bytes: int = 0,
                 max_pinned_layers: int = -1, raw: bool = False):
        """raw: host memory for runs of expert_bytes with no layer shape
        (k3gc_bank_create_raw); expert_bytes alone: the geometry only."""
        self.ptr = C.c_void_p()
        if raw:
            rc = lib().k3gc_bank_create_raw(C.byref(self.ptr), n_layers, n_experts, expert_bytes,
                                            max_pinned_layers)
            layout = K3G_EXPERT_MXFP4
        elif expert_bytes:
            rc = lib().k3gc_bank_geometry(C.byref(self.ptr), n_layers, n_experts, expert_bytes)
        else:
            rc = lib().k3gc_bank_create_ex(C.byref(self.ptr), n_layers, n_experts, hidden,
                                           inter, layout, max_pinned_layers)
        if rc != 0:
            raise RuntimeError("k3gc bank creation failed")
        self.n_layers, self.n_experts, self.layout = n_layers, n_experts, layout
        self.expert_bytes = lib().k3gc_bank_expert_bytes(self.ptr)
        self.pinned_layers = lib().k3gc_bank_pinned_layers(self.ptr)

    def expert(self, layer: int, e: int) -> int:
        return lib().k3gc_bank_expert(self.ptr, layer, e)

    def expert_bytes_of(self, layer: int, e: int) -> np.ndarray:
        """a copy of the run of (layer, e) in the bank's host memory"""
        return np.frombuffer(C.string_at(self.expert(layer, e), self.expert_bytes), np.uint8).copy()

    def load(self, st: "St", ck_layer0: int, bank_layer0: int, n_layers: int) -> None:
        if lib().k3gc_bank_load(self.ptr, st.ptr, ck_layer0, bank_layer0, n_layers) != 0:
            raise RuntimeError("k3gc_bank_load failed")

    def fill_from_layer(self, layer_obj: "SynthLayer", layer: int) -> None:
        """copy every expert run of a device-resident SynthLayer into this bank row"""
        if self.layout == K3G_EXPERT_MXFP4_TILED:
            base, step = layer_obj.tbank.ptr, layer_obj.tiled_sizes()[2]
        else:
            base, step = layer_obj.bank.ptr, layer_obj.geo.nbytes
        assert step == self.expert_bytes
        for e in range(self.n_experts):
            _check(hip().hipMemcpy(C.c_void_p(self.expert(layer, e)), C.c_void_p(base + e * step),
                                   step, D2H), "bank fill")

    def free(self) -> None:
        if self.ptr:
            lib().k3gc_bank_free(self.ptr)
            self.ptr = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class St:
    """An index of the safetensors shards of a directory (k3gc_st_open), or of the engine's
    own K3St (St.from_engine: k3gc_st_from_engine)."""

    def __init__(self, path: str | None):
        self.ptr = C.c_void_p()
        if path is not None and lib().k3gc_st_open(C.byref(self.ptr), path.encode()) != 0:
            raise RuntimeError(f"k3gc_st_open({path}) failed")

    @classmethod
    def from_engine(cls, engine_st) -> "St":
        """engine_st: a K3St the engine's k3_st_open filled (kept alive by the caller)."""
        s = cls(None)
        if lib().k3gc_st_from_engine(C.byref(s.ptr), C.byref(engine_st)) != 0:
            raise RuntimeError("k3gc_st_from_engine failed")
        return s

    def read_run_into(self, r: K3gcExpertRun, buf: np.ndarray) -> int:
        """The run into buf (k3gc_st_read_run_into); returns where it starts in buf."""
        pad = C.c_int64()
        if lib().k3gc_st_read_run_into(self.ptr, C.byref(r), buf.ctypes.data, buf.size,
                                       C.byref(pad)) != 0:
            raise IOError("short read")
        return pad.value

    def count(self) -> int:
        return lib().k3gc_st_count(self.ptr)

    def direct(self) -> int:
        """shards read with O_DIRECT"""
        return lib().k3gc_st_direct(self.ptr)

    def expert(self, layer: int, e: int) -> K3gcExpertRun:
        r = K3gcExpertRun()
        if lib().k3gc_st_expert(self.ptr, layer, e, C.byref(r)) != 0:
            raise KeyError((layer, e))
        return r

    def read_run(self, r: K3gcExpertRun) -> np.ndarray:
        out = np.empty(r.nbytes, np.uint8)
        if lib().k3gc_st_read_run(self.ptr, C.byref(r), out.ctypes.data) != 0:
            raise IOError("short read")
        return out

    def close(self) -> None:
        if self.ptr:
            lib().k3gc_st_close(self.ptr)
            self.ptr = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def tile_mxfp4_host(packed: np.ndarray, scales: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """k3gc_tile_mxfp4_host: the tiled layout written by the host"""
    n = lib().k3g_tiled_mxfp4_bytes(rows, cols)
    out = np.empty(n, np.uint8)
    p, s = np.ascontiguousarray(packed, np.uint8), np.ascontiguousarray(scales, np.uint8)
    if lib().k3gc_tile_mxfp4_host(out.ctypes.data, p.ctypes.data, s.ctypes.data, rows, cols) != 0:
        raise ValueError("no tiled layout for this shape")
    return out


class Cache:
    """The HBM expert cache (k3gc_init): slots in device memory (device >= 0) or the
    bookkeeping alone (device < 0)."""

    def __init__(self, bank: Bank, topk: int, budget_bytes: int, device: int = 0):
        self.bank = bank
        self.ptr = C.c_void_p()
        if lib().k3gc_init(C.byref(self.ptr), device, bank.ptr, topk, int(budget_bytes)) != 0:
            raise RuntimeError("k3gc_init failed")
        self.src_ptr = lib().k3gc_src(self.ptr)
        src = K3ExpertSrc.from_address(self.src_ptr)
        self._get = SRC_GET(src.get)
        # no batch path when the cache was made with K3_NOPREFETCH set
        self._getmany = SRC_GETMANY(src.getmany) if src.getmany else None
        self._resident = SRC_RESIDENT(src.resident)

    def get(self, layer: int, e: int):
        q = K3ExpertQ()
        rc = self._get(self.src_ptr, layer, e, C.addressof(q))
        return q if rc == 0 else None

    def getmany(self, layer: int, experts) -> int:
        if self._getmany is None:
            return 0
        a = np.ascontiguousarray(experts, np.int32)
        return self._getmany(self.src_ptr, layer, a.ctypes.data, a.size)

    def resident(self, layer: int, e: int) -> bool:
        return bool(self._resident(self.src_ptr, layer, e, None))

    def pin(self, layer, e, on=True) -> int:
        return lib().k3gc_pin(self.ptr, layer, e, 1 if on else 0)

    def hist(self) -> np.ndarray:
        """A copy of the request histogram [n_layers][n_experts]."""
        n = self.bank.n_layers * self.bank.n_experts
        p = lib().k3gc_hist(self.ptr)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint32)), (n,)).copy()

    def pin_hottest(self, hist: np.ndarray, npin: int) -> int:
        h = np.ascontiguousarray(hist, np.uint32)
        return lib().k3gc_pin_hottest(self.ptr, h.ctypes.data, npin)

    def prefetch(self, layer, e) -> int:
        return lib().k3gc_prefetch(self.ptr, layer, e)

    def stats(self) -> K3gcStats:
        st = K3gcStats()
        lib().k3gc_stats(self.ptr, C.byref(st))
        return st

    def reset_stats(self) -> None:
        lib().k3gc_reset_stats(self.ptr)

    def trace(self) -> np.ndarray:
        """The (layer, expert) pairs of every get() so far, in order, [n][2] int32 (the
        engine's expert_trace.bin format, through k3gc_dump_trace)."""
        import tempfile
        with tempfile.TemporaryDirectory() as d:
            path = os.path.join(d, "trace.bin")
            if lib().k3gc_dump_trace(self.ptr, path.encode()) != 0:
                return np.zeros((0, 2), np.int32)
            return np.fromfile(path, np.int32).reshape(-1, 2)

    def report(self, label: str = "") -> None:
        lib().k3gc_report(self.ptr, label.encode())

    def step_begin(self) -> None:
        lib().k3gc_step_begin(self.ptr)

    def step_end(self, stream=None) -> None:
        lib().k3gc_step_end(self.ptr, stream)

    def moe(self, ctx: "Ctx", L: K3gLayer, layer: int, x_ptr: int, T: int, out_ptr: int,
            idx_ptr: int, wt_ptr: int, route_idx=None, route_wt=None) -> None:
        ri = None if route_idx is None else np.ascontiguousarray(route_idx, np.int32)
        rw = None if route_wt is None else np.ascontiguousarray(route_wt, np.float32)
        rc = lib().k3gc_moe(ctx.ptr, self.ptr, C.byref(L), layer, x_ptr, T, out_ptr, idx_ptr,
                            wt_ptr, None if ri is None else ri.ctypes.data,
                            None if rw is None else rw.ctypes.data, None)
        if rc != 0:
            raise RuntimeError("k3gc_moe failed")

    def chain(self, ctx: "Ctx", layers: list, post_norms: list, first_layer: int, h_ptr: int,
              T: int, rms_eps: float = 1e-5) -> None:
        """k3gc_chain: h (device [T][hidden]) through the MoE half of len(layers) layers;
        post_norms: device pointers of the RMSNorm weights (None entries: no norm)."""
        self.chain_call(ctx, layers, post_norms, first_layer, h_ptr, T, rms_eps)()

    def chain_call(self, ctx: "Ctx", layers: list, post_norms: list, first_layer: int,
                   h_ptr: int, T: int, rms_eps: float = 1e-5):
        """The same call with its argument arrays formed once, as a C caller holds them:
        returns a function that runs k3gc_chain (and raises on failure)."""
        arr = (K3gLayer * len(layers))(*layers)
        pn = (C.c_void_p * len(layers))(*[p if p else None for p in post_norms])
        fn, n = lib().k3gc_chain, len(layers)
        cp, sp, hp = ctx.ptr, self.ptr, C.c_void_p(h_ptr)

        def run() -> None:
            if fn(cp, sp, arr, pn, first_layer, n, hp, T, rms_eps, None) != 0:
                raise RuntimeError("k3gc_chain failed")
        return run

    def free(self) -> None:
        if self.ptr:
            lib().k3gc_free(self.ptr)
            self.ptr = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
