"""Writes the golden fixtures under tests/golden/ from the reference's own test data.

Run where the reference checkout is (default /root/reference); the tests, on any machine,
only read the .npz / .json files this writes. Inputs are data files the
reference's tests hold:

  tests/fixtures/ops/router.json    k3_router golden (test_ops.c:350-401)
  tests/fixtures/ops/moe.json       k3_moe LatentMoE golden, fp32 bank (test_ops.c:465-545)
  tests/fixtures/ops/situ_glu.json  SiTU-GLU golden
  tests/fixtures/ops/MANIFEST.json  tolerances (fp32_abs, fp32_rel)
  tests/fixtures/mxfp4.json         real checkpoint MXFP4 bytes + exact dequant (test_ops.c:743-796)
  tests/fixtures/expert_trace.bin   100,096 (layer, expert) requests (k3_cache.c:244-255)
  tests/fixtures/cache/model-00001-of-00001.safetensors
                                    a structurally real checkpoint shard, 24 routed experts
                                    (144 tensors) of layer 0 (test_cache.c:86-140), copied as
                                    is into cache_fixture/

plus the byte layout of the engine's public structs, measured by compiling a probe
against include/k3/k3.h, so the ABI test can check this library's layouts without the
reference present.
"""
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
OUT = os.path.dirname(os.path.abspath(__file__))
FX = os.path.join(REF, "tests", "fixtures")


def arr(d, key, dtype=np.float32):
    v = d[key]
    data = v["data"] if isinstance(v, dict) else v
    shape = v.get("shape") if isinstance(v, dict) else None
    a = np.asarray(data, dtype=dtype)
    return a.reshape(shape) if shape else a


def router():
    d = json.load(open(os.path.join(FX, "ops", "router.json")))
    np.savez_compressed(os.path.join(OUT, "router.npz"),
                        gate_weight=arr(d, "gate_weight"), bias=arr(d, "bias"), x=arr(d, "in"),
                        topk_idx=arr(d, "topk_idx", np.int64).astype(np.int32),
                        topk_weight=arr(d, "topk_weight"), top_k=np.int32(d["top_k"]),
                        n_experts=np.int32(d["n_experts"]),
                        rows_where_bias_changed_selection=np.int32(
                            d["rows_where_bias_changed_selection"]))


def moe():
    d = json.load(open(os.path.join(FX, "ops", "moe.json")))
    out = {}
    for k in ("hidden", "latent", "moe_inter", "n_experts", "top_k", "n_shared", "renorm",
              "latent_norm"):
        out[k] = np.int32(d[k])
    for k in ("routed_scale", "rms_eps", "situ_b1", "situ_b2"):
        out[k] = np.float32(d[k])
    for k in ("in", "out", "e_score_correction_bias", "gate_weight", "down_weight", "up_weight",
              "norm_weight", "shared_w1_weight", "shared_w3_weight", "shared_w2_weight"):
        out[k] = arr(d, k)
    E = int(d["n_experts"])
    out["w1"] = np.stack([arr(d, f"experts_{e}_w1_weight") for e in range(E)])
    out["w3"] = np.stack([arr(d, f"experts_{e}_w3_weight") for e in range(E)])
    out["w2"] = np.stack([arr(d, f"experts_{e}_w2_weight") for e in range(E)])
    np.savez_compressed(os.path.join(OUT, "moe.npz"), **out)


def situ():
    d = json.load(open(os.path.join(FX, "ops", "situ_glu.json")))
    np.savez_compressed(os.path.join(OUT, "situ_glu.npz"), x=arr(d, "in"), y=arr(d, "out"),
                        beta=np.float32(d["beta"]), linear_beta=np.float32(d["linear_beta"]),
                        max_abs=np.float32(d["max_abs"]))


def mxfp4():
    d = json.load(open(os.path.join(FX, "mxfp4.json")))
    sw = d["expected_swapped_nibbles"]
    np.savez_compressed(os.path.join(OUT, "mxfp4.npz"),
                        packed=arr(d, "packed", np.uint8), scales=arr(d, "scales", np.uint8),
                        expected=arr(d, "expected"), rows=np.int32(d["rows"]),
                        packed_cols=np.int32(d["packed_cols"]),
                        group_size=np.int32(d["group_size"]),
                        e2m1_lut=np.asarray(d["e2m1_lut"], np.float32),
                        swapped_first64=np.asarray(sw["first64"], np.float32))


def manifest():
    d = json.load(open(os.path.join(FX, "ops", "MANIFEST.json")))
    json.dump({"tolerance": d["tolerance"]}, open(os.path.join(OUT, "tolerance.json"), "w"),
              indent=1)


def trace():
    raw = np.fromfile(os.path.join(FX, "expert_trace.bin"), dtype=np.int32)
    np.savez_compressed(os.path.join(OUT, "expert_trace.npz"), pairs=raw.reshape(-1, 2))


def cache_fixture():
    import shutil
    os.makedirs(os.path.join(OUT, "cache_fixture"), exist_ok=True)
    shutil.copyfile(os.path.join(FX, "cache", "model-00001-of-00001.safetensors"),
                    os.path.join(OUT, "cache_fixture", "model-00001-of-00001.safetensors"))


def layouts():
    fields = {
        "K3Cfg": ["hidden", "rms_eps", "n_experts", "topk", "n_shared", "latent", "moe_inter",
                  "routed_scale", "moe_renorm", "latent_norm", "situ_b1", "situ_b2",
                  "n_full_attn", "full_attn"],
        "K3MoeW": ["gate", "bias", "w1", "w3", "w2", "latent_norm", "down", "up", "sh1", "sh3",
                   "sh2", "wdt", "src", "layer", "cache_only"],
        "K3ExpertQ": ["p1", "s1", "p3", "s3", "p2", "s2"],
        "K3ExpertSrc": ["get", "getmany", "resident", "ctx"],
        "K3Tensor": ["name", "shard", "dtype", "ndim", "shape", "off", "nbytes"],
        "K3St": ["fd", "dfd", "path", "nshard", "t", "nt", "bucket", "nbucket", "strpool",
                 "strcap", "strlen_"],
        "K3QMat": ["p_off", "p_bytes", "s_off", "s_bytes", "rows", "pcols", "scols"],
        "K3ExpertRef": ["layer", "expert", "shard", "off", "nbytes", "contiguous", "m"],
        "K3Cache": ["src", "st", "n_layers", "n_experts", "arena", "slot_bytes", "nslot",
                    "slot_of", "key_of", "used_at", "pinned", "ref", "pad", "clock", "hits",
                    "misses", "evictions", "bytes_read", "prefetch_reads", "load_seconds",
                    "hist", "trace", "ntrace", "captrace"],
    }
    src = ['#include <stdio.h>', '#include <stddef.h>', '#include "k3.h"', '#include "k3_cache.h"',
           'int main(void){', 'printf("{");']
    first = True
    for t, fs in fields.items():
        src.append(f'printf("{"" if first else ","}\\"{t}\\": {{\\"sizeof\\": %zu", sizeof({t}));')
        first = False
        for f in fs:
            src.append(f'printf(", \\"{f}\\": %zu", offsetof({t}, {f}));')
        src.append('printf("}");')
    src.append('printf("}\\n"); return 0; }')
    with tempfile.TemporaryDirectory() as td:
        c = os.path.join(td, "probe.c")
        open(c, "w").write("\n".join(src))
        exe = os.path.join(td, "probe")
        subprocess.check_call(["gcc", "-std=gnu99", "-I", os.path.join(REF, "include", "k3"),
                               "-I", os.path.join(REF, "src", "io"), "-I",
                               os.path.join(REF, "src", "cache"), c, "-o", exe])
        lay = json.loads(subprocess.check_output([exe]).decode())
    json.dump(lay, open(os.path.join(OUT, "layouts.json"), "w"), indent=1)


if __name__ == "__main__":
    if sys.argv[2:] == ["layouts"]:
        layouts()
        sys.exit(0)
    router(); moe(); situ(); mxfp4(); manifest(); trace(); cache_fixture(); layouts()
    for f in sorted(os.listdir(OUT)):
        print(f, os.path.getsize(os.path.join(OUT, f)))
