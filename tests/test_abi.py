"""The C-ABI library on the CPU: it loads, it exports every function include/k3moe.h
declares, its structs keep the engine's layout, and its host-side helpers (expert run
geometry, tiled sizes, the seeded synthetic generator) give the documented values. No
kernel is launched here."""
import ctypes as C
import json
import os
import re
import subprocess
import tempfile

import numpy as np
import pytest

import k3moe

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "k3moe.h")
GOLDEN = os.path.join(ROOT, "tests", "golden")


def declared_functions():
    """Names of the functions include/k3moe.h declares (outside struct bodies)."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"#ifdef __cplusplus.*?#endif", "", text, flags=re.S)
    text = re.sub(r"^\s*#.*$", "", text, flags=re.M)
    depth, flat = 0, []
    for ch in text:
        if ch == "{":
            depth += 1
        elif ch == "}":
            depth -= 1
        elif depth == 0:
            flat.append(ch)
    flat = "".join(flat)
    names = set()
    for stmt in flat.split(";"):
        stmt = " ".join(stmt.split())
        if not stmt or stmt.startswith("typedef") or "extern \"C\"" in stmt:
            continue
        m = re.match(r"^(?:extern\s+)?[A-Za-z_][\w\s\*]*?\b([A-Za-z_]\w*)\s*\(", stmt)
        if m:
            names.add(m.group(1))
    return names


def test_library_loads_and_exports_every_declared_function():
    L = C.CDLL(k3moe.LIB_PATH)
    names = declared_functions()
    assert len(names) >= 25, names
    missing = [n for n in sorted(names) if not hasattr(L, n)]
    assert not missing, missing
    # the engine's global drop counter is exported too
    C.c_long.in_dll(L, "k3_expert_drops")


def test_struct_layouts_match_the_engine():
    """Offsets of K3Cfg / K3MoeW / K3ExpertQ / K3ExpertSrc as declared in
    include/k3moe.h, measured by a compiled probe, against the engine's own k3.h layout
    (tests/golden/layouts.json, probed from include/k3/k3.h)."""
    want = json.load(open(os.path.join(GOLDEN, "layouts.json")))
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "k3moe.h"', 'int main(void){']
    for st, fields in want.items():
        lines.append(f'printf("{st} sizeof %zu\\n", sizeof({st}));')
        for f in fields:
            if f != "sizeof":
                lines.append(f'printf("{st} {f} %zu\\n", offsetof({st}, {f}));')
    lines.append("return 0;}")
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "probe.c"), os.path.join(d, "probe")
        open(src, "w").write("\n".join(lines))
        subprocess.run(["gcc", "-std=c99", "-I", os.path.dirname(HEADER), src, "-o", exe],
                       check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    got = {}
    for line in out.splitlines():
        st, f, v = line.split()
        got.setdefault(st, {})[f] = int(v)
    assert got == want
    # and the ctypes binding agrees with both
    for st in ("K3Cfg", "K3MoeW", "K3ExpertQ", "K3ExpertSrc"):
        cls = getattr(k3moe, st)
        assert C.sizeof(cls) == want[st]["sizeof"], st
        for f, off in want[st].items():
            if f != "sizeof":
                assert getattr(cls, f).offset == off, (st, f)


def test_expert_run_geometry():
    """src/io/k3_load.h:3-9 order w1p w1s w2p w2s w3p w3s; 23,396,352 bytes at d=7168,
    I=2048 and 52,224 at d=256, I=128."""
    g = k3moe.lib().k3g_expert_layout(7168, 2048)
    assert (g.p1_off, g.s1_off, g.p2_off, g.s2_off, g.p3_off, g.s3_off) == (
        0, 7340032, 7798784, 15138816, 15597568, 22937600)
    assert g.nbytes == 23396352
    assert k3moe.lib().k3g_expert_layout(256, 128).nbytes == 52224


def test_tiled_sizes():
    L = k3moe.lib()
    # an MXFP4 matrix keeps its size when the columns are a multiple of 512
    assert L.k3g_tiled_mxfp4_bytes(2048, 7168) == 2048 * 7168 * 17 // 32
    assert L.k3g_tiled_mxfp4_bytes(7168, 2048) == 7168 * 2048 * 17 // 32
    # padded to 512 columns otherwise; unsupported shapes are 0
    assert L.k3g_tiled_mxfp4_bytes(128, 256) == 8 * 1 * 4352
    assert L.k3g_tiled_mxfp4_bytes(100, 256) == 0
    assert L.k3g_tiled_mxfp4_bytes(128, 48) == 0
    assert L.k3g_tiled_bf16_bytes(2048, 7168) == 2048 * 7168 * 2
    assert L.k3g_tiled_bf16_bytes(2048, 100) == 0


M64 = (1 << 64) - 1
GOLDEN_GAMMA = 0x9E3779B97F4A7C15


def _mix64(z):
    """the splitmix64 finaliser (Steele, Lea, Flood, OOPSLA 2014)"""
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def _word(seed, stream, w):
    key = _mix64((seed + GOLDEN_GAMMA * (stream + 1)) & M64)
    return _mix64((key + GOLDEN_GAMMA * (w + 1)) & M64)


def test_synthetic_bytes_are_the_documented_hash():
    """k3s_byte(seed, stream, i): byte i % 8 of the 64-bit word i / 8 of the counter hash,
    so any slice of a device-generated tensor can be regenerated on the host."""
    L = k3moe.lib()
    a = k3moe.host_bytes(64, 7, 3)
    b = np.array([L.k3s_byte(7, 3, i) for i in range(64)], np.uint8)
    assert np.array_equal(a, b)
    c = np.array([(_word(7, 3, i >> 3) >> (8 * (i & 7))) & 0xFF for i in range(64)], np.uint8)
    assert np.array_equal(a, c)
    # a window starting mid-stream equals the same window of the whole stream
    assert np.array_equal(k3moe.host_bytes(16, 7, 3, first=40), a[40:56])
    # different streams and seeds differ
    assert not np.array_equal(a, k3moe.host_bytes(64, 7, 4))
    assert not np.array_equal(a, k3moe.host_bytes(64, 8, 3))


def test_synthetic_scales_and_normals():
    s = k3moe.host_scales(4096, 1, 2, -4, 2)
    assert s.min() >= 123 and s.max() <= 129
    assert len(np.unique(s)) == 7
    x = k3moe.host_normal(1 << 16, 5, 6, 0.0, 1.0)
    assert abs(float(x.mean())) < 0.02 and abs(float(x.std()) - 1.0) < 0.02
    xb = k3moe.host_normal(1024, 5, 6, 0.0, 1.0, bf16=True)
    assert np.all((xb.view(np.uint32) & 0xFFFF) == 0)      # bf16-valued


def test_moe_scratch_matches_the_engine_formula():
    """k3_moe_scratch = 2L + 3I + L + 3SI + d floats (src/core/k3_ops.c:658-666)."""
    lay = k3moe.SynthLayer(k3moe.TINY, seed=1, device=False)
    cfg = lay.cfg()
    L_, I, SI, d = cfg.latent, cfg.moe_inter, cfg.moe_inter * cfg.n_shared, cfg.hidden
    assert k3moe.lib().k3_moe_scratch(C.byref(cfg)) == 2 * L_ + 3 * I + L_ + 3 * SI + d
