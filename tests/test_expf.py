"""The engine's float expf as the device computes it (kimi-k3-in-rust_amd/csrc/k3g_expf.h):
the router scores, their selection and the SiTU/SwiGLU gate all pass through
expf (src/core/k3_ops.c:105, :446-458), and the engine's is the C library's (glibc), which
is not correctly rounded. The restatement is compiled for the host and compared with this
machine's expf on every one of the 2^32 float inputs, and its table of 2^(i/32) with the
powers computed to 60 digits. A correctly rounded expf (what the device used before) is
shown to disagree with the library: the test that the restatement is needed."""
import math
import os
import shutil
import struct
import subprocess
from decimal import Decimal, getcontext

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "kimi-k3-in-rust_amd", "csrc")
HOST = os.path.join(ROOT, "tests", "host")


@pytest.fixture(scope="module")
def audit(tmp_path_factory):
    if not shutil.which("gcc"):
        pytest.skip("no host compiler")
    d = tmp_path_factory.mktemp("expf_audit")
    exe = d / "expf_audit"
    subprocess.run(["gcc", "-O2", "-std=gnu99", "-fopenmp", "-ffp-contract=off", "-I", CSRC,
                    os.path.join(HOST, "expf_audit.c"), "-o", str(exe), "-lm"], check=True)
    return str(exe)


def test_table_is_two_to_the_i_over_32(audit):
    getcontext().prec = 60
    out = subprocess.run([audit, "table"], capture_output=True, text=True, check=True).stdout
    tab = [int(l, 16) for l in out.split()]
    assert len(tab) == 32
    for i, t in enumerate(tab):
        p = float(Decimal(2) ** (Decimal(i) / Decimal(32)))   # correctly rounded to double
        bits = struct.unpack("<Q", struct.pack("<d", p))[0]
        assert (t + (i << 47)) & (2 ** 64 - 1) == bits, i


def test_every_float_matches_the_c_library(audit):
    r = subprocess.run([audit], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout
    assert "mismatches 0" in r.stdout


def test_correct_rounding_is_not_the_engine():
    """The device's former expf, (float)exp((double)x), against the C library on a range of
    router logits: they disagree (the case the full-size router test met: logit
    0.85176116 of token 2527)."""
    import ctypes as C
    libm = C.CDLL("libm.so.6")
    libm.expf.restype, libm.expf.argtypes = C.c_float, [C.c_float]
    x = np.float32(-0.85176116)
    assert np.float32(libm.expf(C.c_float(x))) != np.float32(math.exp(float(x)))
    xs = np.random.default_rng(5).standard_normal(20000).astype(np.float32)
    diff = sum(np.float32(libm.expf(C.c_float(v))) != np.float32(math.exp(float(v))) for v in xs)
    assert diff > 0
