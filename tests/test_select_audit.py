"""The router's certified top-k (kimi-k3-in-rust_amd/csrc/k3g_select.h, the code the GPU
router and the fused decode kernel run) built for the host and run under AddressSanitizer,
UndefinedBehaviorSanitizer and the strict array-bounds checker, one emulated 64-lane wave
per token (tests/host/k3g_dev_host.h), with every token's routing compared bit for bit
with the oracle's k3_router restatement (src/core/k3_ops.c:419-478).

The sweep covers expert counts up to the selection's limit (1024), top-k up to the engine's
K3_MAX_TOPK (64, also above n_experts), exact ties in the choice scores (duplicated router
rows and biases, which fail the certificate and run the exact path), both exact-path
variants (LDS-staged candidate rows as the router kernel runs it, unstaged as the fused
decode kernel runs it) and the four forced modes. Any out-of-bounds access to the LDS
arrays, the score intervals, the router rows or the outputs aborts the run.

The many-token selection (k3d_pick_token, run by k_router_pick after the bounded bf16
logits) is audited the same way (tests/host/pick_audit.cpp): approximate logits placed
adversarially inside their bound (0.9 of it, up for odd experts and down for even ones,
rounded to float), with the bound the GPU path uses and a 200 times tighter one, in the
normal and two forced modes."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "kimi-k3-in-rust_amd", "csrc")
HOST = os.path.join(ROOT, "tests", "host")

CASES = [(E, k, ties) for E in (16, 384, 1024) for k in (1, 8, 64) for ties in (0, 1)] + [
    (896, 16, 1), (384, 16, 0), (1024, 16, 1), (16, 4, 0), (384, 9, 1)]


@pytest.fixture(scope="module")
def audit(tmp_path_factory):
    if not shutil.which("g++") or not shutil.which("gcc"):
        pytest.skip("no host compiler")
    d = tmp_path_factory.mktemp("select_audit")
    shutil.copy(os.path.join(CSRC, "k3g_select.h"), d / "k3g_select.h")
    shutil.copy(os.path.join(HOST, "k3g_dev_host.h"), d / "k3g_dev.h")
    shutil.copy(os.path.join(CSRC, "k3g_expf.h"), d / "k3g_expf.h")
    san = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all"]
    subprocess.run(["gcc", "-O1", "-g", "-ffp-contract=off", *san, "-c",
                    os.path.join(ROOT, "oracle", "k3_oracle.c"), "-I",
                    os.path.join(ROOT, "include"), "-o", str(d / "oracle.o")], check=True)
    exe = d / "select_audit"
    subprocess.run(["g++", "-std=c++20", "-O1", "-g", "-ffp-contract=off", *san,
                    "-fsanitize=bounds-strict", "-Wno-attributes", "-I", str(d),
                    os.path.join(HOST, "select_audit.cpp"), str(d / "oracle.o"), "-o",
                    str(exe), "-lpthread"], check=True)
    return str(exe)


@pytest.mark.parametrize("E,k,ties", CASES)
def test_select_in_bounds_and_bit_exact(audit, E, k, ties):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1")
    r = subprocess.run([audit, str(E), str(k), "256", "2", str(ties), "11"],
                       capture_output=True, text=True, timeout=240, env=env)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    lines = [l for l in r.stdout.splitlines() if l.startswith("E=")]
    assert len(lines) == 8, r.stdout
    assert all(l.endswith("mismatches 0") for l in lines), r.stdout
    if ties and k == 8:
        # the duplicated rows put exact ties at the top-k boundary: the certificate fails
        # and the exact path picks the lower index, as the engine does
        assert all("force=0: rerouted 0" not in l for l in lines if "force=0" in l), r.stdout


@pytest.mark.parametrize("E,k,ties", [(384, 8, 0), (1024, 64, 1), (16, 4, 0)])
def test_unsettled_scores_never_become_weights(audit, E, k, ties):
    """Intervals whose bound spans several float ulps of the logit, with the best guess
    moved inside them: the certificate may still order the experts, but a selected score
    that is not settled is not the engine's (here each guess sits 0.7 of the bound from the
    true sum, several float ulps of the logit). Every such score is recomputed (or the
    token re-routed), and indices and weights come out bit-exact with the oracle."""
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1")
    r = subprocess.run([audit, str(E), str(k), "256", "2", str(ties), "5", "1"],
                       capture_output=True, text=True, timeout=240, env=env)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    lines = [l for l in r.stdout.splitlines() if l.startswith("E=")]
    assert len(lines) == 8, r.stdout
    assert all(l.endswith("mismatches 0") for l in lines), r.stdout
    for l in lines:
        if "force=0" in l:
            rer = int(l.split("rerouted ")[1].split(",")[0])
            rec = int(l.split("recomputed ")[1].split(",")[0])
            # each token either failed its certificate or had its k scores recomputed
            assert rer + rec // k >= 2 and rec % k == 0, l



@pytest.fixture(scope="module")
def pick_audit(tmp_path_factory):
    if not shutil.which("g++") or not shutil.which("gcc"):
        pytest.skip("no host compiler")
    d = tmp_path_factory.mktemp("pick_audit")
    shutil.copy(os.path.join(CSRC, "k3g_select.h"), d / "k3g_select.h")
    shutil.copy(os.path.join(HOST, "k3g_dev_host.h"), d / "k3g_dev.h")
    shutil.copy(os.path.join(CSRC, "k3g_expf.h"), d / "k3g_expf.h")
    san = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all"]
    subprocess.run(["gcc", "-O1", "-g", "-ffp-contract=off", *san, "-c",
                    os.path.join(ROOT, "oracle", "k3_oracle.c"), "-I",
                    os.path.join(ROOT, "include"), "-o", str(d / "oracle.o")], check=True)
    exe = d / "pick_audit"
    subprocess.run(["g++", "-std=c++20", "-O1", "-g", "-ffp-contract=off", *san,
                    "-fsanitize=bounds-strict", "-Wno-attributes", "-I", str(d),
                    os.path.join(HOST, "pick_audit.cpp"), str(d / "oracle.o"), "-o",
                    str(exe), "-lpthread"], check=True)
    return str(exe)


@pytest.mark.parametrize("E,k,ties,mode", [(384, 8, 0, 0), (384, 8, 1, 1), (16, 4, 1, 0),
                                           (1024, 64, 1, 0), (896, 16, 0, 1), (384, 9, 1, 0),
                                           (64, 1, 1, 1), (512, 16, 1, 0)])
def test_many_token_pick_bit_exact(pick_audit, E, k, ties, mode):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1")
    r = subprocess.run([pick_audit, str(E), str(k), "256", "3", str(ties), "13", str(mode)],
                       capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    lines = [l for l in r.stdout.splitlines() if l.startswith("E=")]
    assert len(lines) == 3, r.stdout
    assert all(l.endswith("violations 0, mismatches 0") for l in lines), r.stdout
    # forced mode 2 makes every expert a candidate: every token counts as having extras
    assert all("extra 3," in l for l in lines if "force=2" in l), r.stdout
