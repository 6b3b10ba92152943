"""Routed experts from safetensors shards into the HBM cache's host bank, on the CPU: the
index of the engine's own cache fixture (tests/fixtures/cache, 24 experts, 144 tensors)
and byte-exact runs in a bank; a synthetic checkpoint of the tiny layer (two shards, one
expert whose tensors are out of order, header entries shuffled, a __metadata__ entry) into
checkpoint-layout and tiled banks, against the runs it was written from and the tiled
layout written independently; and the loader's refusals."""
import json
import os
import struct

import numpy as np
import pytest

import k3moe
from safetensors_io import expert_tensors, write_shard

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURE = os.path.join(GOLDEN, "cache_fixture")


def _fixture_runs():
    """The fixture's expert runs, read independently from the file: for expert e the six
    tensors' bytes in the order w1.packed w1.scale w2.packed w2.scale w3.packed w3.scale."""
    raw = open(os.path.join(FIXTURE, "model-00001-of-00001.safetensors"), "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    head = json.loads(raw[8:8 + n])
    runs = {}
    for e in range(24):
        parts = []
        for w in ("w1", "w2", "w3"):
            for kind in ("weight_packed", "weight_scale"):
                o0, o1 = head[f"language_model.model.layers.0.block_sparse_moe.experts.{e}.{w}.{kind}"]["data_offsets"]
                parts.append(np.frombuffer(raw[8 + n + o0:8 + n + o1], np.uint8))
        runs[e] = np.concatenate(parts)
    return runs


def test_index_of_the_engine_fixture():
    st = k3moe.St(FIXTURE)
    assert st.count() == 144
    runs = _fixture_runs()
    for e in range(24):
        r = st.expert(0, e)
        assert r.contiguous == 1 and r.nbytes == 1632
        assert list(r.rows) == [8, 8, 8] and list(r.pcols) == [64, 64, 64]
        assert np.array_equal(st.read_run(r), runs[e])
    with pytest.raises(KeyError):
        st.expert(0, 24)
    with pytest.raises(KeyError):
        st.expert(1, 0)


@pytest.mark.parametrize("direct", [True, False])
def test_fixture_runs_with_and_without_o_direct(monkeypatch, direct):
    """Contiguous runs read with O_DIRECT (the enclosing 4096-byte window into an aligned
    buffer, src/io/k3_st.c:457-497) and with ordinary reads (K3GC_NO_DIRECT) give the same
    bytes: the fixture's 1632-byte runs start at offsets that are not 4096-aligned, so the
    window's padding is exercised. Where the filesystem refuses O_DIRECT the reader falls
    back and the bytes still match."""
    if not direct:
        monkeypatch.setenv("K3GC_NO_DIRECT", "1")
    st = k3moe.St(FIXTURE)
    if not direct:
        assert st.direct() == 0
    print(f"shards read with O_DIRECT: {st.direct()}")
    runs = _fixture_runs()
    assert any(st.expert(0, e).off % 4096 for e in range(24))
    for e in range(24):
        assert np.array_equal(st.read_run(st.expert(0, e)), runs[e]), e


def test_fixture_runs_into_a_bank_byte_exact():
    runs = _fixture_runs()
    bank = k3moe.Bank(1, 24, expert_bytes=1632, raw=True)
    bank.load(k3moe.St(FIXTURE), 0, 0, 1)
    for e in range(24):
        assert np.array_equal(bank.expert_bytes_of(0, e), runs[e]), e
    bank.free()


def _tile_py(packed, scales, rows, cols):
    """The tiled MXFP4 layout, block by block (the layout k3g_tile.hip defines)."""
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


@pytest.mark.parametrize("rows,cols", [(16, 32), (32, 96), (48, 1056)])
def test_host_tiler_matches_the_layout(rows, cols):
    packed = k3moe.host_bytes(rows * cols // 2, 3, 1).reshape(rows, cols // 2)
    scales = k3moe.host_scales(rows * cols // 32, 3, 2, -3, 3).reshape(rows, cols // 32)
    scales[0, 0] = 255
    assert np.array_equal(k3moe.tile_mxfp4_host(packed, scales, rows, cols),
                          _tile_py(packed, scales, rows, cols))


def write_checkpoint(d, layer_objs, scramble=(1, 5)):
    """Two shards for the given layers (checkpoint layers = their .layer): experts 0..7 in
    shard 1, 8..15 in shard 2; expert `scramble` = (layer, e) has its six tensors written
    in reverse order (not one run in the checkpoint order); header entries shuffled."""
    s1, s2 = [], []
    for lay in layer_objs:
        s = lay.shape
        for e in range(s.n_experts):
            t = expert_tensors(lay.layer, e, lay.expert_host(e), lay.geo, s.inter, s.hidden)
            if (lay.layer, e) == scramble:
                t = t[::-1]
            (s1 if e < 8 else s2).extend(t)
    rng = np.random.default_rng(1)
    for name, ts in (("model-00001-of-00002.safetensors", s1),
                     ("model-00002-of-00002.safetensors", s2)):
        order = [n for n, _ in ts]
        rng.shuffle(order)
        write_shard(os.path.join(d, name), ts, metadata={"format": "pt"}, header_order=order)


def test_synthetic_checkpoint_into_banks(tmp_path):
    layers = [k3moe.SynthLayer(k3moe.TINY, seed=88, layer=l, device=False) for l in range(2)]
    write_checkpoint(str(tmp_path), layers)
    st = k3moe.St(str(tmp_path))
    assert st.count() == 2 * 16 * 6
    assert st.expert(1, 5).contiguous == 0 and st.expert(1, 4).contiguous == 1
    assert st.expert(0, 3).shard == 0 and st.expert(0, 12).shard == 1
    d, I = 256, 128
    ck = k3moe.Bank(2, 16, d, I, k3moe.K3G_EXPERT_MXFP4)
    ck.load(st, 0, 0, 2)
    tb = k3moe.Bank(2, 16, d, I, k3moe.K3G_EXPERT_MXFP4_TILED)
    tb.load(st, 0, 0, 2)
    g = layers[0].geo
    for lay in layers:
        for e in range(16):
            run = lay.expert_host(e)
            assert np.array_equal(ck.expert_bytes_of(lay.layer, e), run), (lay.layer, e)
            want = np.concatenate([
                _tile_py(run[g.p1_off:g.s1_off].reshape(I, d // 2), run[g.s1_off:g.p2_off].reshape(I, d // 32), I, d),
                _tile_py(run[g.p3_off:g.s3_off].reshape(I, d // 2), run[g.s3_off:g.nbytes].reshape(I, d // 32), I, d),
                _tile_py(run[g.p2_off:g.s2_off].reshape(d, I // 2), run[g.s2_off:g.p3_off].reshape(d, I // 32), d, I)])
            assert np.array_equal(tb.expert_bytes_of(lay.layer, e), want), (lay.layer, e)
    # checkpoint layer 1 into bank layer 0
    one = k3moe.Bank(1, 16, d, I, k3moe.K3G_EXPERT_MXFP4)
    one.load(st, 1, 0, 1)
    assert np.array_equal(one.expert_bytes_of(0, 7), layers[1].expert_host(7))


def test_loader_refusals(tmp_path):
    lay = k3moe.SynthLayer(k3moe.TINY, seed=89, device=False)
    good = expert_tensors(0, 0, lay.expert_host(0), lay.geo, 128, 256)
    # a span that disagrees with its shape
    bad = str(tmp_path / "bad")
    os.makedirs(bad)
    write_shard(os.path.join(bad, "a.safetensors"), good)
    raw = bytearray(open(os.path.join(bad, "a.safetensors"), "rb").read())
    n = struct.unpack("<Q", raw[:8])[0]
    head = raw[8:8 + n].decode().replace('"shape": [128, 128]', '"shape": [128, 127]', 1)
    raw[8:8 + n] = head.encode()
    open(os.path.join(bad, "a.safetensors"), "wb").write(bytes(raw))
    with pytest.raises(RuntimeError):
        k3moe.St(bad)
    # experts missing: the bank wants 16, the shard has 1
    part = str(tmp_path / "part")
    os.makedirs(part)
    write_shard(os.path.join(part, "a.safetensors"), good)
    b = k3moe.Bank(1, 16, 256, 128, k3moe.K3G_EXPERT_MXFP4)
    with pytest.raises(RuntimeError):
        b.load(k3moe.St(part), 0, 0, 1)
    # an expert of another shape than the bank's
    b2 = k3moe.Bank(1, 1, 512, 128, k3moe.K3G_EXPERT_MXFP4)
    with pytest.raises(RuntimeError):
        b2.load(k3moe.St(part), 0, 0, 1)
    # no shards at all
    with pytest.raises(RuntimeError):
        k3moe.St(str(tmp_path))


def _raw_shard(path, header: str, data: bytes = b"", hlen=None):
    h = header.encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h) if hlen is None else hlen))
        f.write(h)
        f.write(data)


@pytest.mark.parametrize("case", ["negative_offset", "numel_overflow", "dim_past_int",
                                  "span_past_file", "header_length_wraps"])
def test_loader_refuses_crafted_headers(tmp_path, case):
    """Headers an untrusted shard could carry: an offset before the data section (a read
    into the header), a shape whose element count overflows 64 bits, a dimension past what
    the expert API's int holds, a span past the end of the file, and a header length that
    would wrap the size check. Each shard must be refused, not indexed."""
    d = str(tmp_path / case)
    os.makedirs(d)
    f = os.path.join(d, "a.safetensors")
    if case == "negative_offset":
        _raw_shard(f, '{"t": {"dtype": "U8", "shape": [16], "data_offsets": [-8, 8]}}', bytes(8))
    elif case == "numel_overflow":
        _raw_shard(f, '{"t": {"dtype": "U8", "shape": [2147483647, 2147483647, 2147483647], '
                      '"data_offsets": [0, 8]}}', bytes(8))
    elif case == "dim_past_int":
        _raw_shard(f, '{"t": {"dtype": "U8", "shape": [2147483648, 0], "data_offsets": [0, 0]}}')
    elif case == "span_past_file":
        _raw_shard(f, '{"t": {"dtype": "U8", "shape": [64], "data_offsets": [0, 64]}}', bytes(8))
    else:
        _raw_shard(f, '{"t": {"dtype": "U8", "shape": [8], "data_offsets": [0, 8]}}', bytes(8),
                   hlen=(1 << 64) - 1)
    with pytest.raises(RuntimeError):
        k3moe.St(d)


def _engine_st(path):
    import oracle as O
    io = O.engine_io()
    if io is None:
        pytest.skip("oracle/_ref was not built (the engine's k3_st.c fills the K3St)")
    st = k3moe.K3St()
    assert io.L.k3_st_open(C_byref(st), path.encode()) == 0
    return io, st


def C_byref(x):
    import ctypes
    return ctypes.byref(x)


def test_index_from_the_engines_own_k3st(tmp_path):
    """k3gc_st_from_engine over a K3St filled by the engine's k3_st_open (the index the
    engine hands k3_cache_init): every expert of the fixture and of a synthetic two-shard
    checkpoint (one expert out of order) resolves to the engine's k3_expert_ref geometry,
    and k3gc_st_read_run_into gives the engine's k3_expert_load bytes, through O_DIRECT
    into an aligned buffer (run at the returned pad) and ordinary reads otherwise."""
    import ctypes
    lay = k3moe.SynthLayer(k3moe.TINY, seed=5, layer=1, device=False)
    other = k3moe.SynthLayer(k3moe.TINY, seed=5, layer=0, device=False)
    from test_checkpoint import write_checkpoint
    write_checkpoint(str(tmp_path), [other, lay], scramble=(1, 5))
    checked = out_of_order = 0
    for path, layers, ne in ((FIXTURE, [0], 24), (str(tmp_path), [0, 1], 16)):
        io, est = _engine_st(path)
        ours = k3moe.St.from_engine(est)
        assert ours.count() == est.nt
        raw = np.zeros(1 << 20, np.uint8)
        a0 = (-raw.ctypes.data) % 4096
        aligned = raw[a0:a0 + (1 << 19)]
        for l in layers:
            for e in range(ne):
                r = k3moe.K3ExpertRef()
                assert io.L.k3_expert_ref(ctypes.byref(est), l, e, ctypes.byref(r)) == 0
                want = np.zeros(r.nbytes, np.uint8)
                assert io.L.k3_expert_load(ctypes.byref(est), ctypes.byref(r),
                                           want.ctypes.data) == r.nbytes
                g = ours.expert(l, e)
                # the engine calls a run contiguous when its six spans tile one window in
                # any order; this index only when they also come in the checkpoint order
                # (w1p w1s w2p w2s w3p w3s), reading the others as six spans in that order
                assert (g.shard, g.nbytes) == (r.shard, r.nbytes)
                assert g.contiguous <= r.contiguous
                if g.contiguous:
                    assert g.off == r.off
                for i in range(3):
                    assert (g.rows[i], g.pcols[i], g.p_bytes[i], g.s_bytes[i]) == \
                        (r.m[i].rows, r.m[i].pcols, r.m[i].p_bytes, r.m[i].s_bytes)
                canon = np.concatenate([want[o:o + n] for i in range(3) for o, n in
                                        ((r.m[i].p_off, r.m[i].p_bytes),
                                         (r.m[i].s_off, r.m[i].s_bytes))])
                pad = ours.read_run_into(g, aligned)
                assert np.array_equal(aligned[pad:pad + g.nbytes], canon), (l, e)
                unaligned = raw[a0 + 1:a0 + 1 + (1 << 18)]
                assert ours.read_run_into(g, unaligned) == 0
                assert np.array_equal(unaligned[:g.nbytes], canon)
                checked += 1
                out_of_order += r.contiguous and not g.contiguous
        ours.close()
        io.L.k3_st_close(ctypes.byref(est))
    assert checked == 24 + 32 and out_of_order == 1


def test_index_from_a_malformed_k3st_is_refused():
    """An engine index whose tensor points at a shard it does not have is refused."""
    import ctypes
    io, est = _engine_st(FIXTURE)
    t = ctypes.cast(est.t, ctypes.POINTER(ctypes.c_byte * 72))
    shard = ctypes.c_int.from_address(ctypes.addressof(t[3]) + 8)
    keep = shard.value
    shard.value = 7
    p = ctypes.c_void_p()
    assert k3moe.lib().k3gc_st_from_engine(ctypes.byref(p), ctypes.byref(est)) != 0
    shard.value = keep
    assert k3moe.lib().k3gc_st_from_engine(ctypes.byref(p), ctypes.byref(est)) == 0
    k3moe.lib().k3gc_st_close(p)
    io.L.k3_st_close(ctypes.byref(est))
