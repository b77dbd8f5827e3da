"""Streamed layers read from a byte source by layer ranges (the device side
of load_layer's reads, streaming_model.rs:581-847, with the read plan of
layer_read.rs:6-160): a tiny model laid out as a GGUF-like file (tensors
32-byte aligned, layer by layer, with small gaps) gives the same hidden
states and tokens as the pinned-host streaming tier and the oracle; merged
ranges make one read per layer load; tensors larger than a staging buffer
are read in pieces; a failed read releases every charge of the load."""
import os

import numpy as np
import pytest

from helpers import BF16, F16
from test_gpu_model import STREAM_CFG, STREAM_TYPES, _half_tensors, _tiny_tensors

pytestmark = pytest.mark.gpu


def _rf():
    import ramforge_amd as rf

    return rf


def _layout(T, gap=16):
    """File image: non-block tensors first, then each layer's tensors in GGUF
    order, each start aligned to 32 bytes with `gap` spare bytes between."""
    names = [n for n in T if not n.startswith("blk.")] + [n for n in T if n.startswith("blk.")]
    off, spans = 0, {}
    for n in names:
        off = (off + 31) // 32 * 32
        nb = np.asarray(T[n][3]).nbytes
        spans[n] = (off, nb)
        off += nb + gap
    blob = np.full(off, 0xA5, np.uint8)  # filler where no tensor lies
    for n, (o, nb) in spans.items():
        blob[o:o + nb] = np.frombuffer(np.ascontiguousarray(T[n][3]).tobytes(), np.uint8)
    return blob, spans


def _sourced_model(ctx, cfg, T, source, staging, cache_bytes=1 << 30, cap=40):
    rf = _rf()
    m = rf.GpuLlamaModel(ctx, cfg, cap)
    m.enable_streaming(cache_bytes)
    m.set_reader(source, staging)
    spans = source.spans
    for name, (t, ne0, ne1, arr) in T.items():
        if name.startswith("blk."):
            o, nb = spans[name]
            m.set_tensor_source(name, t, ne0, ne1, o, nb)
        else:
            m.set_tensor(name, t, ne0, ne1, arr)
    return m


def _pinned_model(cfg, T, cache_bytes=1 << 30, cap=40):
    """The pinned-host streaming tier, in a context of its own (a context
    holds one model's charges)."""
    rf = _rf()
    m = rf.GpuLlamaModel(rf.Context(0), cfg, cap)
    m.enable_streaming(cache_bytes)
    for name, (t, ne0, ne1, arr) in T.items():
        m.set_tensor(name, t, ne0, ne1, arr)
    return m


@pytest.mark.parametrize("staging", [1 << 20, 4096], ids=["merged-ranges", "pieces"])
@pytest.mark.parametrize("kind", ["file", "buffer"])
def test_byte_source_matches_pinned_streaming(ctx, orc, tmp_path, staging, kind):
    rf = _rf()
    cfg = STREAM_CFG
    T = _tiny_tensors(np.random.default_rng(1400), cfg, STREAM_TYPES, bias=True)
    blob, spans = _layout(T)
    if kind == "file":
        path = tmp_path / "model.bin"
        blob.tofile(path)
        src = rf.ByteSource(str(path))
    else:
        src = rf.ByteSource(blob.tobytes())
    src.spans = spans
    # cache of 0 bytes: every layer is read again for every token
    sm = _sourced_model(ctx, cfg, T, src, staging, cache_bytes=0)
    pm = _pinned_model(cfg, T, cache_bytes=0)
    om = orc.Model(cfg, T, kv_capacity=40, threads=4)
    for pos, tok in enumerate([5, 17, 90, 3]):
        a = sm.forward(tok, pos, want_hidden=True)
        b = pm.forward(tok, pos, want_hidden=True)
        r = om.forward(tok, pos)
        assert np.array_equal(a, b), pos
        assert np.max(np.abs(a - r)) <= 2e-4 * max(1.0, np.abs(r).max()), pos
    st = sm.read_stats()
    nl = cfg["block_count"]
    layer_bytes = sum(nb for n, (o, nb) in spans.items() if n.startswith("blk."))
    if staging == 1 << 20:
        # each layer's tensors are one merged range: one read per layer load
        assert st["calls"] == 4 * nl, st
    else:
        assert st["calls"] > 4 * nl, st
    # merged reads include the gaps between a layer's tensors (<= 4 KiB each)
    assert 4 * layer_bytes <= st["bytes"] <= 4 * (layer_bytes + 16 * 12 * nl + 32 * 12 * nl)
    sm.reset()
    pm.reset()
    assert sm.generate([1, 2, 3], 12) == pm.generate([1, 2, 3], 12)
    for m in (sm, pm):
        m.close()
    pm.ctx.close()
    om.close()
    src.close()


@pytest.mark.parametrize("half", ["f16", "bf16"])
def test_byte_source_widens_half_weights(ctx, orc, half):
    """F16 / BF16 block tensors read from the source are widened on the device
    (tensor.rs:967-1014) into the same values the oracle decodes."""
    rf = _rf()
    t = {"f16": F16, "bf16": BF16}[half]
    cfg = dict(STREAM_CFG)
    T, R = _half_tensors(np.random.default_rng(1410 + t), cfg, t, orc)
    blob, spans = _layout(T)
    src = rf.ByteSource(blob.tobytes())
    src.spans = spans
    sm = _sourced_model(ctx, cfg, T, src, 1 << 20)
    om = orc.Model(cfg, R, kv_capacity=40, threads=4)
    for pos, tok in enumerate([7, 1, 33]):
        a = sm.forward(tok, pos, want_hidden=True)
        r = om.forward(tok, pos)
        assert np.max(np.abs(a - r)) <= 2e-4 * max(1.0, np.abs(r).max()), pos
    sm.close()
    om.close()


def test_failed_read_releases_the_load(ctx):
    rf = _rf()
    cfg = STREAM_CFG
    T = _tiny_tensors(np.random.default_rng(1420), cfg, STREAM_TYPES)
    blob, spans = _layout(T)
    src = rf.ByteSource(blob.tobytes())
    src.spans = spans
    m = _sourced_model(ctx, cfg, T, src, 1 << 20, cache_bytes=0)
    used = ctx.vram_used
    src.fail_at = spans["blk.2.ffn_up.weight"][0] + 10  # layer 2's range fails
    with pytest.raises(rf.RamforgeError) as ei:
        m.forward(4, 0)
    assert ei.value.code == rf.RF_ERR_IO and "layer 2" in str(ei.value)
    assert ctx.vram_used == used
    assert all(ctx.charge(f"layer:2:{s}") is None for s in ("attn_q.weight", "ffn_up.weight", "ffn_down.weight"))
    src.fail_at = None
    m.reset()
    h = m.forward(4, 0, want_hidden=True)
    pm = _pinned_model(cfg, T, cache_bytes=0)
    assert np.array_equal(h, pm.forward(4, 0, want_hidden=True))
    m.close()
    pm.close()
    pm.ctx.close()


def _layer_bytes(T, i):
    return sum(np.asarray(a).nbytes for n, (_, _, _, a) in T.items() if n.startswith(f"blk.{i}."))


@pytest.mark.parametrize("per_layer", [2, 3])
@pytest.mark.parametrize("read_ahead", [True, False])
def test_stream_units_from_file_source(ctx, tmp_path, read_ahead, per_layer):
    """Layer parts as streaming units (2: attention tensors with the norms |
    gate, up, down; 3: attention | gate, up | down) read from the library's
    file source, with and without read-ahead, through a cache of one and a
    half layers: hidden state and greedy tokens equal the pinned tier's with
    whole layers bit for bit, with fewer bytes uploaded."""
    rf = _rf()
    cfg = STREAM_CFG
    T = _tiny_tensors(np.random.default_rng(1460), cfg, STREAM_TYPES, bias=True)
    blob, spans = _layout(T)
    path = tmp_path / "model.bin"
    blob.tofile(path)
    cache = _layer_bytes(T, 0) * 3 // 2
    prompt = [5, 60, 2, 41]
    src = rf.FileSource(str(path), threads=2)
    src.spans = spans
    m = _sourced_model(ctx, cfg, T, src, 1 << 20, cache_bytes=cache)
    try:
        m.set_cache_policy(1)
        m.set_stream_units(per_layer)
        m.set_read_ahead(read_ahead)
        h = m.forward(prompt[0], 0, want_hidden=True)
        m.reset()
        toks = m.generate(prompt, 12)
        up_half = m.residency_stats()["uploaded_bytes"]
    finally:
        m.close()
        src.close()
    pm = _pinned_model(cfg, T, cache_bytes=cache)
    pm.set_cache_policy(1)
    hp = pm.forward(prompt[0], 0, want_hidden=True)
    pm.reset()
    tp = pm.generate(prompt, 12)
    up_whole = pm.residency_stats()["uploaded_bytes"]
    pm.close()
    pm.ctx.close()
    assert np.array_equal(h, hp)
    assert toks == tp
    assert up_half < up_whole, (up_half, up_whole)


@pytest.mark.parametrize("kind", ["file_source", "python_source"])
@pytest.mark.parametrize("cached_layers", [0, 2])
def test_read_ahead_matches_pinned_streaming(ctx, tmp_path, kind, cached_layers):
    """Read-ahead (the model's worker thread reads the next layer the pass
    will load into a pinned buffer of one layer while the pass queues the
    layers before it): every layer streamed each token, or two cached,
    through the library's file source (read-ahead on by default) and a
    Python source with read-ahead turned on.  Hidden states and greedy
    tokens equal the pinned tier's and the same source's without read-ahead
    bit for bit; the read-ahead buffer shows in the pinned host bytes."""
    rf = _rf()
    cfg = STREAM_CFG
    T = _tiny_tensors(np.random.default_rng(1450 + cached_layers), cfg, STREAM_TYPES, bias=True)
    blob, spans = _layout(T)
    path = tmp_path / "model.bin"
    blob.tofile(path)
    cache = cached_layers * _layer_bytes(T, 0)
    prompt = [7, 1, 33, 90]

    def run(read_ahead):
        src = rf.FileSource(str(path), threads=2) if kind == "file_source" else rf.ByteSource(blob.tobytes())
        src.spans = spans
        m = _sourced_model(ctx, cfg, T, src, 1 << 20, cache_bytes=cache)
        try:
            if kind == "python_source" or not read_ahead:
                m.set_read_ahead(read_ahead)
            before = m.host_bytes()
            h = m.forward(prompt[0], 0, want_hidden=True)
            m.reset()
            toks = m.generate(prompt, 12)
            return h, toks, m.host_bytes() - before
        finally:
            m.close()
            src.close()

    h1, t1, grown = run(True)
    h0, t0, grown0 = run(False)
    pm = _pinned_model(cfg, T, cache_bytes=cache)
    hp = pm.forward(prompt[0], 0, want_hidden=True)
    pm.reset()
    tp = pm.generate(prompt, 12)
    pm.close()
    pm.ctx.close()
    assert np.array_equal(h1, h0) and np.array_equal(h1, hp)
    assert t1 == t0 == tp
    assert grown >= _layer_bytes(T, 1) and grown0 == 0, (grown, grown0)


def test_read_ahead_failed_read_releases_the_load(ctx):
    """A read-ahead that fails is reported by the load that needs it
    (RF_ERR_IO naming the layer), with every charge of that load released;
    the model then runs normally."""
    rf = _rf()
    cfg = STREAM_CFG
    T = _tiny_tensors(np.random.default_rng(1460), cfg, STREAM_TYPES)
    blob, spans = _layout(T)
    src = rf.ByteSource(blob.tobytes())
    src.spans = spans
    m = _sourced_model(ctx, cfg, T, src, 1 << 20, cache_bytes=0)
    m.set_read_ahead(True)
    used = ctx.vram_used
    src.fail_at = spans["blk.2.ffn_up.weight"][0] + 10  # layer 2's range fails
    with pytest.raises(rf.RamforgeError) as ei:
        m.forward(4, 0)
    assert ei.value.code == rf.RF_ERR_IO and "layer 2" in str(ei.value)
    assert ctx.vram_used == used
    assert all(ctx.charge(f"layer:2:{s}") is None for s in ("attn_q.weight", "ffn_up.weight", "ffn_down.weight"))
    src.fail_at = None
    m.reset()
    h = m.forward(4, 0, want_hidden=True)
    pm = _pinned_model(cfg, T, cache_bytes=0)
    assert np.array_equal(h, pm.forward(4, 0, want_hidden=True))
    m.close()
    pm.close()
    pm.ctx.close()
    with pytest.raises(rf.RamforgeError, match="0 or 1"):
        m2 = _sourced_model(ctx, cfg, T, src, 1 << 20, cache_bytes=0)
        try:
            _rf()._lib.check(ctx.lib.rf_model_set_read_ahead(m2.handle, 7))
        finally:
            m2.close()
