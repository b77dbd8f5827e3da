"""rf_matvec's repack cache (rf_matvec_cache): with it on, rf_matvec packs a
GGUF tensor once and runs the packed kernel on later calls.

Bars: every cached result equals rf_matvec_packed on the same tensor packed
by the caller, bit for bit (the same kernel on the same bytes), and the
oracle's matvec (quant.rs:898-1327) within the matvec bar of 1e-4 scaled.
"""
import numpy as np
import pytest

from helpers import (NAMES, Q4_0, Q4_K, Q5_0, Q6_K, Q8_0, assert_close_scaled, pack_host, random_matrix)

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _rf():
    import ramforge_amd as rf

    return rf


@pytest.fixture
def cctx():
    """A context of its own: the cache's entries and charges start empty."""
    rf = _rf()
    c = rf.Context(0)
    yield c
    c.close()


def _tensor(ctx, t, out_dim, in_dim, seed):
    rng = np.random.default_rng(seed)
    raw = random_matrix(t, out_dim, in_dim, rng)
    x = rng.normal(0, 1, in_dim).astype(np.float32)
    return raw, x, ctx.array(raw), ctx.array(x)


def _packed_ref(ctx, t, raw, out_dim, in_dim, xd, row_start=0, row_count=None):
    rf = _rf()
    p = ctx.array(pack_host(t, raw, out_dim, in_dim))
    n = out_dim - row_start if row_count is None else row_count
    y = ctx.empty((n,))
    rf.matvec_packed(ctx, t, p, (out_dim, in_dim), xd, y, row_start, row_count)
    out = y.numpy()
    p.free()
    y.free()
    return out


def _check_oracle(orc, t, raw, out_dim, in_dim, x, got, row_start=0):
    ref = orc.dispatch_matvec(t, raw, in_dim, out_dim, x, 16)[row_start:row_start + len(got)]
    wdec = orc.dequantize_rows(t, raw, in_dim, out_dim)[row_start:row_start + len(got)].astype(np.float64)
    scale = np.abs(wdec) @ np.abs(x.astype(np.float64))
    assert_close_scaled(got, ref, scale, TOL, what=f"cached {NAMES[t]} {out_dim}x{in_dim}")


@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K, Q6_K])
def test_cached_matvec_matches_packed_and_oracle(cctx, orc, t):
    rf = _rf()
    out_dim, in_dim = 300, 2048
    print(f"  repack cache {NAMES[t]} {out_dim}x{in_dim}", flush=True)
    raw, x, w, xd = _tensor(cctx, t, out_dim, in_dim, 40 + t)
    want = _packed_ref(cctx, t, raw, out_dim, in_dim, xd)
    cctx.matvec_cache(64 << 20)
    y = cctx.empty((out_dim,))
    for call in range(3):  # a miss, then hits
        y.upload(np.full(out_dim, np.nan, np.float32))
        rf.matvec(cctx, t, w, (out_dim, in_dim), xd, y)
        got = y.numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (NAMES[t], call)
    _check_oracle(orc, t, raw, out_dim, in_dim, x, got)
    st = cctx.matvec_cache_stats()
    assert st == {"entries": 1, "bytes": raw.nbytes, "hits": 2, "misses": 1}, st
    assert cctx.charge("workspace:repack:1") == raw.nbytes
    # a row range of the same tensor is served by the same entry
    ys = cctx.empty((37,))
    rf.matvec(cctx, t, w, (out_dim, in_dim), xd, ys, 101, 37)
    part = _packed_ref(cctx, t, raw, out_dim, in_dim, xd, 101, 37)
    assert np.array_equal(ys.numpy().view(np.uint32), part.view(np.uint32))
    assert cctx.matvec_cache_stats()["hits"] == 3
    used = cctx.vram_used
    cctx.matvec_cache(0)  # off: the copy is freed and its charge released
    assert cctx.vram_used == used - raw.nbytes
    assert cctx.matvec_cache_stats()["entries"] == 0
    for a in (w, xd, y, ys):
        a.free()


def test_cache_evicts_least_recently_used(cctx, orc):
    rf = _rf()
    t, out_dim, in_dim = Q8_0, 256, 1024
    tensors = [_tensor(cctx, t, out_dim, in_dim, 70 + i) for i in range(3)]
    size = tensors[0][0].nbytes
    cctx.matvec_cache(2 * size)  # room for two of the three
    y = cctx.empty((out_dim,))
    wants = [_packed_ref(cctx, t, raw, out_dim, in_dim, xd) for raw, _, _, xd in tensors]
    for order in ([0, 1, 2], [1, 2, 0], [0, 0, 2]):
        for i in order:
            raw, x, w, xd = tensors[i]
            rf.matvec(cctx, t, w, (out_dim, in_dim), xd, y)
            assert np.array_equal(y.numpy().view(np.uint32), wants[i].view(np.uint32)), (order, i)
            st = cctx.matvec_cache_stats()
            assert st["entries"] <= 2 and st["bytes"] <= 2 * size, st
    # calls: 0m 1m 2m(evicts 0) | 1h 2h 0m(evicts 1) | 0h 0h 2h
    assert cctx.matvec_cache_stats() == {"entries": 2, "bytes": 2 * size, "hits": 5, "misses": 4}
    _check_oracle(orc, t, tensors[2][0], out_dim, in_dim, tensors[2][1], y.numpy())
    cctx.matvec_cache(0)
    for raw, x, w, xd in tensors:
        w.free()
        xd.free()
    y.free()


def test_forget_after_the_weights_change(cctx, orc):
    rf = _rf()
    t, out_dim, in_dim = Q4_K, 64, 4096
    raw, x, w, xd = _tensor(cctx, t, out_dim, in_dim, 90)
    cctx.matvec_cache(64 << 20)
    y = cctx.empty((out_dim,))
    rf.matvec(cctx, t, w, (out_dim, in_dim), xd, y)
    _check_oracle(orc, t, raw, out_dim, in_dim, x, y.numpy())
    raw2 = random_matrix(t, out_dim, in_dim, np.random.default_rng(91))
    w.upload(raw2)
    # a range that overlaps the tensor's bytes drops its entry; one that does not keeps it
    cctx.matvec_cache_forget(w.ptr + raw.nbytes, 4096)
    assert cctx.matvec_cache_stats()["entries"] == 1
    cctx.matvec_cache_forget(w.ptr + 1000, 1)
    assert cctx.matvec_cache_stats()["entries"] == 0
    rf.matvec(cctx, t, w, (out_dim, in_dim), xd, y)
    _check_oracle(orc, t, raw2, out_dim, in_dim, x, y.numpy())
    assert cctx.matvec_cache_stats()["misses"] == 2
    cctx.matvec_cache(0)
    for a in (w, xd, y):
        a.free()


def test_uncacheable_calls_run_the_gguf_kernel(cctx, orc):
    rf = _rf()
    y = cctx.empty((512,))
    # a type without a packed layout
    raw, x, w, xd = _tensor(cctx, Q5_0, 96, 512, 120)
    cctx.matvec_cache(64 << 20)
    rf.matvec(cctx, Q5_0, w, (96, 512), xd, y)
    _check_oracle(orc, Q5_0, raw, 96, 512, x, y.numpy()[:96])
    # a tensor larger than the cache
    raw2, x2, w2, xd2 = _tensor(cctx, Q8_0, 512, 1024, 121)
    cctx.matvec_cache(raw2.nbytes - 1)
    rf.matvec(cctx, Q8_0, w2, (512, 1024), xd2, y)
    _check_oracle(orc, Q8_0, raw2, 512, 1024, x2, y.numpy())
    assert cctx.matvec_cache_stats()["entries"] == 0
    # fixed workspaces: no new entry (a miss would allocate)
    cctx.matvec_cache(64 << 20)
    cctx.reserve(fixed=True)
    rf.matvec(cctx, Q8_0, w2, (512, 1024), xd2, y)
    _check_oracle(orc, Q8_0, raw2, 512, 1024, x2, y.numpy())
    assert cctx.matvec_cache_stats() == {"entries": 0, "bytes": 0, "hits": 0, "misses": 0}
    for a in (w, xd, w2, xd2, y):
        a.free()


def test_cache_at_the_8b_shapes(cctx, orc):
    """The metric model's Q projection (4096x4096 Q8_0) and gate (14336 rows
    of 4096) shapes and a 14336-wide Q6_K, each hit after one miss."""
    rf = _rf()
    cctx.matvec_cache(1 << 30)
    for t, out_dim, in_dim, seed in ((Q8_0, 4096, 4096, 130), (Q8_0, 14336, 4096, 131), (Q6_K, 1024, 14336, 132)):
        print(f"  repack cache {NAMES[t]} {out_dim}x{in_dim}", flush=True)
        raw, x, w, xd = _tensor(cctx, t, out_dim, in_dim, seed)
        y = cctx.empty((out_dim,))
        rf.matvec(cctx, t, w, (out_dim, in_dim), xd, y)
        first = y.numpy()
        rf.matvec(cctx, t, w, (out_dim, in_dim), xd, y)
        assert np.array_equal(y.numpy().view(np.uint32), first.view(np.uint32))
        _check_oracle(orc, t, raw, out_dim, in_dim, x, first)
        cctx.matvec_cache_forget(w)  # before the weights are freed
        for a in (w, xd, y):
            a.free()
    assert cctx.matvec_cache_stats()["hits"] == 3


def test_graph_capture_uses_settled_entries(cctx, orc):
    rf = _rf()
    t, out_dim, in_dim = Q8_0, 512, 2048
    raw, x, w, xd = _tensor(cctx, t, out_dim, in_dim, 150)
    raw2, x2, w2, xd2 = _tensor(cctx, t, out_dim, in_dim, 151)
    want = _packed_ref(cctx, t, raw, out_dim, in_dim, xd)
    cctx.matvec_cache(64 << 20)
    y = cctx.empty((out_dim,))
    y2 = cctx.empty((out_dim,))
    rf.matvec(cctx, t, w, (out_dim, in_dim), xd, y)  # the miss packs w, outside the capture
    cctx.synchronize()
    with cctx.capture() as cap:
        rf.matvec(cctx, t, w, (out_dim, in_dim), xd, y)    # served from the cache
        rf.matvec(cctx, t, w2, (out_dim, in_dim), xd2, y2)  # a miss: no entry inside a capture
    g = cap.graph
    assert cctx.matvec_cache_stats() == {"entries": 1, "bytes": raw.nbytes, "hits": 1, "misses": 1}
    for rep in range(3):  # replays with eager work between them
        y.upload(np.full(out_dim, np.nan, np.float32))
        y2.upload(np.full(out_dim, np.nan, np.float32))
        g.replay(1)
        assert np.array_equal(y.numpy().view(np.uint32), want.view(np.uint32)), rep
        _check_oracle(orc, t, raw2, out_dim, in_dim, x2, y2.numpy())
    # dropping the entry makes the graph stale: replay is refused, not run
    cctx.matvec_cache_forget(w)
    with pytest.raises(rf.RamforgeError, match="repack cache"):
        g.replay(1)
    g.close()
    # a graph that captured no cached call is unaffected by drops
    with cctx.capture() as cap2:
        rf.matvec(cctx, t, w2, (out_dim, in_dim), xd2, y2)
    rf.matvec(cctx, t, w, (out_dim, in_dim), xd, y)
    cctx.matvec_cache(0)
    cap2.graph.replay(1)
    _check_oracle(orc, t, raw2, out_dim, in_dim, x2, y2.numpy())
    cap2.graph.close()
    for a in (w, xd, w2, xd2, y, y2):
        a.free()
