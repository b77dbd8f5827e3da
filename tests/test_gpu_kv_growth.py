"""KV cache growth on the device: the cache starts small and is reallocated
in 256-position chunks (KvCache::GROW_CHUNK_TOKENS and grow_to_with_budget,
kv_cache.rs:49, 297-356, as generate_impl uses them, inference.rs:478-496 and
666-687).  Checked: the same tokens as a cache allocated up front, the
reference's capacity sequence (prompt length, then multiples of 256 capped at
prompt + max_tokens), ledger charges that match the buffers, a refused growth
that leaves cache, charges and model usable, streamed layers evicted to make
room, and graph replay across a growth."""
import numpy as np
import pytest

from helpers import Q8_0
from test_gpu_model import ALL_Q8, REGIME5_CFG, STREAM_CFG, STREAM_TYPES, TINY, _tiny_tensors

pytestmark = pytest.mark.gpu

# head_dim 64: the split attention kernel (the any-shape kernel takes 32)
GCFG = dict(TINY, context_length=1024, head_dim=64)


def _rf():
    import ramforge_amd as rf

    return rf


def _kv_bytes(cfg, n):
    """Bytes of one of the K / V caches for n positions (all layers, f32)."""
    return cfg["block_count"] * n * cfg["head_count_kv"] * cfg["head_dim"] * 4


def _model(ctx, cfg, T, cap, initial=None, stream_bytes=None):
    m = _rf().GpuLlamaModel(ctx, cfg, cap, kv_initial=initial)
    if stream_bytes is not None:
        m.enable_streaming(stream_bytes)
    for name, (t, ne0, ne1, arr) in T.items():
        m.set_tensor(name, t, ne0, ne1, arr)
    return m


def test_generate_grows_in_256_chunks(ctx):
    T = _tiny_tensors(np.random.default_rng(1300), GCFG, ALL_Q8)
    prompt = [1, 2, 3, 4]
    fixed = _model(ctx, GCFG, T, 700)
    ref = fixed.generate(prompt, 250)
    fixed.decode_steps(10)
    ref_steps = fixed.read_tokens(10)
    fixed.close()

    m = _model(ctx, GCFG, T, 700, initial=1)
    assert m.kv_positions() == 1
    assert ctx.charge("kv_cache:k") == _kv_bytes(GCFG, 1) == ctx.charge("kv_cache:v")
    toks = m.generate(prompt, 250)
    assert toks == ref
    # the prompt's 4 positions exactly, then min(256, 4 + 250) at position 4
    assert m.kv_positions() == 254
    assert ctx.charge("kv_cache:k") == _kv_bytes(GCFG, 254) == ctx.charge("kv_cache:v")
    assert ctx.charge("kv_cache:k:growth") is None and ctx.charge("kv_cache:v:growth") is None
    # decode steps past the generate bound grow to the next multiple of 256
    m.decode_steps(10)
    assert m.read_tokens(10) == ref_steps
    assert m.kv_positions() == 512
    assert ctx.charge("kv_cache:k") == _kv_bytes(GCFG, 512)
    m.close()


def test_growth_refused_by_budget_changes_nothing(ctx):
    rf = _rf()
    T = _tiny_tensors(np.random.default_rng(1301), GCFG, ALL_Q8)
    probe = rf.Context(0)
    base = probe.vram_used
    pm = _model(probe, GCFG, T, 700, initial=16)
    pm.forward(3, 0)  # any workspace a forward allocates on first use
    need = probe.vram_used - base
    pm.close()
    probe.close()
    # room for the model with a 16-position cache and 100 more positions, not
    # for the 256-position replacement next to the old cache
    tctx = rf.Context(0, 0)
    budget = tctx.vram_used + need + 2 * _kv_bytes(GCFG, 100)
    tctx.close()
    tctx = rf.Context(0, budget)
    m = _model(tctx, GCFG, T, 700, initial=16)
    for p in range(16):
        m.forward(3 + p, p)
    used = tctx.vram_used
    with pytest.raises(rf.RamforgeError) as ei:
        m.forward(7, 16)
    assert ei.value.code == rf.RF_ERR_BUDGET and "failed to grow KV cache from 16 to 256" in str(ei.value)
    assert m.kv_positions() == 16 and m.seq_len == 16 and tctx.vram_used == used
    assert tctx.charge("kv_cache:k") == _kv_bytes(GCFG, 16)
    assert tctx.charge("kv_cache:k:growth") is None and tctx.charge("kv_cache:v:growth") is None
    # still usable within its capacity
    m.reset()
    a = m.forward(5, 0, want_hidden=True)
    m.close()
    ref = _model(ctx, GCFG, T, 16)
    b = ref.forward(5, 0, want_hidden=True)
    ref.close()
    assert np.allclose(a, b, rtol=0, atol=1e-6)
    tctx.close()


def test_growth_evicts_streamed_layers(ctx):
    """A streamed model whose layer cache fills the budget: the growth
    reservation evicts cached layers (ensure_layer_cache_headroom) instead of
    failing, and the tokens match a resident model with a fixed cache."""
    rf = _rf()
    cfg = dict(STREAM_CFG, context_length=1024)
    T = _tiny_tensors(np.random.default_rng(1302), cfg, STREAM_TYPES)
    prompt = [9, 8, 7]
    ref_m = _model(ctx, cfg, T, 600)
    ref = ref_m.generate(prompt, 200)
    ref_m.close()

    probe = rf.Context(0)
    base = probe.vram_used
    pm = _model(probe, cfg, T, 600, initial=3, stream_bytes=1 << 30)
    pm.generate(prompt, 2)  # every layer cached
    full = probe.vram_used - base
    pm.close()
    probe.close()
    # budget: the model with every layer cached and its cache, plus one
    # 203-position cache: the growth to 203 positions (old and new caches
    # both charged) fits only once cached layers are evicted
    sctx = rf.Context(0, 0)
    budget = sctx.vram_used + full + _kv_bytes(cfg, 203)
    sctx.close()
    sctx = rf.Context(0, budget)
    m = _model(sctx, cfg, T, 600, initial=3, stream_bytes=1 << 30)
    toks = m.generate(prompt, 200)
    st = m.residency_stats()
    assert toks == ref
    assert m.kv_positions() == 203
    assert st["evictions"] > 0, st
    assert sctx.charge("kv_cache:k") == _kv_bytes(cfg, 203)
    m.close()
    sctx.close()


def test_graph_replay_across_growth(ctx):
    """Decode-step graphs are dropped at a growth (they hold the old buffers)
    and captured again: the tokens equal eager steps on a fixed cache."""
    T = _tiny_tensors(np.random.default_rng(1303), GCFG, ALL_Q8)
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, GCFG["vocab_size"], 40)]
    fixed = _model(ctx, GCFG, T, 900)
    fixed.prefill(prompt)
    fixed.decode_steps(200)
    a = fixed.read_tokens(200)
    fixed.decode_steps(300)
    b = fixed.read_tokens(300)
    fixed.close()

    m = _model(ctx, GCFG, T, 900, initial=40)
    assert m.paths()["split_attention"]
    m.prefill(prompt)
    m.use_graph(True)
    m.decode_steps(200)
    assert m.kv_positions() == 256
    assert m.read_tokens(200) == a
    m.decode_steps(300)
    assert m.kv_positions() == 768
    assert m.read_tokens(300) == b
    m.close()


def test_graph_replay_across_growth_and_all_regimes(ctx):
    """The split kernel's five regimes (64 query / 16 KV heads, head_dim 64,
    capacity 1100: per KV head past 512 positions, longer chunks past 1024)
    on a cache that starts at the prompt's 40 positions and grows in
    256-position chunks while graph-replayed decode steps cross every growth
    and regime boundary: the tokens of eager steps on a cache allocated up
    front."""
    T = _tiny_tensors(np.random.default_rng(1304), REGIME5_CFG, ALL_Q8)
    prompt = [int(t) for t in np.random.default_rng(6).integers(0, REGIME5_CFG["vocab_size"], 40)]
    steps = (150, 250, 300, 200, 150, 9)  # ends at position 1099, the last slot of the capacity
    fixed = _model(ctx, REGIME5_CFG, T, 1100)
    fixed.prefill(prompt)
    want = []
    for k in steps:
        fixed.decode_steps(k)
        want.append(fixed.read_tokens(k))
    fixed.close()

    m = _model(ctx, REGIME5_CFG, T, 1100, initial=40)
    assert m.paths()["split_attention"]
    assert {m.paths(p)["regime"] for p in range(40, 40 + sum(steps))} == {0, 1, 2, 3, 4}
    m.prefill(prompt)
    m.use_graph(True)
    caps = []
    for k, w in zip(steps, want):
        m.decode_steps(k)
        assert m.read_tokens(k) == w
        caps.append(m.kv_positions())
    m.use_graph(False)
    assert caps == [256, 512, 768, 1024, 1100, 1100], caps
    m.close()
