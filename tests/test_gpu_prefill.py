"""GPU parity of the batched prompt prefill (no reference counterpart: the
reference forwards prompt tokens one at a time, inference.rs:580-592).

* rf_matmul_packed: every token row equals the oracle's matvec of that token
  (quant.rs:898-1327 restated) within 1e-4 scaled relative error, and the
  float64 product of the decoded matrix within 256 * 2^-24 of the row's term
  magnitude sum_j |w_ij x_j| (f32-level accuracy of the bf16 three-piece
  split on the matrix cores).
* rf_model_prefill: the last token's output-normed hidden state and logits
  are within 2e-4 of the oracle's token-by-token forward (the reference's
  own forward-test EPS, inference.rs:2508), and the greedy tokens generated
  after a batched prompt equal the oracle's.
"""
import numpy as np
import pytest

from helpers import F32, GEOM, NAMES, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, assert_close_scaled, pack_host, random_matrix
from test_gpu_model import ALL_Q4, ALL_Q8, MIXED, TINY, _load_gpu, _tiny_tensors

pytestmark = pytest.mark.gpu
TOL = 1e-4
PACKED = [Q8_0, Q4_0, Q4_K, Q6_K]


def _rf():
    import ramforge_amd as rf

    return rf


def _check_matmul(ctx, orc, t, out_dim, in_dim, n, seed, oracle_rows=3):
    rf = _rf()
    rng = np.random.default_rng(seed)
    raw = random_matrix(t, out_dim, in_dim, rng)
    x = rng.normal(0, 1, (n, in_dim)).astype(np.float32)
    print(f"  matmul {NAMES[t]} out={out_dim} in={in_dim} n={n} seed={seed}", flush=True)
    w = ctx.array(pack_host(t, raw, out_dim, in_dim))
    xd = ctx.array(x.reshape(-1))
    y = ctx.empty((n * out_dim,))
    rf.matmul_packed(ctx, t, w, (out_dim, in_dim), xd, n, y)
    got = y.numpy().reshape(n, out_dim)
    wdec = orc.dequantize_rows(t, raw, in_dim, out_dim).astype(np.float64)
    ref64 = x.astype(np.float64) @ wdec.T
    scale = np.abs(x.astype(np.float64)) @ np.abs(wdec).T
    assert np.all(np.abs(got - ref64) <= scale * 256 * 2.0 ** -24), NAMES[t]
    worst = 0.0
    for ti in sorted({0, n // 2, n - 1})[:oracle_rows]:
        ref = orc.dispatch_matvec(t, raw, in_dim, out_dim, x[ti], 16)
        worst = max(worst, assert_close_scaled(got[ti], ref, scale[ti], TOL, what=f"{NAMES[t]} token {ti}"))
    print(f"    scaled rel err vs oracle {worst:.2e}, vs float64 {np.max(np.abs(got - ref64) / scale):.2e}",
          flush=True)
    for a in (w, xd, y):
        a.free()


@pytest.mark.parametrize("t", PACKED)
@pytest.mark.parametrize("out_dim,in_dim,n", [(1, 256, 1), (67, 96, 5), (130, 1024, 16), (257, 4096, 33),
                                              (300, 2048, 64), (33, 3328, 17), (1000, 5120, 100),
                                              (4096, 4096, 64), (4096, 14336, 48), (14336, 4096, 7)])
def test_matmul_packed_matches_per_token_matvec(ctx, orc, t, out_dim, in_dim, n):
    """Ragged token counts (1 .. 100: one to four 16-token tiles, and two
    64-token chunks), rows not a multiple of the 128-row workgroup tile, k
    not a multiple of the 256-element slice (Q8_0 / Q4_0), and the 8B
    projection shapes."""
    if in_dim % GEOM[t][0]:
        pytest.skip(f"{NAMES[t]} rows are whole {GEOM[t][0]}-element blocks")
    _check_matmul(ctx, orc, t, out_dim, in_dim, n, 3100 + t + out_dim % 997 + n)


@pytest.mark.parametrize("t", PACKED)
def test_matmul_reduce_forms_agree(ctx, t):
    """The four-column split-K reduce (aligned output) and the one-column
    reduce (an output 4 bytes past alignment) give the same bits."""
    rf = _rf()
    rng = np.random.default_rng(3150 + t)
    out_dim, in_dim, n = 1024, 4096, 40
    raw = random_matrix(t, out_dim, in_dim, rng)
    w = ctx.array(pack_host(t, raw, out_dim, in_dim))
    x = ctx.array(rng.normal(0, 1, n * in_dim).astype(np.float32))
    y = ctx.empty((n * out_dim + 4,))
    rf.matmul_packed(ctx, t, w, (out_dim, in_dim), x, n, y.ptr)
    a = y.numpy()[: n * out_dim].copy()
    rf.matmul_packed(ctx, t, w, (out_dim, in_dim), x, n, y.ptr + 4)
    b = y.numpy()[1: n * out_dim + 1]
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), NAMES[t]
    for arr in (w, x, y):
        arr.free()


def test_matmul_packed_validation(ctx):
    rf = _rf()
    w = ctx.array(np.zeros(34 * 8, np.uint8))
    x = ctx.array(np.zeros(256, np.float32))
    y = ctx.empty((8,))
    with pytest.raises(rf.RamforgeError, match="does not support"):
        rf.matmul_packed(ctx, Q5_K, w, (1, 256), x, 1, y)
    with pytest.raises(rf.RamforgeError, match="not divisible"):
        rf.matmul_packed(ctx, Q8_0, w, (1, 48), x, 1, y)
    with pytest.raises(rf.RamforgeError, match="truncated"):
        rf.matmul_packed(ctx, Q8_0, w, (2, 256), x, 1, y, w_bytes=34 * 8 - 1)
    with pytest.raises(rf.RamforgeError, match="overflows"):
        rf.matmul_packed(ctx, Q8_0, w, (1 << 40, 1 << 30), x.ptr, 1, y.ptr)
    with pytest.raises(rf.RamforgeError, match="overflows"):
        rf.matmul_packed(ctx, Q8_0, w, (1, 256), x.ptr, 1 << 60, y.ptr)
    for a in (w, x, y):
        a.free()


KQ_CFG = dict(TINY, embedding_length=256, feed_forward_length=512, head_dim=64, context_length=256)
# head_dim 64: the split attention kernel, which the batched prefill needs
# (with head_dim 32 the model runs the any-shape kernel and prefill falls
# back to one forward per token)
PF_CFG = dict(TINY, context_length=256, head_dim=64)
ALL_KQ = dict(embd=Q4_K, out=Q6_K, q=Q4_K, k=Q4_K, v=Q6_K, o=Q4_K, gate=Q4_K, up=Q4_K, down=Q6_K)


@pytest.mark.parametrize("kind,history,plen", [("q8", 0, 1), ("q8", 0, 37), ("q8", 3, 64), ("q8", 0, 150),
                                               ("q4", 0, 70), ("mixed", 0, 40), ("kq", 2, 90), ("kq_bias", 0, 20),
                                               ("q8_bias", 2, 90), ("q8_attn0", 3, 150), ("kq_attn0", 0, 90)])
def test_prefill_matches_token_by_token(ctx, orc, kind, history, plen):
    """Prompt of plen tokens after `history` single-token forwards: hidden
    state and logits of the last token against the oracle, then greedy
    tokens from there.  150 and 90 tokens span several 64-token chunks; 64
    tokens at history 3 crosses the 64-position attention regime inside a
    chunk.  The matrix-core prefill attention runs every chunk (these
    contexts are below its default threshold); *_attn0: the decode split
    kernel with a token dimension instead.  Q, K and V of one weight type
    take RoPE and the K/V rows in their split-K reduce (q8, q4, q8_bias with
    Q/K/V biases); mixed types (kq, kq_bias) a launch of its own."""
    import ramforge_amd as rf

    old_attn = rf.tune_prefill_attention(0 if kind.endswith("_attn0") else 2)
    kind = kind.replace("_attn0", "")
    try:
        _prefill_case(ctx, orc, kind, history, plen)
    finally:
        rf.tune_prefill_attention(old_attn)


def _prefill_case(ctx, orc, kind, history, plen):
    types = {"q8": ALL_Q8, "q4": ALL_Q4, "mixed": MIXED, "kq": ALL_KQ, "kq_bias": ALL_KQ, "q8_bias": ALL_Q8}[kind]
    cfg = dict(PF_CFG) if kind in ("q8", "q4", "q8_bias") else dict(KQ_CFG)
    rng = np.random.default_rng(3300 + plen + history)
    T = _tiny_tensors(rng, cfg, types, bias=kind.endswith("_bias"))
    cap = history + plen + 24
    gm = _load_gpu(ctx, cfg, T, cap)
    om = orc.Model(cfg, T, kv_capacity=cap, threads=8)
    try:
        assert gm.paths()["batched_prefill"], "prefill fell back to one forward per token"
        prompt = [int(v) for v in rng.integers(0, cfg["vocab_size"], history + plen)]
        print(f"  prefill {kind} history={history} plen={plen}", flush=True)
        for p in range(history):
            gm.forward(prompt[p], p)
        h = gm.prefill(prompt[history:], want_hidden=True)
        assert gm.seq_len == history + plen
        hr = None
        for p, tok in enumerate(prompt):
            hr = om.forward(tok, p)
        assert np.max(np.abs(h - hr)) <= 2e-4 * max(1.0, np.abs(hr).max()), kind
        lg = gm.logits()
        lr = om.logits(hr)
        assert np.max(np.abs(lg - lr)) <= 2e-4 * max(1.0, np.abs(lr).max()), kind
        gm.reset()
        om.reset()
        gm.set_prefill(True)
        toks = gm.generate(prompt, 20)
        ref, margin = om.generate(prompt, 20)
        assert toks == ref, f"greedy divergence (min top-2 margin {margin.min():.3g})"
    finally:
        om.close()
        gm.close()


@pytest.mark.parametrize("qh,kvh,hd", [(4, 4, 64), (8, 1, 64), (8, 4, 128), (16, 2, 128), (4, 2, 64)])
def test_prefill_attention_gqa_shapes(ctx, qh, kvh, hd):
    """The matrix-core prefill attention (forced on every chunk) for every
    query-head group size it takes (1, 2, 4, 8) and head_dim 64 / 128: a
    150-token prompt after 70
    single-token forwards (position splits with chunk records and their
    merge, partial 16-token tiles) gives the hidden state and logits of the
    token-by-token forward within 2e-4 of their maximum, and so does the
    split kernel it replaces."""
    import ramforge_amd as rf

    cfg = dict(PF_CFG, head_count=qh, head_count_kv=kvh, head_dim=hd, embedding_length=max(128, qh * hd // 2),
               context_length=256)
    rng = np.random.default_rng(3500 + qh * 10 + kvh + hd)
    T = _tiny_tensors(rng, cfg, ALL_Q8)
    gm = _load_gpu(ctx, cfg, T, 240)
    prompt = [int(v) for v in rng.integers(0, cfg["vocab_size"], 220)]
    print(f"  prefill attention qh={qh} kvh={kvh} hd={hd}", flush=True)
    try:
        assert gm.paths()["batched_prefill"]
        gm.reset()
        href = None
        for p, t in enumerate(prompt):
            href = gm.forward(t, p, want_hidden=True)
        lref = gm.logits().copy()
        for mode in (2, 0):
            rf.tune_prefill_attention(mode)
            gm.reset()
            for p in range(70):
                gm.forward(prompt[p], p)
            h = gm.prefill(prompt[70:], want_hidden=True)
            lg = gm.logits()
            assert np.max(np.abs(h - href)) <= 2e-4 * max(1.0, np.abs(href).max()), (mode, qh, kvh, hd)
            assert np.max(np.abs(lg - lref)) <= 2e-4 * max(1.0, np.abs(lref).max()), (mode, qh, kvh, hd)
    finally:
        rf.tune_prefill_attention(1)
        gm.close()


def test_prefill_attention_past_threshold_small_chunks(ctx):
    """Chunks of 1 and 17 tokens after 1030 positions (the default mode runs
    the matrix-core prefill attention there): hidden state and logits equal
    the token-by-token forward's within 2e-4 of their maximum."""
    cfg = dict(PF_CFG, context_length=1100)
    rng = np.random.default_rng(3600)
    T = _tiny_tensors(rng, cfg, ALL_Q8)
    gm = _load_gpu(ctx, cfg, T, 1100)
    prompt = [int(v) for v in rng.integers(0, cfg["vocab_size"], 1048)]
    try:
        assert gm.paths()["batched_prefill"]
        gm.reset()
        ref = {}
        for p, t in enumerate(prompt):
            h = gm.forward(t, p, want_hidden=p in (1030, 1047))
            if p in (1030, 1047):
                ref[p] = (h, gm.logits().copy())
        gm.reset()
        for p in range(1030):
            gm.forward(prompt[p], p)
        for end in (1031, 1048):
            h = gm.prefill(prompt[gm.seq_len:end], want_hidden=True)
            hr, lr = ref[end - 1]
            assert np.max(np.abs(h - hr)) <= 2e-4 * max(1.0, np.abs(hr).max()), end
            lg = gm.logits()
            assert np.max(np.abs(lg - lr)) <= 2e-4 * max(1.0, np.abs(lr).max()), end
    finally:
        gm.close()


def test_prefill_then_device_decode_graph(ctx, orc):
    """A batched prompt followed by graph-replayed device decode steps gives
    the tokens of the host generate loop with a token-by-token prompt."""
    cfg = dict(PF_CFG)
    rng = np.random.default_rng(3400)
    T = _tiny_tensors(rng, cfg, ALL_Q8)
    gm = _load_gpu(ctx, cfg, T, 200)
    try:
        assert gm.paths()["batched_prefill"]
        prompt = [int(v) for v in rng.integers(0, cfg["vocab_size"], 45)]
        ref = gm.generate(prompt, 41)
        gm.reset()
        gm.prefill(prompt)
        gm.use_graph(True)
        gm.decode_steps(40)
        got = gm.read_tokens(40)
        assert got == ref[:40]
        gm.use_graph(False)
    finally:
        gm.close()


def test_prefill_falls_back_for_unpacked_weights(ctx, orc):
    """With packing disabled the projections stay in GGUF layout and the
    prefill runs the token-by-token forward: bit-identical hidden state."""
    rf = _rf()
    cfg = dict(PF_CFG, context_length=128)
    rng = np.random.default_rng(3500)
    T = _tiny_tensors(rng, cfg, ALL_Q8)
    prompt = [int(v) for v in rng.integers(0, cfg["vocab_size"], 12)]
    old = rf.tune_packed_weights(-1)
    rf.tune_packed_weights(0)
    try:
        gm = _load_gpu(ctx, cfg, T, 32)
        assert not gm.paths()["batched_prefill"]
        h = gm.prefill(prompt, want_hidden=True)
        gm.reset()
        hr = None
        for p, tok in enumerate(prompt):
            hr = gm.forward(tok, p, want_hidden=True)
        assert np.array_equal(h.view(np.uint32), hr.view(np.uint32))
        gm.close()
    finally:
        rf.tune_packed_weights(old)


def test_prefill_validation(ctx):
    rf = _rf()
    cfg = dict(TINY, context_length=64)
    T = _tiny_tensors(np.random.default_rng(3600), cfg, ALL_Q8)
    gm = _load_gpu(ctx, cfg, T, 16)
    try:
        with pytest.raises(rf.RamforgeError, match="KV cache full"):
            gm.prefill([1] * 17)
        with pytest.raises(rf.RamforgeError, match="out of bounds"):
            gm.prefill([1, 2, cfg["vocab_size"]])
        assert gm.seq_len == 0
        gm.prefill([1, 2, 3])
        assert gm.seq_len == 3
    finally:
        gm.close()


def test_prefill_streaming_model(ctx, orc):
    """Layer streaming: a batched prompt loads each layer once per 64-token
    chunk, gives the resident model's tokens and hands its workspace back
    (the layer cache may use that VRAM while decoding)."""
    cfg = dict(PF_CFG)
    rng = np.random.default_rng(3700)
    T = _tiny_tensors(rng, cfg, ALL_Q8)
    prompt = [int(v) for v in rng.integers(0, cfg["vocab_size"], 80)]
    gm = _load_gpu(ctx, cfg, T, 128)
    ref = gm.generate(prompt, 10)
    gm.close()
    rf = _rf()
    sm = rf.GpuLlamaModel(ctx, cfg, 128)
    try:
        sm.enable_streaming(0)
        for name, (t, ne0, ne1, arr) in T.items():
            sm.set_tensor(name, t, ne0, ne1, arr)
        used = ctx.vram_used
        assert sm.paths()["batched_prefill"]
        sm.prefill(prompt)
        # no layer cache: every layer and the prefill workspace are released again
        assert ctx.vram_used == used
        sm.reset()
        sm.set_prefill(True)
        assert sm.generate(prompt, 10) == ref
    finally:
        sm.close()


def test_prefill_evicts_cached_layers_for_its_workspace():
    """A streaming model whose layer cache has filled the budget makes room
    for the batched prefill's workspace by evicting cached layers (as a KV
    growth does, ensure_layer_cache_headroom, streaming_model.rs:555-572)
    instead of failing, and gives the tokens of the same model with room to
    spare."""
    from test_gpu_model import STREAM_CFG, STREAM_TYPES

    rf = _rf()
    cfg = dict(STREAM_CFG, context_length=256)
    T = _tiny_tensors(np.random.default_rng(3800), cfg, STREAM_TYPES)
    prompt = [int(v) for v in np.random.default_rng(3801).integers(0, cfg["vocab_size"], 70)]

    def model(c):
        m = rf.GpuLlamaModel(c, cfg, 128)
        m.enable_streaming(1 << 30)
        for name, (t, ne0, ne1, arr) in T.items():
            m.set_tensor(name, t, ne0, ne1, arr)
        return m

    pctx = rf.Context(0, 0)
    pm = model(pctx)
    pm.generate([1, 2, 3], 4)  # token by token: every layer cached, no prefill workspace
    cached = pctx.vram_used
    assert pm.paths()["batched_prefill"]
    pm.reset()
    pm.prefill(prompt)
    ws = pctx.vram_peak - cached
    pm.reset()
    pm.set_prefill(True)
    ref = pm.generate(prompt, 12)
    pm.close()
    pctx.close()
    assert ws > 0
    budget = cached + ws // 2  # the cached layers fit, the workspace beside them does not
    sctx = rf.Context(0, budget)
    m = model(sctx)
    try:
        m.generate([1, 2, 3], 4)
        before = m.residency_stats()["evictions"]
        m.reset()
        m.set_prefill(True)
        assert m.generate(prompt, 12) == ref
        assert m.residency_stats()["evictions"] > before
        assert sctx.vram_peak <= budget
    finally:
        m.close()
        sctx.close()
