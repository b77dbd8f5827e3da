"""GPU decode parity: the device-resident llama executor against the oracle's
restatement of forward_single_streaming / compute_logits / generate_impl.

Hidden states and logits are within 2e-4 of the oracle (the reference's own
GQA forward test uses EPS = 2e-4, inference.rs:2508); greedy token sequences
are identical."""
import numpy as np
import pytest

from helpers import F32, Q4_0, Q4_K, Q6_K, Q8_0, random_matrix

pytestmark = pytest.mark.gpu


def _rf():
    import ramforge_amd as rf

    return rf


TINY = dict(vocab_size=96, context_length=64, embedding_length=128, block_count=3, feed_forward_length=192,
            head_count=4, head_count_kv=2, head_dim=32, rms_eps=1e-5, rope_freq_base=10000.0)


def _tiny_tensors(rng, cfg, types, bias=False):
    d, f, V = cfg["embedding_length"], cfg["feed_forward_length"], cfg["vocab_size"]
    qd, kvd = cfg["head_count"] * cfg["head_dim"], cfg["head_count_kv"] * cfg["head_dim"]
    sig = {F32: 0.05, Q8_0: 0.3, Q4_0: 0.02, Q4_K: 0.002, Q6_K: 0.0004}
    T = {}

    def mat(name, t, ne0, ne1):
        T[name] = (t, ne0, ne1, random_matrix(t, ne1, ne0, rng, sig[t]))
        if t == F32:
            T[name] = (t, ne0, ne1, (rng.normal(0, 0.05, ne0 * ne1)).astype(np.float32))

    mat("token_embd.weight", types["embd"], d, V)
    mat("output.weight", types["out"], d, V)
    T["output_norm.weight"] = (F32, d, 1, rng.normal(1, 0.1, d).astype(np.float32))
    for i in range(cfg["block_count"]):
        p = f"blk.{i}."
        T[p + "attn_norm.weight"] = (F32, d, 1, rng.normal(1, 0.1, d).astype(np.float32))
        T[p + "ffn_norm.weight"] = (F32, d, 1, rng.normal(1, 0.1, d).astype(np.float32))
        for n, ne0, ne1, key in (("attn_q", d, qd, "q"), ("attn_k", d, kvd, "k"), ("attn_v", d, kvd, "v"),
                                 ("attn_output", qd, d, "o"), ("ffn_gate", d, f, "gate"), ("ffn_up", d, f, "up"),
                                 ("ffn_down", f, d, "down")):
            mat(p + n + ".weight", types[key], ne0, ne1)
        if bias:
            for n, w in (("attn_q", qd), ("attn_k", kvd), ("attn_v", kvd)):
                T[p + n + ".bias"] = (F32, w, 1, rng.normal(0, 0.3, w).astype(np.float32))
    return T


def _load_gpu(ctx, cfg, T, cap):
    rf = _rf()
    m = rf.GpuLlamaModel(ctx, cfg, cap)
    for name, (t, ne0, ne1, arr) in T.items():
        m.set_tensor(name, t, ne0, ne1, arr)
    return m


ALL_Q8 = dict(embd=Q8_0, out=Q8_0, q=Q8_0, k=Q8_0, v=Q8_0, o=Q8_0, gate=Q8_0, up=Q8_0, down=Q8_0)
MIXED = dict(embd=Q4_K, out=Q6_K, q=Q4_K, k=Q4_K, v=Q6_K, o=Q4_K, gate=Q4_K, up=Q6_K, down=Q4_0)
ALL_F32 = dict(embd=F32, out=F32, q=F32, k=F32, v=F32, o=F32, gate=F32, up=F32, down=F32)
ALL_Q4 = dict(embd=Q8_0, out=Q4_0, q=Q4_0, k=Q4_0, v=Q4_0, o=Q4_0, gate=Q4_0, up=Q4_0, down=Q4_0)


@pytest.fixture(params=["packed", "stream", "oneshot"])
def layout_mode(request):
    """packed: Q8_0/Q4_0 projections in the device-native layout (default);
    stream / oneshot: GGUF layout with the persistent or one-shot kernel."""
    rf = _rf()
    old_k, old_p = rf.tune_matvec_kernel(-1), rf.tune_packed_weights(-1)
    rf.tune_matvec_kernel(0 if request.param == "oneshot" else 1)
    rf.tune_packed_weights(1 if request.param == "packed" else 0)
    yield request.param
    rf.tune_matvec_kernel(old_k)
    rf.tune_packed_weights(old_p)


@pytest.mark.parametrize("kind,bias", [("q8", False), ("q4", False), ("mixed", True), ("f32", True)])
def test_tiny_model_forward_and_generate(ctx, orc, kind, bias, layout_mode):
    cfg = dict(TINY)
    types = {"q8": ALL_Q8, "q4": ALL_Q4, "mixed": MIXED, "f32": ALL_F32}[kind]
    if kind == "mixed":
        cfg.update(embedding_length=256, feed_forward_length=512, head_dim=64)
    rng = np.random.default_rng(900 + len(kind))
    T = _tiny_tensors(rng, cfg, types, bias)
    print(f"  tiny model {kind} bias={bias}", flush=True)
    gm = _load_gpu(ctx, cfg, T, 48)
    om = orc.Model(cfg, T, kv_capacity=48, threads=4)
    for pos, tok in enumerate([5, 17, 90, 3, 3, 41]):
        h = gm.forward(tok, pos, want_hidden=True)
        hr = om.forward(tok, pos)
        assert np.max(np.abs(h - hr)) <= 2e-4 * max(1.0, np.abs(hr).max()), (kind, pos)
        lg = gm.logits()
        lr = om.logits(hr)
        assert np.max(np.abs(lg - lr)) <= 2e-4 * max(1.0, np.abs(lr).max()), (kind, pos)
    gm.reset()
    om.reset()
    toks = gm.generate([1, 2, 3, 4], 20)
    ref, margin = om.generate([1, 2, 3, 4], 20)
    assert toks == ref, f"greedy divergence (min top-2 margin {margin.min():.3g})"
    assert gm.seq_len == 4 + 19
    gm.close()
    om.close()
    _rf().tune_matvec_kernel(1)


@pytest.mark.parametrize("digits", [2, 0], ids=["digit-planes", "float-x"])
@pytest.mark.parametrize("kind", ["q8", "q4"])
def test_tiny_model_digit_modes(ctx, orc, kind, digits):
    """The whole forward and greedy loop with every packed Q8_0 / Q4_0 launch
    taking x as digit planes (mode 2), and with float x everywhere (mode 0)."""
    rf = _rf()
    cfg = dict(TINY)
    types = {"q8": ALL_Q8, "q4": ALL_Q4}[kind]
    T = _tiny_tensors(np.random.default_rng(930 + digits), cfg, types, bias=True)
    old = rf.tune_matvec_digits(-1)
    rf.tune_matvec_digits(digits)
    print(f"  tiny model {kind}, digits mode {digits}", flush=True)
    try:
        gm = _load_gpu(ctx, cfg, T, 48)
        om = orc.Model(cfg, T, kv_capacity=48, threads=4)
        for pos, tok in enumerate([5, 17, 90, 3]):
            h = gm.forward(tok, pos, want_hidden=True)
            hr = om.forward(tok, pos)
            assert np.max(np.abs(h - hr)) <= 2e-4 * max(1.0, np.abs(hr).max()), (kind, pos)
            lr = om.logits(hr)
            assert np.max(np.abs(gm.logits() - lr)) <= 2e-4 * max(1.0, np.abs(lr).max()), (kind, pos)
        gm.reset()
        om.reset()
        toks = gm.generate([1, 2, 3, 4], 20)
        ref, margin = om.generate([1, 2, 3, 4], 20)
        assert toks == ref, f"greedy divergence (min top-2 margin {margin.min():.3g})"
        gm.close()
        om.close()
    finally:
        rf.tune_matvec_digits(old)


@pytest.mark.parametrize("mode", [1, 0], ids=["inflight", "ring"])
@pytest.mark.parametrize("kind", ["q8", "q4"])
def test_tiny_model_inflight_modes(ctx, orc, kind, mode):
    """The whole forward and greedy loop with the one-row-per-wavefront
    launches (mode 1: residual, RMSNorm and store epilogues) and with the
    two-step ring everywhere (mode 0)."""
    rf = _rf()
    cfg = dict(TINY)
    types = {"q8": ALL_Q8, "q4": ALL_Q4}[kind]
    T = _tiny_tensors(np.random.default_rng(950 + mode), cfg, types, bias=True)
    old = rf.tune_packed_inflight(-1)
    rf.tune_packed_inflight(mode)
    print(f"  tiny model {kind}, inflight mode {mode}", flush=True)
    try:
        gm = _load_gpu(ctx, cfg, T, 48)
        om = orc.Model(cfg, T, kv_capacity=48, threads=4)
        for pos, tok in enumerate([5, 17, 90, 3]):
            h = gm.forward(tok, pos, want_hidden=True)
            hr = om.forward(tok, pos)
            assert np.max(np.abs(h - hr)) <= 2e-4 * max(1.0, np.abs(hr).max()), (kind, pos)
        gm.reset()
        om.reset()
        toks = gm.generate([1, 2, 3, 4], 20)
        ref, margin = om.generate([1, 2, 3, 4], 20)
        assert toks == ref, f"greedy divergence (min top-2 margin {margin.min():.3g})"
        gm.close()
        om.close()
    finally:
        rf.tune_packed_inflight(old)


# Q6_K gate/up over an 8448-wide hidden state: x fills 43.5 KB of LDS, the
# size at which the packed matvec would use 1024-thread workgroups; the Q6_K
# gate/up kernel stays at 512 (its 1024-thread form spilled to scratch).
WIDE_CFG = dict(TINY, embedding_length=8448, feed_forward_length=256, block_count=1)
WIDE_Q6 = dict(ALL_Q8, gate=Q6_K, up=Q6_K)


def test_wide_hidden_q6k_gateup(ctx, orc):
    rng = np.random.default_rng(970)
    T = _tiny_tensors(rng, WIDE_CFG, WIDE_Q6)
    print("  wide hidden 8448, Q6_K gate/up", flush=True)
    gm = _load_gpu(ctx, WIDE_CFG, T, 16)
    om = orc.Model(WIDE_CFG, T, kv_capacity=16, threads=8)
    try:
        for pos, tok in enumerate([5, 17, 90, 3]):
            h = gm.forward(tok, pos, want_hidden=True)
            hr = om.forward(tok, pos)
            assert np.max(np.abs(h - hr)) <= 2e-4 * max(1.0, np.abs(hr).max()), pos
            # the output stage on the same input: the 8448-term projection
            # amplifies the hidden state's allowed difference past the bound
            lr = om.logits(h)
            assert np.max(np.abs(gm.logits() - lr)) <= 2e-4 * max(1.0, np.abs(lr).max()), pos
    finally:
        gm.close()
        om.close()


# Gate/up and down at the 8B FFN width (14336 rows / inputs) through the
# fused ffn RMSNorm + gate/up + SiLU*up and down + residual launches; on a
# 256-CU device gate/up leaves half of its wavefronts a fourth row.
FFN8B_CFG = dict(TINY, feed_forward_length=14336, block_count=1)


@pytest.mark.parametrize("kind", ["q8_0", "q4_0"])
def test_ffn_14336_width(ctx, orc, kind):
    types = ALL_Q8 if kind == "q8_0" else ALL_Q4
    T = _tiny_tensors(np.random.default_rng(975), FFN8B_CFG, types)
    print(f"  ffn 14336, {kind} gate/up", flush=True)
    gm = _load_gpu(ctx, FFN8B_CFG, T, 16)
    om = orc.Model(FFN8B_CFG, T, kv_capacity=16, threads=8)
    try:
        for pos, tok in enumerate([7, 40, 2, 88]):
            h = gm.forward(tok, pos, want_hidden=True)
            hr = om.forward(tok, pos)
            assert np.max(np.abs(h - hr)) <= 2e-4 * max(1.0, np.abs(hr).max()), pos
    finally:
        gm.close()
        om.close()


# d 4096 with the 14336 FFN: gate/up wavefronts hold 32 KiB of codes, so the
# fused ffn RMSNorm + gate/up + SiLU*up launch takes x as int8 digit planes.
DIGITS_CFG = dict(TINY, embedding_length=4096, feed_forward_length=14336, block_count=1)


def test_gateup_digit_planes(ctx, orc):
    rf = _rf()
    T = _tiny_tensors(np.random.default_rng(976), DIGITS_CFG, ALL_Q8)
    print("  d 4096, ffn 14336, Q8_0 gate/up on digit planes (mode 1)", flush=True)
    old = rf.tune_matvec_digits(-1)
    rf.tune_matvec_digits(1)
    gm = _load_gpu(ctx, DIGITS_CFG, T, 16)
    om = orc.Model(DIGITS_CFG, T, kv_capacity=16, threads=8)
    try:
        for pos, tok in enumerate([7, 40, 2]):
            h = gm.forward(tok, pos, want_hidden=True)
            hr = om.forward(tok, pos)
            assert np.max(np.abs(h - hr)) <= 2e-4 * max(1.0, np.abs(hr).max()), pos
    finally:
        rf.tune_matvec_digits(old)
        gm.close()
        om.close()


def test_model_create_validation(ctx):
    rf = _rf()
    used = ctx.vram_used
    bad = [(dict(TINY, head_dim=0), "non-zero"), (dict(TINY, head_count_kv=3), "divisible"),
           (dict(TINY, head_dim=33), "even"), (dict(TINY, vocab_size=1 << 25), "out of range"),
           (dict(TINY, block_count=1 << 17), "out of range"),
           (dict(TINY, embedding_length=1 << 25), "out of range")]
    for cfg, msg in bad:
        with pytest.raises(rf.RamforgeError, match=msg):
            rf.GpuLlamaModel(ctx, cfg, 16)
    with pytest.raises(rf.RamforgeError, match="context_length"):
        rf.GpuLlamaModel(ctx, TINY, TINY["context_length"] + 1)
    assert ctx.vram_used == used


def test_set_tensor_failure_rolls_back(ctx):
    """A set_tensor that fails after its buffer was charged (here: no room for
    the temporary packing copy) frees the buffer and drops the charge, so the
    same call can succeed later (load_layer's rollback rule,
    streaming_model.rs:581-847)."""
    rf = _rf()
    T = _tiny_tensors(np.random.default_rng(980), TINY, ALL_Q8)
    name, charge = "blk.0.attn_q.weight", "layer:0:attn_q.weight"
    t, ne0, ne1, arr = T[name]
    with rf.Context(0) as probe:
        pm = rf.GpuLlamaModel(probe, TINY, 16)
        base = probe.vram_used
        pm.close()
    with rf.Context(0, vram_budget_bytes=base + arr.nbytes + arr.nbytes // 2) as small:
        m = rf.GpuLlamaModel(small, TINY, 16)
        try:
            assert small.vram_used == base
            with pytest.raises(rf.RamforgeError, match="insufficient memory"):
                m.set_tensor(name, t, ne0, ne1, arr)
            assert small.vram_used == base
            assert small.charge(charge) is None
            old = rf.tune_packed_weights(-1)
            rf.tune_packed_weights(0)  # no packing copy: the tensor alone fits
            try:
                m.set_tensor(name, t, ne0, ne1, arr)
            finally:
                rf.tune_packed_weights(old)
            assert small.charge(charge) == arr.nbytes
        finally:
            m.close()


def test_counts_do_not_wrap_the_capacity_checks(ctx):
    """Step and token counts near 2^64 are refused by the capacity checks
    instead of wrapping past them (a wrapped check would let the decode write
    K/V rows past the end of the cache)."""
    import ctypes as C

    rf = _rf()
    gm = _load_gpu(ctx, TINY, _tiny_tensors(np.random.default_rng(990), TINY, ALL_Q8), 32)
    try:
        gm.forward(1, 0)
        with pytest.raises(rf.RamforgeError, match="KV cache full"):
            gm.decode_steps((1 << 64) - 1)
        p = np.array([1, 2], np.uint32)
        out = np.zeros(4, np.uint32)
        n = C.c_uint64(7)
        rc = ctx.lib.rf_model_generate(gm.handle, p.ctypes.data, 2, (1 << 64) - 1, -1, out.ctypes.data, C.byref(n))
        assert rc != 0 and n.value == 0 and not out.any()
        assert gm.seq_len == 1
    finally:
        gm.close()


def test_generate_stop_rules(ctx, orc):
    rng = np.random.default_rng(950)
    T = _tiny_tensors(rng, TINY, ALL_Q8)
    gm = _load_gpu(ctx, TINY, T, 64)
    full = gm.generate([7, 8], 12)
    gm.reset()
    eos = full[5]
    cut = gm.generate([7, 8], 12, eos=eos)
    assert cut == full[:full.index(eos)]
    gm.reset()
    rf = _rf()
    with pytest.raises(rf.RamforgeError, match="context length"):
        gm.generate([1] * 60, 10)
    gm.reset()
    with pytest.raises(rf.RamforgeError, match="position"):
        gm.forward(1, 3)
    gm.close()


def test_device_decode_steps_graph_replay_matches_eager(ctx):
    """rf_model_decode_steps (device-side argmax -> embedding -> forward, no
    host round-trip) with and without a captured hipGraph gives the greedy
    tokens of the host-driven loop; every replay is checked."""
    rng = np.random.default_rng(960)
    T = _tiny_tensors(rng, TINY, ALL_Q8)
    gm = _load_gpu(ctx, TINY, T, 64)
    ref = gm.generate([3, 1, 4, 1, 5], 25)
    for graph in (False, True):
        gm.reset()
        for p, t in enumerate([3, 1, 4, 1, 5]):
            gm.forward(t, p)
        gm.use_graph(graph)
        got = []
        for _ in range(6):  # several replays with host syncs between them
            gm.decode_steps(4)
            got += gm.read_tokens(4)
            ctx.synchronize()
        assert got[:24] == ref[:24], f"graph={graph}"
        gm.use_graph(False)
    gm.close()


REGIME_CFG = dict(TINY, context_length=256, embedding_length=256, feed_forward_length=512, head_dim=64)
# 64 KV heads: per query head up to 4 chunks (256 / 64 heads), so 8 wavefronts
# past 256 positions
REGIME2_CFG = dict(TINY, context_length=512, embedding_length=256, feed_forward_length=512, head_count=64,
                   head_count_kv=64, head_dim=64)
# 64 query / 16 KV heads (4:1 GQA, head_dim 64) at capacity 1100: per query
# head with 4 chunks up to 512 positions (4 then 8 wavefronts), then per KV
# head with 16 chunks of 64 positions up to 1024 and longer chunks beyond:
# all five regimes of the split kernel
REGIME5_CFG = dict(TINY, context_length=1100, embedding_length=256, feed_forward_length=512, head_count=64,
                   head_count_kv=16, head_dim=64)


@pytest.mark.parametrize("cfg,cap,steps,regimes",
                         [(REGIME_CFG, 160, (30, 40, 80), {0, 1}), (REGIME2_CFG, 320, (30, 40, 200, 40), {0, 1, 2}),
                          (REGIME5_CFG, 1100, (30, 40, 200, 300, 500, 20), {0, 1, 2, 3, 4})],
                         ids=["regimes-0-1", "regimes-0-1-2", "regimes-0-to-4"])
def test_decode_graphs_cross_the_attention_regimes(ctx, orc, cfg, cap, steps, regimes):
    """Decode from position 5 with graph replay across the attention launch
    regimes of the split kernel: one chunk per query head up to 64
    positions, then several chunks per query head (4 and 8 wavefronts), then
    chunks per KV head (64 positions with 4 wavefronts, longer with 8); each
    regime's graph is captured lazily.  The model must run the split kernel
    and visit the listed regimes; tokens equal the eager loop's and the
    oracle's."""
    rng = np.random.default_rng(961)
    T = _tiny_tensors(rng, cfg, ALL_Q8)
    prompt = [3, 1, 4, 1, 5]
    n = sum(steps)
    gm = _load_gpu(ctx, cfg, T, cap)
    om = orc.Model(cfg, T, kv_capacity=cap, threads=8)
    orc.set_parity_threads(8)
    try:
        assert gm.paths()["split_attention"], "the model fell back to the any-shape attention kernel"
        seen = {gm.paths(p)["regime"] for p in range(len(prompt), len(prompt) + n)}
        assert seen == regimes, seen
        ref = gm.generate(prompt, n)
        oref, margin = om.generate(prompt, n)
        first = next((i for i, (a, b) in enumerate(zip(ref, oref)) if a != b), None)
        assert ref == oref, f"eager vs oracle: first divergence at {first}, margin {margin[first]:.3g}"
        gm.reset()
        for p, t in enumerate(prompt):
            gm.forward(t, p)
        gm.use_graph(True)
        got = []
        for k in steps:
            gm.decode_steps(k)
            got += gm.read_tokens(k)
            ctx.synchronize()
        assert got == ref[:n]
        gm.use_graph(False)
    finally:
        orc.set_parity_threads(0)
        om.close()
        gm.close()


def test_config4_greedy_tokens_identical(ctx, orc):
    """random-init llama, 16 layers, d 2048, 32/8 heads,
    FFN 8192, vocab 32000, Q8_0 everywhere; 32-token random prompt, 128 greedy
    tokens.  Weights are generated on the device and, byte-identically, on the
    host for the oracle.  The prompt is forwarded token by token and, again,
    batched (rf_model_prefill)."""
    from ramforge_amd import synthetic as syn

    cfg = syn.CONFIG_4
    specs = syn.llama_specs(cfg, syn.Q8_0, seed=4)
    prompt = [int(t) for t in np.random.default_rng(4).integers(0, cfg["vocab_size"], 32)]
    print("  config4: building device model", flush=True)
    gm = syn.build_device_model(ctx, cfg, specs, kv_capacity=256)
    print("  config4: building host model", flush=True)
    T = orc.model_tensors(specs)
    orc.set_parity_threads(16)
    om = orc.Model(cfg, T, kv_capacity=256, threads=16)
    try:
        # hidden-state agreement on the first positions
        for pos in range(3):
            h = gm.forward(prompt[pos], pos, want_hidden=True)
            hr = om.forward(prompt[pos], pos)
            assert np.max(np.abs(h - hr)) <= 2e-4 * max(1.0, np.abs(hr).max())
        gm.reset()
        om.reset()
        print("  config4: GPU generate", flush=True)
        toks = gm.generate(prompt, 128)
        print("  config4: oracle generate", flush=True)
        ref, margin = om.generate(prompt, 128)
        first = next((i for i, (a, b) in enumerate(zip(toks, ref)) if a != b), None)
        assert toks == ref, f"first divergence at {first}, top-2 margin there {margin[first]:.3g}"
        # the same prompt through the batched prefill
        gm.reset()
        gm.set_prefill(True)
        ptoks = gm.generate(prompt, 128)
        first = next((i for i, (a, b) in enumerate(zip(ptoks, ref)) if a != b), None)
        assert ptoks == ref, f"batched prompt: first divergence at {first}"
    finally:
        orc.set_parity_threads(0)
        om.close()
        gm.close()


# ------------------------------------------------- residency tier (streaming)

STREAM_CFG = dict(TINY, block_count=4, embedding_length=256, feed_forward_length=512, head_dim=64)
STREAM_TYPES = dict(embd=Q8_0, out=Q6_K, q=Q8_0, k=Q4_K, v=Q4_0, o=Q8_0, gate=Q4_0, up=Q4_0, down=Q6_K)


def _layer_bytes(T, li):
    return sum(arr.nbytes for name, (t, ne0, ne1, arr) in T.items() if name.startswith(f"blk.{li}."))


def _streaming_model(cfg, T, budget, cache_bytes, cap=40):
    rf = _rf()
    ctx = rf.Context(0, budget)
    ctx.base_used = ctx.vram_used  # the context's own buffers
    m = rf.GpuLlamaModel(ctx, cfg, cap)
    m.enable_streaming(cache_bytes)
    for name, (t, ne0, ne1, arr) in T.items():
        m.set_tensor(name, t, ne0, ne1, arr)
    return ctx, m


def _resident_reference(ctx, cfg, T, prompt, n):
    gm = _load_gpu(ctx, cfg, T, 40)
    logits = []
    for p, tok in enumerate(prompt):
        gm.forward(tok, p)
        logits.append(gm.logits())
    gm.reset()
    toks = gm.generate(prompt, n)
    gm.close()
    return logits, toks


def test_streamed_layers_match_resident_model(ctx):
    """Layers streamed from pinned host memory through an LRU cache that holds
    one of four layers give bit-identical logits and tokens; charges follow
    load_layer / LayerCache naming; the ledger never exceeds the budget."""
    rng = np.random.default_rng(1234)
    T = _tiny_tensors(rng, STREAM_CFG, STREAM_TYPES, bias=True)
    prompt = [3, 14, 15, 92]
    ref_logits, ref_toks = _resident_reference(ctx, STREAM_CFG, T, prompt, 10)
    lb = max(_layer_bytes(T, i) for i in range(4))
    # persistent tensors, KV, activations and workspaces of this model, measured
    probe_ctx, probe = _streaming_model(STREAM_CFG, T, 0, 0)
    base = probe_ctx.vram_used
    probe.close()
    probe_ctx.close()
    budget = base + 2 * lb + 4096  # two layers in flight at once, at most
    sctx, sm = _streaming_model(STREAM_CFG, T, budget, lb)
    for p, tok in enumerate(prompt):
        sm.forward(tok, p)
        got = sm.logits()
        assert np.array_equal(got.view(np.uint32), ref_logits[p].view(np.uint32)), p
        cached = [i for i in range(4) if sctx.charge(f"cache:layer:{i}:attn_q.weight") is not None]
        active = [i for i in range(4) if sctx.charge(f"layer:{i}:attn_q.weight") is not None]
        assert len(cached) <= 1 and not active, (cached, active)
    sm.reset()
    assert sm.generate(prompt, 10) == ref_toks
    st = sm.residency_stats()
    passes = len(prompt) + len(prompt) + 9  # forwards before the reset, then generate (terminal forward skipped)
    assert st["hits"] + st["misses"] == 4 * passes
    assert st["evictions"] > 0 and st["uploaded_bytes"] >= st["misses"] * min(_layer_bytes(T, i) for i in range(4))
    assert sctx.vram_peak <= budget
    sm.close()
    assert sctx.vram_used == sctx.base_used
    sctx.close()


def test_next_use_policy_keeps_what_fits(ctx):
    """Policy 1 on the in-order layer scan: once the cache is full, the layers
    in it stay (hits every pass) and only the rest are re-uploaded; outputs
    are identical to the resident model."""
    rng = np.random.default_rng(1238)
    T = _tiny_tensors(rng, STREAM_CFG, STREAM_TYPES)
    prompt = [9, 8, 7]
    _, ref_toks = _resident_reference(ctx, STREAM_CFG, T, prompt, 8)
    lb = max(_layer_bytes(T, i) for i in range(4))
    sctx, sm = _streaming_model(STREAM_CFG, T, 0, 2 * lb)
    sm.set_cache_policy(1)
    assert sm.generate(prompt, 8) == ref_toks
    st = sm.residency_stats()
    passes = len(prompt) + 7
    assert st["cached_layers"] == 2
    assert st["misses"] == 4 + 2 * (passes - 1)  # first pass loads all, then two streamed layers per pass
    assert st["hits"] == 2 * (passes - 1)
    sm.close()
    sctx.close()


@pytest.mark.parametrize("per_layer", [2, 3])
def test_stream_units_match_resident_model(ctx, per_layer):
    """Layers streamed in parts (2: attention tensors with both norms | gate,
    up, down; 3: attention | gate, up | down) through an LRU cache of one and
    a half layers under a VRAM budget: bit-identical logits per forward and
    the same greedy tokens as the resident model; the batched prefill equals
    the whole-layer streamed one bit for bit; charges keep their per-tensor
    names; the ledger stays within the budget and returns to the model's own
    buffers."""
    rng = np.random.default_rng(1240)
    T = _tiny_tensors(rng, STREAM_CFG, STREAM_TYPES, bias=True)
    prompt = [3, 14, 15, 92]
    ref_logits, ref_toks = _resident_reference(ctx, STREAM_CFG, T, prompt, 10)
    lb = max(_layer_bytes(T, i) for i in range(4))
    probe_ctx, probe = _streaming_model(STREAM_CFG, T, 0, 0)
    base = probe_ctx.vram_used
    probe.close()
    probe_ctx.close()
    budget = base + 2 * lb + 4096
    sctx, sm = _streaming_model(STREAM_CFG, T, budget, lb + lb // 2)
    sm.set_stream_units(per_layer)
    names = ("attn_q.weight", "ffn_gate.weight", "ffn_down.weight")
    for p, tok in enumerate(prompt):
        sm.forward(tok, p)
        got = sm.logits()
        assert np.array_equal(got.view(np.uint32), ref_logits[p].view(np.uint32)), p
        active = [(i, n) for i in range(4) for n in names if sctx.charge(f"layer:{i}:{n}") is not None]
        assert not active, active
    cached = [(i, n) for i in range(4) for n in names if sctx.charge(f"cache:layer:{i}:{n}") is not None]
    assert cached, "nothing cached"
    sm.reset()
    assert sm.generate(prompt, 10) == ref_toks
    st = sm.residency_stats()
    passes = len(prompt) + len(prompt) + 9
    assert st["hits"] + st["misses"] == 4 * per_layer * passes  # units per layer and pass
    assert sctx.vram_peak <= budget
    sm.close()
    assert sctx.vram_used == sctx.base_used
    sctx.close()
    # batched prefill (its workspace needs more than that budget): the same
    # hidden state and logits as with whole layers
    sctx, sm = _streaming_model(STREAM_CFG, T, 0, lb + lb // 2)
    sm.set_stream_units(per_layer)
    h_half = sm.prefill(prompt, want_hidden=True)
    l_half = sm.logits()
    sm.set_stream_units(1)  # releases every resident unit
    assert not [(i, n) for i in range(4) for n in names
                if sctx.charge(f"cache:layer:{i}:{n}") is not None or sctx.charge(f"layer:{i}:{n}") is not None]
    sm.reset()
    h_whole = sm.prefill(prompt, want_hidden=True)
    assert np.array_equal(h_half.view(np.uint32), h_whole.view(np.uint32))
    assert np.array_equal(l_half.view(np.uint32), sm.logits().view(np.uint32))
    sm.close()
    sctx.close()


def test_stream_units_next_use_stream_fewer_bytes(ctx):
    """Next-use policy with a cache of two and a half layers: with whole
    layers two layers stream every pass; with two or three units per layer
    the cache also keeps part of a third layer, so fewer bytes are uploaded,
    with the resident model's tokens either way."""
    rng = np.random.default_rng(1241)
    T = _tiny_tensors(rng, STREAM_CFG, STREAM_TYPES)
    prompt = [9, 8, 7]
    _, ref_toks = _resident_reference(ctx, STREAM_CFG, T, prompt, 8)
    lb = max(_layer_bytes(T, i) for i in range(4))
    st = {}
    for k in (1, 2, 3):
        sctx, sm = _streaming_model(STREAM_CFG, T, 0, lb * 5 // 2)
        sm.set_cache_policy(1)
        sm.set_stream_units(k)
        assert sm.generate(prompt, 8) == ref_toks, k
        st[k] = sm.residency_stats()
        sm.close()
        sctx.close()
        print(f"  {k} units per layer: {st[k]}", flush=True)
    assert st[1]["cached_layers"] == 2
    for k in (2, 3):
        assert st[k]["cached_bytes"] > st[1]["cached_bytes"], k
        assert st[k]["uploaded_bytes"] < st[1]["uploaded_bytes"], k


def test_stream_units_validation(ctx):
    rf = _rf()
    rng = np.random.default_rng(1242)
    T = _tiny_tensors(rng, STREAM_CFG, STREAM_TYPES)
    gm = _load_gpu(ctx, STREAM_CFG, T, 40)
    with pytest.raises(rf.RamforgeError, match="layer streaming"):
        gm.set_stream_units(2)
    gm.close()
    sctx, sm = _streaming_model(STREAM_CFG, T, 0, 1 << 30)
    for bad in (0, 4):
        with pytest.raises(rf.RamforgeError, match="must be 1, 2 or 3"):
            sm.set_stream_units(bad)
    sm.forward(5, 0)
    assert all(sctx.charge(f"cache:layer:{i}:attn_q.weight") is not None for i in range(4))
    sm.set_stream_units(3)  # releases every resident layer
    for i in range(4):
        assert sctx.charge(f"cache:layer:{i}:attn_q.weight") is None
    sm.forward(6, 1)
    assert sm.residency_stats()["cached_layers"] == 12  # units
    sm.close()
    assert sctx.vram_used == sctx.base_used
    sctx.close()


def test_streaming_without_cache_releases_every_layer(ctx):
    rng = np.random.default_rng(1235)
    T = _tiny_tensors(rng, STREAM_CFG, STREAM_TYPES)
    sctx, sm = _streaming_model(STREAM_CFG, T, 0, 0)
    before = sctx.vram_used
    sm.forward(7, 0)
    assert sctx.vram_used == before  # release_layer after the pass: no layer or cache charge left
    for i in range(4):
        assert sctx.charge(f"layer:{i}:attn_q.weight") is None
        assert sctx.charge(f"cache:layer:{i}:attn_q.weight") is None
    assert sm.residency_stats()["misses"] == 4 and sm.residency_stats()["cached_layers"] == 0
    sm.close()
    sctx.close()


def test_streaming_budget_too_small_rolls_back(ctx):
    rf = _rf()
    rng = np.random.default_rng(1236)
    T = _tiny_tensors(rng, STREAM_CFG, STREAM_TYPES)
    probe_ctx, probe = _streaming_model(STREAM_CFG, T, 0, 0)
    base = probe_ctx.vram_used
    probe.close()
    probe_ctx.close()
    lb = min(_layer_bytes(T, i) for i in range(4))
    sctx, sm = _streaming_model(STREAM_CFG, T, base + lb // 2, 10 ** 9)
    used = sctx.vram_used
    with pytest.raises(rf.RamforgeError, match="insufficient memory"):
        sm.forward(7, 0)
    assert sctx.vram_used == used  # every charge of the failed load released
    assert sm.seq_len == 0
    sm.close()
    sctx.close()


def test_streaming_refuses_graph_and_late_enable(ctx):
    rf = _rf()
    rng = np.random.default_rng(1237)
    T = _tiny_tensors(rng, STREAM_CFG, STREAM_TYPES)
    gm = _load_gpu(ctx, STREAM_CFG, T, 40)
    with pytest.raises(rf.RamforgeError, match="before block tensors"):
        gm.enable_streaming(1 << 20)
    gm.close()
    sctx, sm = _streaming_model(STREAM_CFG, T, 0, 1 << 30)
    with pytest.raises(rf.RamforgeError, match="resident"):
        sm.use_graph(True)
    sm.close()
    sctx.close()


def _half_tensors(rng, cfg, t, orc):
    """Tiny-model tensors with every matrix (embedding, output and the seven
    projections) in F16 or BF16, plus the oracle's view of them: the same
    values decoded to F32, as the reference decodes F16 / BF16 tensors to f32
    at load (core/src/tensor.rs:498-521, 967-1014) and multiplies them as f32
    rows.  F16 payloads include subnormals (quant.rs:40-65 decodes them at
    half the IEEE value) and signed zeros."""
    from helpers import BF16, F16

    base = _tiny_tensors(rng, cfg, ALL_F32)
    T, R = {}, {}
    for name, (bt, ne0, ne1, arr) in base.items():
        if name.endswith("norm.weight") or name.endswith(".bias"):
            T[name] = R[name] = (bt, ne0, ne1, arr)
            continue
        v = rng.normal(0, 0.05, ne0 * ne1).astype(np.float32)
        if t == F16:
            bits = v.astype(np.float16).view(np.uint16).copy()
            sub = rng.random(bits.size) < 0.02  # f16 subnormals, either sign
            bits[sub] = (rng.integers(1, 0x400, sub.sum()) | (rng.integers(0, 2, sub.sum()) << 15)).astype(np.uint16)
            bits[rng.random(bits.size) < 0.005] = 0x8000
        else:
            assert t == BF16
            bits = (v.view(np.uint32) >> 16).astype(np.uint16)
        raw = bits.view(np.uint8)
        T[name] = (t, ne0, ne1, raw)
        R[name] = (F32, ne0, ne1, orc.dequantize_rows(t, raw, ne0, ne1).reshape(-1))
    return T, R


@pytest.mark.parametrize("streamed", [False, True], ids=["resident", "streamed"])
@pytest.mark.parametrize("half", ["f16", "bf16"])
def test_tiny_model_f16_bf16_weights(ctx, orc, half, streamed):
    """F16 / BF16 weights widened to F32 at install (on the device when
    resident, on the host when the layers stream), against the oracle running
    the f32 values the reference decodes at load: hidden states and logits
    within 2e-4, identical greedy tokens."""
    from helpers import BF16, F16

    t = {"f16": F16, "bf16": BF16}[half]
    cfg = dict(TINY)
    T, R = _half_tensors(np.random.default_rng(970 + t), cfg, t, orc)
    print(f"  tiny model {half} weights, {'streamed' if streamed else 'resident'}", flush=True)
    if streamed:
        sctx, gm = _streaming_model(cfg, T, 0, 1 << 30, cap=48)
    else:
        sctx, gm = None, _load_gpu(ctx, cfg, T, 48)
    om = orc.Model(cfg, R, kv_capacity=48, threads=4)
    for pos, tok in enumerate([5, 17, 90, 3]):
        h = gm.forward(tok, pos, want_hidden=True)
        hr = om.forward(tok, pos)
        assert np.max(np.abs(h - hr)) <= 2e-4 * max(1.0, np.abs(hr).max()), (half, pos)
        lr = om.logits(hr)
        assert np.max(np.abs(gm.logits() - lr)) <= 2e-4 * max(1.0, np.abs(lr).max()), (half, pos)
    gm.reset()
    om.reset()
    toks = gm.generate([1, 2, 3, 4], 20)
    ref, margin = om.generate([1, 2, 3, 4], 20)
    assert toks == ref, f"greedy divergence (min top-2 margin {margin.min():.3g})"
    gm.close()
    om.close()
    if sctx is not None:
        sctx.close()


def test_forward_profiler_records_every_group(ctx):
    """rf_model_profile: per-group device time of real forwards, logits and
    eager decode steps (compute_dispatch.rs:48-56, profile.rs:7-23), with the
    results unchanged and graph replay refused while it is on."""
    rf = _rf()
    cfg = dict(TINY)
    T = _tiny_tensors(np.random.default_rng(990), cfg, ALL_Q8)
    gm = _load_gpu(ctx, cfg, T, 48)
    plain = [gm.forward(t, p, want_hidden=True) for p, t in enumerate([5, 17, 90])]
    gm.reset()
    gm.profile(True)
    with pytest.raises(rf.RamforgeError, match="profiler"):
        gm.use_graph(True)
    prof = [gm.forward(t, p, want_hidden=True) for p, t in enumerate([5, 17, 90])]
    for a, b in zip(plain, prof):
        assert np.array_equal(a, b)
    gm.logits()
    gm.decode_steps(2)
    r = gm.profile_read(reset=True)
    nl = cfg["block_count"]
    for k in ("qkv", "attention", "oproj", "gateup", "down"):
        assert r[k][1] == 5 * nl and r[k][0] > 0, (k, r[k])
    assert r["logits"][1] == 3 and r["logits"][0] > 0, r["logits"]  # logits() + 2 decode steps
    assert all(v == (0.0, 0) for v in gm.profile_read().values())
    gm.profile(False)
    gm.use_graph(True)
    gm.close()
