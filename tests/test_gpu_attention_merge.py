"""Decode with the o-projection merging the attention's chunk records
(rf_tune_attention_merge 1, the default) against the separate merge kernel
(mode 0) and the oracle (attention_reference, compute.rs:461-547, then the
o-projection, model_executor.rs:102-236).

The models have 32 query heads of 128 dims (q_heads * head_dim = 4096, as
the 8B shape), 64 of 64, or 32 of 64 (2048 inputs, as BASELINE config 4:
Q8_0 rows of two 1024-element chunks, the 4-bit and 6-bit formats' rows of one), so the
packed Q8_0 / Q4_0 / Q4_K / Q6_K o-projection takes the merged-x launch at every
context the attention splits per query head (65 to 1024 positions here: 2 to
8 chunks, or to 4 with 64 heads).  The two modes differ in the merge's
rounding only: hidden states within 1e-5 of each other, both within 2e-4 of
the oracle, and identical greedy tokens, eager and replayed from the decode
graphs, across the launch regimes."""
import numpy as np
import pytest

from helpers import Q4_0, Q4_K, Q6_K, Q8_0
from test_gpu_model import _load_gpu, _tiny_tensors

pytestmark = pytest.mark.gpu

CFG = dict(vocab_size=192, context_length=1100, embedding_length=256, block_count=2, feed_forward_length=512,
           head_count=32, head_count_kv=8, head_dim=128, rms_eps=1e-5, rope_freq_base=10000.0)
# 64 heads of 64 dims: at most 4 chunks per query head (256 / 64), records of 68 floats
CFG64 = dict(CFG, head_count=64, head_count_kv=16, head_dim=64)
# 32 heads of 64 dims: a 2048-wide o-projection
CFG2K = dict(CFG, head_count=32, head_count_kv=8, head_dim=64)
CAP = 1100


def _types(o):
    return dict(embd=Q8_0, out=Q8_0, q=Q8_0, k=Q8_0, v=Q8_0, o=o, gate=Q8_0, up=Q8_0, down=Q8_0)


@pytest.fixture
def merge_mode():
    import ramforge_amd as rf

    old = rf.tune_attention_merge(-1)
    yield rf.tune_attention_merge
    rf.tune_attention_merge(old)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("o,cfg", [(Q8_0, CFG), (Q4_0, CFG), (Q4_K, CFG), (Q6_K, CFG), (Q8_0, CFG64),
                                   (Q8_0, CFG2K), (Q4_0, CFG2K), (Q4_K, CFG2K), (Q6_K, CFG2K)],
                         ids=["q8_0", "q4_0", "q4_k", "q6_k", "q8_0-hd64", "q8_0-2048", "q4_0-2048", "q4_k-2048",
                              "q6_k-2048"])
def test_merged_oproj_matches_merge_kernel(ctx, orc, merge_mode, o, cfg):
    T = _tiny_tensors(np.random.default_rng(2400 + o), cfg, _types(o))
    import ramforge_amd as rf

    om = orc.Model(cfg, T, kv_capacity=CAP, threads=8)
    ctxs = {1: ctx, 0: rf.Context(0)}  # a model's ledger names are per context
    gm = {mode: _load_gpu(ctxs[mode], cfg, T, CAP) for mode in (1, 0)}
    prompt = [int(t) for t in np.random.default_rng(7).integers(0, cfg["vocab_size"], 40)]
    differs = False
    try:
        # eager forward across positions 0..199 (regimes 0 and 1) and a few
        # later ones; the oracle at every 16th position
        for mode in (1, 0):
            merge_mode(mode)
            gm[mode].reset()
        om.reset()
        worst = 0.0
        for pos in range(200):
            tok = prompt[pos % len(prompt)]
            h = {}
            for mode in (1, 0):
                merge_mode(mode)
                h[mode] = gm[mode].forward(tok, pos, want_hidden=True)
            hr = om.forward(tok, pos)
            scale = max(1.0, float(np.abs(hr).max()))
            d10 = float(np.max(np.abs(h[1] - h[0])))
            assert d10 <= 1e-5 * scale, (pos, d10)
            differs = differs or not np.array_equal(h[1].view(np.uint32), h[0].view(np.uint32))
            if pos % 16 == 15 or pos in (64, 65, 66):
                for mode in (1, 0):
                    dr = float(np.max(np.abs(h[mode] - hr)))
                    assert dr <= 2e-4 * scale, (mode, pos, dr)
                    worst = max(worst, dr / scale)
        print(f"  o-proj {o}: 200 positions, modes within 1e-5, oracle within {worst:.3g} (relative)", flush=True)
        # merged and separate merges round differently: the merged launch ran
        assert differs
        # greedy tokens: graph replay across regimes 0, 1 and 2 (up to 700
        # positions), both modes against the oracle
        n = 660
        om.reset()
        ref, margin = om.generate(prompt, n)
        for mode in (1, 0):
            merge_mode(mode)
            g = gm[mode]
            g.reset()
            for p, t in enumerate(prompt):
                g.forward(t, p)
            g.use_graph(True)
            got = []
            for k in (20, 100, 400, 140):
                g.decode_steps(k)
                got += g.read_tokens(k)
                ctxs[mode].synchronize()
            g.use_graph(False)
            first = next((i for i, (a, b) in enumerate(zip(got, ref)) if a != b), None)
            assert got == ref[:n], f"mode {mode}: first divergence at {first}, margin {margin[first]:.3g}"
        print(f"  o-proj {o}: {n} greedy tokens identical in both modes and the oracle", flush=True)
    finally:
        for g in gm.values():
            g.close()
        ctxs[0].close()
        om.close()
