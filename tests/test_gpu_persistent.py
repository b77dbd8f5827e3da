"""Persistent weights of a streaming model (persistent.rs:1-6, 286-470): the
embedding and the output projection stay resident when they take at most a
quarter of the VRAM budget (should_keep_resident) and are otherwise streamed;
streamed, they stay in mapped pinned host memory that the embedding gather
and the logits matvec read in place.  Checked: the same hidden states,
logits and tokens as the resident policy (bit-identical: the same kernels
over the same bytes) and the oracle, with and without a tied output, through
the batched prefill, and the 25% rule choosing by budget."""
import numpy as np
import pytest

from helpers import Q6_K, Q8_0
from test_gpu_model import STREAM_CFG, STREAM_TYPES, _tiny_tensors

pytestmark = pytest.mark.gpu


def _rf():
    import ramforge_amd as rf

    return rf


def _model(cfg, T, policy, budget=0, cap=48):
    rf = _rf()
    ctx = rf.Context(0, budget)
    m = rf.GpuLlamaModel(ctx, cfg, cap)
    m.enable_streaming(1 << 30)
    m.set_persistent_policy(policy)
    for name, (t, ne0, ne1, arr) in T.items():
        m.set_tensor(name, t, ne0, ne1, arr)
    return ctx, m


@pytest.mark.parametrize("tied", [False, True], ids=["output", "tied"])
def test_streamed_persistent_matches_resident(orc, tied):
    cfg = STREAM_CFG
    T = _tiny_tensors(np.random.default_rng(1500), cfg, STREAM_TYPES)
    if tied:
        del T["output.weight"]  # logits from token_embd (compute_logits' tied case)
    sctx, sm = _model(cfg, T, 1)
    rctx, rm = _model(cfg, T, 2)
    assert sm.persistent_streamed() == {"token_embd": True, "output": not tied}
    assert rm.persistent_streamed() == {"token_embd": False, "output": False}
    assert sctx.charge("persistent:token_embd.weight") is None
    assert rctx.charge("persistent:token_embd.weight") is not None
    om = orc.Model(cfg, T, kv_capacity=48, threads=4)
    for pos, tok in enumerate([5, 17, 90, 3]):
        a = sm.forward(tok, pos, want_hidden=True)
        b = rm.forward(tok, pos, want_hidden=True)
        assert np.array_equal(a, b), pos
        la, lb = sm.logits(), rm.logits()
        assert np.array_equal(la, lb), pos
        lr = om.logits(om.forward(tok, pos))
        assert np.max(np.abs(la - lr)) <= 2e-4 * max(1.0, np.abs(lr).max()), pos
    for m in (sm, rm):
        m.reset()
    prompt = [int(t) for t in np.random.default_rng(7).integers(0, cfg["vocab_size"], 20)]
    assert sm.paths()["batched_prefill"] and rm.paths()["batched_prefill"]
    ha = sm.prefill(prompt, want_hidden=True)  # batched: embedding rows read from host memory
    hb = rm.prefill(prompt, want_hidden=True)
    assert np.array_equal(ha, hb)
    for m in (sm, rm):
        m.reset()
    assert sm.generate([1, 2, 3], 16) == rm.generate([1, 2, 3], 16)
    sm.close(); rm.close(); om.close()
    sctx.close(); rctx.close()


def test_quarter_budget_rule():
    """should_keep_resident: at most budget / 4 stays resident."""
    cfg = dict(STREAM_CFG, vocab_size=8192)
    T = _tiny_tensors(np.random.default_rng(1501), cfg, dict(STREAM_TYPES, embd=Q8_0, out=Q6_K))
    embd, out = T["token_embd.weight"][3].nbytes, T["output.weight"][3].nbytes
    rf = _rf()
    probe = rf.Context(0, 0)
    base = probe.vram_used
    probe.close()
    ctx, m = _model(cfg, T, 0, budget=base + 64 * max(embd, out))
    assert m.persistent_streamed() == {"token_embd": False, "output": False}
    m.close(); ctx.close()
    # room for two layers, the KV cache and the workspaces, not for a quarter
    # that holds either persistent tensor
    lb = sum(arr.nbytes for n, (t, a, b, arr) in T.items() if n.startswith("blk.0."))
    ctx, m = _model(cfg, T, 0, budget=base + 4 * lb + (2 << 20))
    assert ctx.vram_total // 4 < min(embd, out)
    assert m.persistent_streamed() == {"token_embd": True, "output": True}
    h = m.forward(3, 0, want_hidden=True)
    assert np.all(np.isfinite(h))
    m.close(); ctx.close()


def test_embedding_only_policy():
    """Policy 3: the embedding table streamed whatever its size (a step reads
    one of its rows), the output projection by the 25% rule; the same results
    as the resident policy."""
    cfg = STREAM_CFG
    T = _tiny_tensors(np.random.default_rng(1502), cfg, STREAM_TYPES)
    sctx, sm = _model(cfg, T, 3)
    rctx, rm = _model(cfg, T, 2)
    assert sm.persistent_streamed() == {"token_embd": True, "output": False}
    assert sctx.charge("persistent:token_embd.weight") is None
    assert sctx.charge("persistent:output.weight") is not None
    for pos, tok in enumerate([8, 1, 44]):
        assert np.array_equal(sm.forward(tok, pos, want_hidden=True), rm.forward(tok, pos, want_hidden=True))
        assert np.array_equal(sm.logits(), rm.logits())
    for m in (sm, rm):
        m.reset()
    assert sm.generate([4, 5], 12) == rm.generate([4, 5], 12)
    sm.close(); rm.close()
    sctx.close(); rctx.close()
    # with a budget whose quarter holds neither tensor the rule streams the output too
    cfg2 = dict(STREAM_CFG, vocab_size=8192)
    T2 = _tiny_tensors(np.random.default_rng(1503), cfg2, dict(STREAM_TYPES, embd=Q8_0, out=Q6_K))
    rf = _rf()
    probe = rf.Context(0, 0)
    base = probe.vram_used
    probe.close()
    lb = sum(arr.nbytes for n, (t, a, b, arr) in T2.items() if n.startswith("blk.0."))
    ctx, m = _model(cfg2, T2, 3, budget=base + 4 * lb + (2 << 20))
    assert m.persistent_streamed() == {"token_embd": True, "output": True}
    m.close(); ctx.close()
