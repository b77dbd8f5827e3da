"""The bench's secondary modes run end to end (short)
(resident 16-layer model) and config 5 (the streamed 8B Q4_K/Q6_K model),
with the same functions `bench.py --config4` / `--config5` call, and their
result records carry the fields the profiles quote.  (Their token parity
with the oracle is test_gpu_model.py / test_gpu_8b_tokens.py.)"""
import importlib.util
import os

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def _bench():
    spec = importlib.util.spec_from_file_location("rf_bench", os.path.join(HERE, "..", "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_config4_mode():
    import ramforge_amd as rf
    from ramforge_amd import synthetic as syn

    out = _bench().config4_bench(rf, syn, tokens=8, prompt_len=4)
    assert out["tokens"] == 8 and len(out["tokens_head"]) == 8
    assert out["tok_s"] > 0 and out["prompt_batched_ms"] > 0
    print(f"  config 4 (8 tokens): {out['tok_s']} tok/s", flush=True)


@pytest.mark.timeout(300)
def test_config5_mode():
    import ramforge_amd as rf
    from ramforge_amd import synthetic as syn

    out = _bench().config5_bench(rf, syn, 4, 4, 1, 3)
    assert out["tokens"] == 4 and out["cache"]["misses"] > 0
    assert out["vram_peak_bytes"] <= out["vram_budget_bytes"]
    assert 0 < out["host_link_frac"] <= 1.05
    print(f"  config 5 (4 tokens): {out['tok_s']} tok/s, {out['uploaded_GB_per_token']} GB/token", flush=True)
