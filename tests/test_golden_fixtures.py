"""CPU checks of the committed model-token fixture (tests/golden/model_tokens.json,
written by tests/golden/make_model_tokens.py from the oracle): its prompts
follow from its seeds, and its greedy runs are long and varied enough for a
token-identity test to mean something."""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def test_model_token_fixture_is_consistent():
    from ramforge_amd import synthetic as syn

    fx = json.load(open(os.path.join(HERE, "golden", "model_tokens.json")))
    assert {"metric_8b_q8_0": 128, "config5_8b_q4k_q6k": 256} == {k: len(v["tokens"]) for k, v in fx.items()}
    for name, v in fx.items():
        prompt = [int(t) for t in np.random.default_rng(v["seed"]).integers(0, syn.CONFIG_8B["vocab_size"], 32)]
        assert v["prompt"] == prompt, name
        assert len(v["margins"]) == len(v["tokens"]) and min(v["margins"]) >= 0.0
        assert all(0 <= t < syn.CONFIG_8B["vocab_size"] for t in v["tokens"])
        assert len(set(v["tokens"])) >= 20, f"{name}: a degenerate greedy run proves little"
