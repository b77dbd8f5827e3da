"""Writes tests/golden/model_tokens.json: the oracle's greedy tokens for the
BASELINE 8B-shape models, for the GPU token-identity tests.

The models are the seeded random-init llamas of ramforge_amd.synthetic (the
generator is byte-identical on the host and the device), the prompts 32 ids
from numpy's default_rng(seed).  For each model the CPU oracle (the C
restatement of the reference's decode loop, oracle/ramforge_oracle.c) forwards
the prompt token by token and then decodes greedily, as
InferenceEngine::generate_impl does (inference.rs:580-707), recording every
chosen token and the top-2 logit margin of the step that chose it
(sampling.rs:45-57 picks the first maximum).

    python tests/golden/make_model_tokens.py [--threads N]

Runs for several minutes on 8 cores (the oracle splits rows over threads in
parity mode, which changes no result).  Only tests/ use the output."""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "model_tokens.json")

# name -> (body type, output type, seed, greedy tokens)
MODELS = {
    "metric_8b_q8_0": ("Q8_0", None, 8, 128),
    "config5_8b_q4k_q6k": ("Q4_K", "Q6_K", 5, 256),
}
PROMPT_LEN = 32


def model_case(name: str):
    from ramforge_amd import synthetic as syn

    body, out, seed, n = MODELS[name]
    cfg = syn.CONFIG_8B
    specs = syn.llama_specs(cfg, getattr(syn, body), output_type=getattr(syn, out) if out else None, seed=seed)
    prompt = [int(t) for t in np.random.default_rng(seed).integers(0, cfg["vocab_size"], PROMPT_LEN)]
    return cfg, specs, prompt, n


def main() -> int:
    import oracle as orc

    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 8)
    ap.add_argument("--only", default=None)
    args = ap.parse_args()
    res = json.load(open(OUT)) if os.path.exists(OUT) else {}
    orc.set_parity_threads(args.threads)
    for name in MODELS:
        if args.only and name != args.only:
            continue
        cfg, specs, prompt, n = model_case(name)
        t0 = time.time()
        T = orc.model_tensors(specs)
        om = orc.Model(cfg, T, kv_capacity=PROMPT_LEN + n + 8, threads=args.threads)
        toks, margin = om.generate(prompt, n)
        om.close()
        print(f"{name}: {len(toks)} tokens ({len(set(toks))} distinct) in {time.time() - t0:.0f} s; "
              f"min margin {float(np.min(margin)):.3g}",
              flush=True)
        res[name] = {"body": MODELS[name][0], "output": MODELS[name][1] or MODELS[name][0], "seed": MODELS[name][2],
                     "prompt": prompt, "tokens": toks, "margins": [float(f"{m:.6g}") for m in margin[:len(toks)]]}
        del T
    with open(OUT, "w") as f:
        json.dump(res, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
