"""Writes config4_prefill.json: the f64 oracle's logits for BASELINE config 4's
long prefill, which the GPU tests compare with the device's.

Config 4 (V256 W512 H8x64 L4, butterfly meshes of depth 9, context 8448),
weights from the reference's seeded initialisation (seed 7,
src/gpt/config.rs:443-449), prompt = sequence 0 of the benchmark's prompts
(Random::new(7).index(256), 8 sequences of 8192 tokens, drawn in order).  The
oracle runs the whole 8192-row forward once (og_logits: full causal attention
at every layer, reference.rs:104-228); by causality, row n - 1 of it is the
last-row logit vector of the prompt's first n tokens, recorded for n = 1024,
4096 and 8192.  Run from the repository root after building the oracle
(make -C oracle): python tests/golden/make_config4_prefill.py (about three
minutes on one core).
"""
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle_lib as O  # noqa: E402
import grokking_abmod_amd as G  # noqa: E402  (random_prompts is pure Python)

LENGTHS = (1024, 4096, 8192)


def main():
    kw = {k: v for k, v in G.named_config("long").as_dict().items() if k != "long_context"}
    c = O.config(**kw)
    params = O.initialize(c, 7)
    prompt = G.random_prompts(256, 8, 8192, 7)[0]
    t0 = time.time()
    logits = O.logits(c, params, prompt, 8192)
    out = {
        "config": G.named_config("long").as_dict(),
        "init_seed": 7,
        "prompt": "random_prompts(256, 8, 8192, 7)[0]",
        "prompt_sha": int(np.bitwise_xor.reduce(prompt.astype(np.uint64) * (np.arange(8192, dtype=np.uint64) + 1))),
        "rows": {str(n): [float(v) for v in logits[n - 1]] for n in LENGTHS},
        "oracle_seconds": round(time.time() - t0, 1),
    }
    with open(os.path.join(HERE, "config4_prefill.json"), "w") as f:
        json.dump(out, f, indent=0)
    print(f"wrote config4_prefill.json in {out['oracle_seconds']} s")


if __name__ == "__main__":
    main()
