"""Writes tests/golden/*.json from the pinned CPU oracle (run from the repository root).

c0_seed0.json — the tiny Mistral-architecture config (synthetic GGUF, seed 0): a 16-token prompt
of uniform ids in [3, 32000) from seed 1, then 32 greedy decode tokens at batch 1. Stores the
prompt, the greedy tokens and the chosen token's logit per step.
"""
import json
import os
import sys
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import oracle as O  # noqa: E402
from inference_engine_rust_amd import synth  # noqa: E402


def main():
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "c0.gguf")
        synth.write_llama(p, synth.preset("c0"), seed=0)
        m = O.Model(p)
        s = O.Session(m)
        prompt = synth.prompt_ids(0, 16)
        toks, logs = O.greedy_generate(s, prompt, 32, record_logits=True)
        out = {"config": "c0", "seed": 0, "prompt": [int(x) for x in prompt], "n_decode": 32, "tokens": toks,
               "top_logits": [float(l[t]) for l, t in zip(logs, toks)],
               "top2_gap_min": float(min(sorted(l)[-1] - sorted(l)[-2] for l in logs))}
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "c0_seed0.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
