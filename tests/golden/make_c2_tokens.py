"""Writes tests/golden/c2_seed0_tokens.json from the pinned CPU oracle (run from the repository
root; a few minutes on 8 cores).

The full 32-layer C2 model (synthetic GGUF ``c2``, seed 0) and bench.py's prompt (512 uniform ids
from seed 0): the first 8 greedy tokens, with each step's runner-up token, the gap between the two largest
logits, the chosen token's logit, the first 1024 logits and the L2 norm of all of them. bench.py and the GPU tests compare the device's tokens with
these; a step whose gap is within float rounding of the 32-layer sum (below 1e-2) only requires
the device's token to be one of the two.
"""
import json
import os
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import oracle as O  # noqa: E402
from inference_engine_rust_amd import synth  # noqa: E402

N_PROMPT, N_DECODE = 512, 8


def main():
    with tempfile.TemporaryDirectory(dir="/dev/shm" if os.path.isdir("/dev/shm") else None) as d:
        p = os.path.join(d, "c2.gguf")
        spec = synth.preset("c2")
        synth.write_llama(p, spec, seed=0)
        s = O.Session(O.Model(p))
        s.prefill(synth.prompt_ids(0, N_PROMPT, spec.vocab))
        toks, second, gaps, vals, heads, norms = [], [], [], [], [], []
        for i in range(N_DECODE):
            lg = s.logits()
            t = O.argmax(lg)
            order = np.argsort(-lg.astype(np.float64), kind="stable")
            toks.append(int(t))
            second.append(int(order[1]))
            gaps.append(float(lg[order[0]]) - float(lg[order[1]]))
            vals.append(float(lg[t]))
            heads.append([round(float(x), 6) for x in lg[:1024]])
            norms.append(float(np.linalg.norm(lg.astype(np.float64))))
            s.decode(t)
    out = {"config": "c2", "seed": 0, "prompt_seed": 0, "n_prompt": N_PROMPT, "tokens": toks, "runner_up": second,
           "top2_gap": gaps, "top_logit": vals, "head": heads, "norm": norms}
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "c2_seed0_tokens.json"), "w") as f:
        json.dump(out, f)


if __name__ == "__main__":
    main()
