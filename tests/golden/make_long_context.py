"""Writes tests/golden/c4_l2_seed0.json from the pinned CPU oracle (run from the repository root;
about two minutes on 8 cores).

The C4 widths and context at 2 layers (synthetic GGUF ``c4_l2``, seed 0): an 8192-token prompt of
uniform ids from seed 7, then 6 greedy decode steps at batch 1. For the prefill state and each
decode state it stores the greedy token, the first 1024 logits, the 8 largest logits with their
indices, the L2 norm of the whole logits vector and the gap between the two largest logits. The
GPU test compares its logits on those indices and norms, and its tokens, with these values.
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

N_PROMPT, N_DECODE, N_HEAD = 8192, 6, 1024


def main():
    with tempfile.TemporaryDirectory(dir="/dev/shm" if os.path.isdir("/dev/shm") else None) as d:
        p = os.path.join(d, "c4_l2.gguf")
        synth.write_llama(p, synth.preset("c4_l2"), seed=0)
        s = O.Session(O.Model(p))
        prompt = synth.prompt_ids(7, N_PROMPT)
        s.prefill(prompt)
        steps = []
        for i in range(N_DECODE + 1):
            lg = s.logits().astype(np.float64)
            order = np.argsort(-lg, kind="stable")
            tok = O.argmax(lg.astype(np.float32))
            steps.append({"token": int(tok), "head": [round(float(x), 6) for x in lg[:N_HEAD]],
                          "top_idx": [int(i) for i in order[:8]], "top_val": [float(lg[i]) for i in order[:8]],
                          "norm": float(np.linalg.norm(lg)), "gap": float(lg[order[0]] - lg[order[1]])})
            if i < N_DECODE:
                s.decode(tok)
    out = {"config": "c4_l2", "seed": 0, "prompt_seed": 7, "n_prompt": N_PROMPT, "n_decode": N_DECODE,
           "steps": steps}
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "c4_l2_seed0.json"), "w") as f:
        json.dump(out, f)


if __name__ == "__main__":
    main()
