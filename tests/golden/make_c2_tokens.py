"""Writes tests/golden/c2_seed0.json from the pinned CPU oracle (run from the repository root;
a few minutes on 8 cores).

The full 32-layer C2 model (synthetic GGUF ``c2``, seed 0) and bench.py's prompt (512 uniform ids
from seed 0): the prefill state and 32 decode states of the oracle's greedy run, with the figures
``golden_run.step_record`` keeps per step (token, runner-up, top-2 gap, first logits, the 8
largest, the norm). The GPU test feeds the oracle's tokens to the device (teacher forcing) and
compares every step; bench.py compares its first greedy tokens with these.
"""
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import oracle as O  # noqa: E402
from golden_run import record  # noqa: E402
from inference_engine_rust_amd import synth  # noqa: E402

N_PROMPT, N_STEPS, PROMPT_SEED = 512, 33, 0


def main():
    t0 = time.time()
    log = lambda m: print(f"[{time.time() - t0:7.1f}s] {m}", flush=True)  # noqa: E731
    with tempfile.TemporaryDirectory(dir="/dev/shm" if os.path.isdir("/dev/shm") else None) as d:
        p = os.path.join(d, "c2.gguf")
        spec = synth.preset("c2")
        synth.write_llama(p, spec, seed=0)
        s = O.Session(O.Model(p))
        s.prefill(synth.prompt_ids(PROMPT_SEED, N_PROMPT, spec.vocab))
        log("prefill done")
        steps = record(O, s, N_STEPS, log)
    out = {"config": "c2", "seed": 0, "prompt_seed": PROMPT_SEED, "n_prompt": N_PROMPT, "steps": steps}
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "c2_seed0.json"), "w") as f:
        json.dump(out, f)


if __name__ == "__main__":
    main()
