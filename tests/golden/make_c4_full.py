"""Writes tests/golden/c4_seed0.json from the pinned CPU oracle (run from the repository root;
about half an hour on 8 cores).

The full 32-layer C4 model (synthetic GGUF ``c4``, seed 0: C2 with an 8704-token context) and
bench.py's C4 prompt (8192 uniform ids from seed 0, full causal attention over the prompt): the
prefill state and 4 decode states of the oracle's greedy run, with the figures
``golden_run.step_record`` keeps per step.
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

N_PROMPT, N_STEPS, PROMPT_SEED = 8192, 5, 0


def main():
    t0 = time.time()
    log = lambda m: print(f"[{time.time() - t0:7.1f}s] {m}", flush=True)  # noqa: E731
    with tempfile.TemporaryDirectory(dir="/dev/shm" if os.path.isdir("/dev/shm") else None) as d:
        p = os.path.join(d, "c4.gguf")
        spec = synth.preset("c4")
        synth.write_llama(p, spec, seed=0)
        s = O.Session(O.Model(p))
        s.prefill(synth.prompt_ids(PROMPT_SEED, N_PROMPT, spec.vocab))
        log("prefill done")
        steps = record(O, s, N_STEPS, log)
    out = {"config": "c4", "seed": 0, "prompt_seed": PROMPT_SEED, "n_prompt": N_PROMPT, "steps": steps}
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "c4_seed0.json"), "w") as f:
        json.dump(out, f)


if __name__ == "__main__":
    main()
