"""Shared recorder for the oracle golden runs in this directory (test infrastructure).

``record(session, n_steps)`` reads the logits of the current state, stores the greedy token and
the figures the GPU tests compare, decodes that token, and repeats: the oracle's own greedy
sequence, which the GPU tests then feed to the device (teacher forcing), so that a near-tie at
one step cannot end the comparison.
"""
import numpy as np

N_HEAD = 512


def step_record(lg: np.ndarray, tok: int) -> dict:
    """Per-step figures of one logits vector: the greedy token, runner-up and gap between the two
    largest logits, the first N_HEAD logits, the 8 largest with their indices, the L2 norm."""
    l64 = lg.astype(np.float64)
    order = np.argsort(-l64, kind="stable")
    return {"token": int(tok), "runner_up": int(order[1]), "gap": float(l64[order[0]] - l64[order[1]]),
            "head": [round(float(x), 6) for x in lg[:N_HEAD]], "top_idx": [int(i) for i in order[:8]],
            "top_val": [float(l64[i]) for i in order[:8]], "norm": float(np.linalg.norm(l64))}


def record(O, session, n_steps: int, log=None, shadows=None) -> list:
    """Steps 0..n_steps-1: step 0 is the prefill state; step i > 0 follows i decodes of the
    oracle's greedy tokens. `shadows`, when given, maps a name to a second oracle session over the
    same model and prompt in another arithmetic mode: "reassoc" (REASSOC: every f32 matmul summed
    as two halves of K, a legitimate reordering of the reference's arithmetic) and "pair" (PAIR:
    that, with every prefill matmul input first rounded to its fp16 (hi, lo) pair, the device
    prefill's operands). Each decodes the same tokens, and each step records how far it moves the
    logits: the relative L2 over the whole vector (<name>_rel) and the largest change among the 8
    largest logits (<name>_top_dmax)."""
    steps = []
    shadows = shadows or {}
    for i in range(n_steps):
        lg = session.logits()
        tok = O.argmax(lg)
        steps.append(step_record(lg, tok))
        l64 = lg.astype(np.float64)
        top = steps[-1]["top_idx"]
        extra = ""
        for name, sh in shadows.items():
            ls = sh.logits().astype(np.float64)
            steps[-1][f"{name}_rel"] = float(np.linalg.norm(ls - l64) / np.linalg.norm(l64))
            steps[-1][f"{name}_top_dmax"] = float(np.max(np.abs(ls[top] - l64[top])))
            extra += f" {name} {steps[-1][f'{name}_rel']:.3g}"
        if log:
            log(f"step {i}: token {tok} gap {steps[-1]['gap']:.4g}{extra}")
        if i + 1 < n_steps:
            session.decode(tok)
            for sh in shadows.values():
                sh.decode(tok)
    return steps
