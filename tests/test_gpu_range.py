"""Prefill activations beyond the fp16 pair's range, against the CPU oracle.

The prefill's matrix-core GEMMs and attention take each f32 activation as an fp16 (hi, lo) pair,
which holds |x| <= 65504. The reference's f32 arithmetic (src/ops/matmul.rs:176-204,
src/layers/attention.rs:175-422) takes any finite value. Here the FFN norm weights of a layer
are scaled up (in the GGUF bytes) so that the SwiGLU / GeGLU outputs feeding the down projection
exceed 65504: the kernel that splits them flags it, the prefill runs again on f32 activations
(iek_session_f32_prefills counts it), and the logits match the oracle's.
"""
import numpy as np
import pytest

import oracle as O
from inference_engine_rust_amd import engine as E
from inference_engine_rust_amd import synth

pytestmark = pytest.mark.gpu

LOGIT_REL_L2 = 1e-3


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def _scale_f32_tensor(path, name, factor):
    start, gt, dims = synth.tensor_offsets(path)[name]
    assert gt == synth.GGML_F32
    n = int(np.prod(dims))
    with open(path, "r+b") as f:
        f.seek(start)
        w = np.frombuffer(f.read(4 * n), np.float32) * np.float32(factor)
        f.seek(start)
        f.write(w.astype(np.float32).tobytes())


@pytest.mark.parametrize("preset,n_prompt", [("c2_l2", 512), ("c0", 48)])
def test_prefill_beyond_fp16_range_matches_oracle(gpu, tmp_path, preset, n_prompt):
    p = str(tmp_path / f"{preset}_big.gguf")
    synth.write_llama(p, synth.preset(preset), seed=7)
    # x1000 on the FFN norm of layer 0: gate and up grow ~1000x, their SwiGLU product ~1e6x
    _scale_f32_tensor(p, "blk.0.ffn_norm.weight", 1000.0)
    m, om = E.LoadedModel.load(p), O.Model(p)
    prompt = synth.prompt_ids(9, n_prompt)
    s, r = E.InferenceSession(m), O.Session(om)
    s.prefill(prompt)
    r.prefill(prompt)
    assert s.f32_prefills() == 1
    assert rel_l2(s.hidden(), r.hidden()) < 1e-4
    for step in range(4):
        lg, lr = s.logits_last_token(), r.logits()
        assert rel_l2(lg, lr) < LOGIT_REL_L2, (step, rel_l2(lg, lr))
        t = O.argmax(lr)
        assert E.greedy_next_token(s) == t, step
        s.decode_token(t)
        r.decode(t)
    # the unscaled model stays on the matrix-core path
    q = str(tmp_path / f"{preset}.gguf")
    synth.write_llama(q, synth.preset(preset), seed=7)
    s2 = E.InferenceSession(E.LoadedModel.load(q))
    s2.prefill(prompt)
    assert s2.f32_prefills() == 0


def test_gemma_prefill_beyond_fp16_range_matches_oracle(gpu, tmp_path):
    p = str(tmp_path / "g0_big.gguf")
    synth.write_gemma4(p, synth.preset("g0"), seed=3)
    _scale_f32_tensor(p, "blk.1.ffn_norm.weight", 3000.0)
    m, om = E.LoadedModel.load(p), O.Model(p)
    prompt = synth.prompt_ids(2, 40, 8192)
    s, r = E.InferenceSession(m), O.Session(om)
    s.prefill(prompt)
    r.prefill(prompt)
    assert s.f32_prefills() == 1
    for step in range(3):
        lg, lr = s.logits_last_token(), r.logits()
        assert rel_l2(lg, lr) < LOGIT_REL_L2, (step, rel_l2(lg, lr))
        t = O.argmax(lr)
        assert E.greedy_next_token(s) == t, step
        s.decode_token(t)
        r.decode(t)


def test_layer_level_prefill_reruns_the_flagged_layer(gpu, tmp_path):
    """The layer-level forward (prefill_layer_block, src/layers/block.rs:12) keeps each layer's
    input and runs a flagged layer again on f32 activations; its state matches the oracle's."""
    p = str(tmp_path / "c0_big.gguf")
    synth.write_llama(p, synth.preset("c0"), seed=7)
    _scale_f32_tensor(p, "blk.1.ffn_norm.weight", 1000.0)
    m = E.LoadedModel.load(p)
    prompt = synth.prompt_ids(9, 48)
    r = O.Session(O.Model(p))
    r.prefill(prompt)
    b = E.InferenceSession(m)
    b.embed(prompt)
    b.prefill_layer_block(0)
    assert b.f32_prefills() == 0
    b.prefill_layer_block(1)
    assert b.f32_prefills() == 1
    assert rel_l2(b.hidden(), r.hidden()) < 1e-4
    assert rel_l2(b.logits_last_token(), r.logits()) < LOGIT_REL_L2
