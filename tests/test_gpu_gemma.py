"""Gemma-4 family on the device (A14, A23, A32 and the Q8_0 path A5/A9) against the CPU oracle,
on the tiny seeded Gemma-4 model ``g0`` (every Gemma feature switched on: sliding window below
the prompt length, KV borrowing, per-layer embeddings, partial rotary with freq factors, F32 and
Q8_0 layer scales, tied Q8_0 LM head with soft cap).

Bars (north star): greedy tokens identical; per-step logits within 1e-3 relative L2.
"""
import numpy as np
import pytest

import oracle as O
from inference_engine_rust_amd import engine as E
from inference_engine_rust_amd import synth

pytestmark = pytest.mark.gpu

LOGIT_REL_L2 = 1e-3
SPEC = synth.preset("g0")


def rel_l2(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / np.linalg.norm(b.astype(np.float64)))


@pytest.fixture(scope="module")
def g0_path(model_dir):
    p = str(model_dir / "g0_gpu.gguf")
    synth.write_gemma4(p, SPEC, seed=0)
    return p


@pytest.fixture(scope="module")
def g0_gpu(gpu, g0_path):
    return E.LoadedModel.load(g0_path)


@pytest.fixture(scope="module")
def g0_orc(g0_path):
    return O.Model(g0_path)


def test_gemma_config_matches_oracle(g0_gpu, g0_orc):
    a, b = g0_gpu.config, g0_orc.cfg
    assert a.family == b.family == 1
    for f in ["context_length", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "head_dim", "ffn_dim",
              "vocab_size"]:
        assert getattr(a, f) == getattr(b, f), f
    assert a.embedding_length_per_layer == b.ple_dim
    assert a.has_final_logit_softcapping == b.has_softcap and a.final_logit_softcapping == b.softcap
    for li in range(SPEC.n_layers):
        ga, gb = g0_gpu.layer_spec(li), g0_orc.layer_spec(li)
        for f in ("sliding_window", "rope_theta", "rotary_dim", "kv_borrow", "head_dim"):
            assert ga[f] == gb[f], (li, f)


def test_gemma_prefill_logits_and_hidden(g0_gpu, g0_orc):
    """Gemma-4 sessions keep an f32 KV cache like the reference, so the borrowing layers read
    exactly the K/V their source layer computed."""
    prompt = synth.prompt_ids(0, 20, SPEC.vocab)  # longer than the window (16)
    s = E.InferenceSession(g0_gpu)
    r = O.Session(g0_orc)
    s.prefill(prompt)
    r.prefill(prompt)
    h = rel_l2(s.hidden(), r.hidden())
    assert h < 2e-5
    lg, lr = s.logits_last_token(), r.logits()
    assert rel_l2(lg, lr) < LOGIT_REL_L2
    assert E.greedy_next_token(s) == O.argmax(lr)


def test_gemma_prefill_without_borrowing(gpu, model_dir):
    """The same model with no shared-KV layers (every layer appends to and attends over its own
    cache)."""
    spec = synth.preset("g0", shared_kv_layers=0)
    p = str(model_dir / "g0_noborrow.gguf")
    synth.write_gemma4(p, spec, seed=0)
    m, om = E.LoadedModel.load(p), O.Model(p)
    prompt = synth.prompt_ids(0, 20, spec.vocab)
    s, r = E.InferenceSession(m), O.Session(om)
    s.prefill(prompt)
    r.prefill(prompt)
    h = rel_l2(s.hidden(), r.hidden())
    assert h < 2e-5
    assert rel_l2(s.logits_last_token(), r.logits()) < 1e-4


def test_gemma_greedy_tokens_and_logits(g0_gpu, g0_orc):
    prompt = synth.prompt_ids(1, 10, SPEC.vocab)
    s = E.InferenceSession(g0_gpu)
    r = O.Session(g0_orc)
    s.prefill(prompt)
    r.prefill(prompt)
    worst = 0.0
    for step in range(14):  # the context grows past the window
        lg, lr = s.logits_last_token(), r.logits()
        worst = max(worst, rel_l2(lg, lr))
        t = E.greedy_next_token(s)
        assert t == O.argmax(lr), f"step {step}"
        s.decode_token(t)
        r.decode(t)
    assert worst < LOGIT_REL_L2, worst
    for layer in range(SPEC.n_layers):  # f32 cache: equal to the oracle's up to f32 reordering
        src = g0_gpu.layer_spec(layer)["kv_borrow"]
        for which in (False, True):
            kg = s.kv(layer, which)
            kr = r.kv(layer if src < 0 else src, which).transpose(1, 0, 2)
            assert kg.shape == kr.shape
            np.testing.assert_allclose(kg, kr, rtol=1e-4, atol=2e-4)


def test_gemma_decode_eight_query_heads_per_kv_head(gpu, model_dir):
    """A GQA group of 8 (as in the Gemma-4-E2B shape): the f32-cache decode attention splits the
    group's query heads over two workgroups per slice, each with its own merge."""
    spec = synth.preset("g0", n_heads=8)
    p = str(model_dir / "g0_h8.gguf")
    synth.write_gemma4(p, spec, seed=4)
    m, om = E.LoadedModel.load(p), O.Model(p)
    assert m.config.n_heads // m.config.n_kv_heads == 8
    prompt = synth.prompt_ids(4, 9, spec.vocab)
    s, r = E.InferenceSession(m), O.Session(om)
    s.prefill(prompt)
    r.prefill(prompt)
    worst = 0.0
    for step in range(12):  # past the window (16) into the second window
        lg, lr = s.logits_last_token(), r.logits()
        worst = max(worst, rel_l2(lg, lr))
        t = E.greedy_next_token(s)
        assert t == O.argmax(lr), f"step {step}"
        s.decode_token(t)
        r.decode(t)
    assert worst < LOGIT_REL_L2, worst


def test_gemma_graph_generate_matches_stepwise(g0_gpu):
    prompt = synth.prompt_ids(2, 9, SPEC.vocab)
    a = E.InferenceSession(g0_gpu)
    a.prefill(prompt)
    ga = a.generate_greedy(16)
    b = E.InferenceSession(g0_gpu)
    b.prefill(prompt)
    gb = []
    for _ in range(16):
        t = E.greedy_next_token(b)
        gb.append(t)
        b.decode_token(t)
    assert ga == gb
    np.testing.assert_array_equal(a.logits_last_token(), b.logits_last_token())


def test_gemma_prefill_vs_prefill_plus_decode(g0_gpu):  # gemma_decode_self_consistency.rs on the device
    ids = synth.prompt_ids(3, 19, SPEC.vocab)
    a = E.InferenceSession(g0_gpu)
    a.prefill(ids)
    b = E.InferenceSession(g0_gpu)
    b.prefill(ids[:-1])
    b.decode_token(int(ids[-1]))
    assert np.max(np.abs(a.logits_last_token() - b.logits_last_token())) < 1e-3


def test_gemma_borrowed_prefill_needs_fresh_cache(g0_gpu):
    """A prompt on a non-empty cache: the borrowing layers' source caches no longer hold exactly
    the prompt, which the reference rejects (attention.rs:219-241)."""
    s = E.InferenceSession(g0_gpu)
    s.prefill(synth.prompt_ids(0, 4, SPEC.vocab))
    with pytest.raises(E.EngineError) as e:
        s.prefill(synth.prompt_ids(1, 3, SPEC.vocab))
    assert e.value.kind == "Model"
