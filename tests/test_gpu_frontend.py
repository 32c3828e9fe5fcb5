"""Text front end on the device: temperature sampling (src/engine/sampling.rs:54-79) through the
host-buffer, device and session entries against the oracle; the tokenizer prompt config read by
the library against the oracle's; and the greedy CLI loop (src/main.rs:84-126) on the C0 model with
a word-level tokenizer covering its vocabulary: golden tokens, EOS stop, BOS insertion, and the
temperature path against the oracle driven by the same uniform draws."""
import json
import os
import random

import numpy as np
import pytest

import oracle as O
from inference_engine_rust_amd import engine as E
from inference_engine_rust_amd import frontend as F
from inference_engine_rust_amd import synth

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _margin(logits, temperature, r):
    """Distance of r to the nearest cumulative-probability boundary of the reference's f32
    arithmetic (sequential sums, as np.cumsum adds): the device and the oracle agree unless r is
    within the 1-ulp differences of their exponentials of one."""
    s = (np.asarray(logits, np.float32) / np.float32(temperature)).astype(np.float32)
    e = np.exp((s - s.max()).astype(np.float32)).astype(np.float32)
    total = np.cumsum(e, dtype=np.float32)[-1]
    cum = np.cumsum((e / total).astype(np.float32), dtype=np.float32)
    return float(np.min(np.abs(cum.astype(np.float64) - r)))


def test_sample_temperature_matches_oracle(gpu):
    import torch

    rng = np.random.default_rng(11)
    checked = 0
    for n in (2, 1000, 32000, 262144):
        logits = rng.normal(0, 4, n).astype(np.float32)
        dev = torch.from_numpy(logits).cuda()
        for t in (0.3, 1.0, 1.7):
            for r in (0.0, 0.013, 0.5, 0.77, 0.999999):
                want = O.sample_temperature(logits, t, r)
                if _margin(logits, t, r) < 1e-6:
                    continue
                assert E.host_sample_temperature(logits, t, r) == want, (n, t, r)
                assert E.sample_temperature(dev.data_ptr(), n, t, r) == want, (n, t, r)
                checked += 1
    assert checked >= 40


def test_sample_temperature_special_values_and_errors(gpu):
    assert E.host_sample_temperature([0.0, np.nan, 1.0, 2.0], 1.0, 0.1) == 3
    assert E.host_sample_temperature([0.0, np.inf, 1.0], 1.0, 0.1) == 2
    assert E.host_sample_temperature([-np.inf, -np.inf], 1.0, 0.1) == 1
    assert E.host_sample_temperature([-np.inf, 0.0, -np.inf], 1.0, 0.999) == 1
    assert E.host_sample_temperature(np.zeros(8, np.float32), 0.7, 0.55) == 4
    # overflow of x / T to +inf behaves as +inf
    assert E.host_sample_temperature([1e30, 0.0, 1.0], 1e-10, 0.5) == 2
    for logits, t, r, kind in (([], 1.0, 0.5, "Sampling"), ([1.0], 0.0, 0.5, "Sampling"),
                               ([1.0], -2.0, 0.5, "Sampling"), ([1.0], float("nan"), 0.5, "Sampling"),
                               ([1.0], 1.0, 1.0, "Op"), ([1.0], 1.0, -0.1, "Op")):
        with pytest.raises(E.EngineError) as e:
            E.host_sample_temperature(logits, t, r)
        assert e.value.kind == kind


@pytest.fixture(scope="module")
def c0_tok(model_dir):
    """The C0 model with tokenizer metadata (EOS = the first golden greedy token not seen before it,
    no BOS) and a
    word-level tokenizer.json mapping id i <-> the word "w<i>" for every id of the vocabulary."""
    from tokenizers import Tokenizer, models, pre_tokenizers

    g = json.load(open(os.path.join(GOLDEN, "c0_seed0.json")))
    eos_at = next(k for k in range(1, len(g["tokens"])) if g["tokens"][k] not in g["tokens"][:k])
    base = synth.write_llama(str(model_dir / "c0_plain_fe.gguf"), synth.preset("c0"), seed=0)
    path = synth.with_metadata(base, str(model_dir / "c0_tok.gguf"), [
        ("tokenizer.ggml.model", synth.GGUF_STR, "llama"), ("tokenizer.ggml.add_bos_token", synth.GGUF_BOOL, False),
        ("tokenizer.ggml.eos_token_id", synth.GGUF_U32, g["tokens"][eos_at])])
    vocab = {f"w{i}": i for i in range(32000)}
    tk = Tokenizer(models.WordLevel(vocab=vocab, unk_token="w0"))
    tk.pre_tokenizer = pre_tokenizers.WhitespaceSplit()
    tj = str(model_dir / "words.json")
    tk.save(tj)
    return path, tj, g, eos_at


def test_tokenizer_prompt_config_matches_oracle(gpu, c0_tok, model_dir):
    path, _, g, eos_at = c0_tok
    m = E.LoadedModel.load(path)
    t = m.tokenizer_prompt()
    assert (bool(t.add_bos_token), bool(t.add_eos_token), t.bos_token_id, t.eos_token_id) == \
        O.Model(path).tokenizer_prompt() == (False, False, 1, g["tokens"][eos_at])
    p2 = synth.with_metadata(path, str(model_dir / "c0_tok2.gguf"), [
        ("tokenizer.ggml.add_bos_token", synth.GGUF_BOOL, True), ("tokenizer.ggml.bos_token_id", synth.GGUF_I64, 17)])
    t2 = E.LoadedModel.load(p2).tokenizer_prompt()
    assert (bool(t2.add_bos_token), bool(t2.add_eos_token), t2.bos_token_id, t2.eos_token_id) == \
        O.Model(p2).tokenizer_prompt() == (True, False, 17, g["tokens"][eos_at])


def test_generate_greedy_stops_at_eos(gpu, c0_tok):
    path, tj, g, eos_at = c0_tok
    m = E.LoadedModel.load(path)
    tok = F.Tokenizer.load_from_file(tj)
    prompt = " ".join(f"w{i}" for i in g["prompt"])
    assert tok.encode(prompt) == list(g["prompt"])
    text, ids = F.generate(m, tok, prompt, new_tokens=len(g["tokens"]))
    assert ids == g["tokens"][:eos_at]
    assert text == " ".join(f"w{i}" for i in g["tokens"][:eos_at])
    # without the EOS stop inside the budget the loop runs n tokens
    text, ids = F.generate(m, tok, prompt, new_tokens=eos_at - 1)
    assert ids == g["tokens"][:eos_at - 1]


def test_cli_main_prints_the_continuation(gpu, c0_tok, capsys):
    path, tj, g, eos_at = c0_tok
    prompt = " ".join(f"w{i}" for i in g["prompt"])
    assert F.main(["-m", path, "-t", tj, "-n", "32", prompt]) == 0
    assert capsys.readouterr().out.strip() == " ".join(f"w{i}" for i in g["tokens"][:eos_at])


def test_generate_bos_insertion_changes_the_prefill(gpu, c0_tok, model_dir):
    path, tj, g, _ = c0_tok
    p2 = synth.with_metadata(path, str(model_dir / "c0_bos.gguf"), [
        ("tokenizer.ggml.add_bos_token", synth.GGUF_BOOL, True), ("tokenizer.ggml.eos_token_id", synth.GGUF_U32, 31999)])
    m = E.LoadedModel.load(p2)
    tok = F.Tokenizer.load_from_file(tj)
    prompt = " ".join(f"w{i}" for i in g["prompt"])
    _, ids = F.generate(m, tok, prompt, new_tokens=6)
    r = O.Session(O.Model(p2))
    r.prefill(np.array([1] + list(g["prompt"]), np.uint32))
    want = []
    for _ in range(6):
        t = O.argmax(r.logits())
        if t == 31999:
            break
        want.append(t)
        r.decode(t)
    assert ids == want


def test_generate_temperature_matches_oracle_draws(gpu, c0_tok):
    """generate() with temperature = a manual loop drawing the same uniforms, each step's token the
    oracle's sample_temperature of the device's own logits (the logits themselves are held to the
    oracle by the end-to-end tests; over a 32000-token vocabulary at T = 0.8 the boundaries are
    ~3e-5 apart, closer than two logit vectors within 1e-5 of each other can be told apart)."""
    path, tj, g, _ = c0_tok
    m = E.LoadedModel.load(path)
    tok = F.Tokenizer.load_from_file(tj)
    prompt = " ".join(f"w{i}" for i in g["prompt"])
    text, ids = F.generate(m, tok, prompt, new_tokens=12, temperature=0.8, rng=random.Random(5))
    assert text == " ".join(f"w{i}" for i in ids)
    draws = random.Random(5)
    s = E.InferenceSession(m)
    s.prefill(np.array(g["prompt"], np.uint32))
    eos = m.tokenizer_prompt().eos_token_id
    want = []
    for _ in range(12):
        lg = s.logits_last_token()
        u = draws.random()
        if _margin(lg, 0.8, u) < 1e-6:
            ids = ids[:len(want)]
            break
        t = O.sample_temperature(lg, 0.8, u)
        assert E.sample_temperature_next_token(s, 0.8, u) == t
        if t == eos:
            break
        want.append(t)
        s.decode_token(t)
    assert len(want) >= 4 and ids == want
