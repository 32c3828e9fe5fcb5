"""Model-level invariants of the CPU oracle on the seeded tiny Mistral-architecture model.

* prefill [t0..tN] vs prefill [t0..tN-1] + decode tN         (tests/prefill_smoke.rs:99-144)
* greedy decode loop == teacher-forced re-prefill argmax     (tests/gemma_decode_self_consistency.rs:219-320)
* parity mode == baseline (reference Rayon decomposition) bit for bit
* config resolution of the synthetic GGUF (model_config.rs:143-306)
"""
import json
import os

import numpy as np
import pytest

import oracle as O
from inference_engine_rust_amd import synth

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def c0(c0_path):
    return O.Model(c0_path)


def test_config_resolution(c0):
    c = c0.cfg
    assert (c.hidden_dim, c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn_dim, c.vocab_size) == (
        512, 2, 8, 2, 64, 1408, 32000)
    assert c.rope_theta == 10000.0 and abs(c.rms_norm_eps - 1e-5) < 1e-12
    assert c.unpack_qk == 0  # general.name contains "mistral" (model_config.rs:209-224)
    spec = c0.layer_spec(0)
    assert spec["sliding_window"] == -1 and spec["rotary_dim"] == 64 and spec["kv_borrow"] == -1


def test_rope_theta_key_resolution(c0_path, tmp_path):
    """model_config.rs:160-162: llama.rope.theta, else gemma4.rope.freq_base, else 10000; a
    llama.rope.freq_base key (llama.cpp's name) is not read."""
    F = synth.GGUF_F32
    cases = [([("llama.rope.theta", F, 50000.0), ("llama.rope.freq_base", F, 10000.0)], 50000.0),
             ([("llama.rope.freq_base", F, 77000.0)], 10000.0),
             ([("gemma4.rope.freq_base", F, 30000.0)], 10000.0),  # the synthetic file holds llama.rope.theta
             ([("llama.rope.theta", F, 20000.0), ("gemma4.rope.freq_base", F, 30000.0)], 20000.0)]
    logits = {}
    ids = synth.prompt_ids(1, 24)
    for i, (entries, want) in enumerate(cases):
        p = synth.with_metadata(c0_path, str(tmp_path / f"theta{i}.gguf"), entries)
        m = O.Model(p)
        assert m.cfg.rope_theta == want and m.layer_spec(0)["rope_theta"] == want, (entries, m.cfg.rope_theta)
        s = O.Session(m)
        s.prefill(ids)
        logits[want] = s.logits()
    # the base reaches the rotation: another base gives other logits
    assert np.max(np.abs(logits[50000.0] - logits[10000.0])) > 1e-3


def test_prefill_vs_prefill_plus_decode(c0):
    ids = synth.prompt_ids(0, 9)
    a = O.Session(c0)
    a.prefill(ids)
    la = a.logits()
    b = O.Session(c0)
    b.prefill(ids[:-1])
    b.decode(int(ids[-1]))
    lb = b.logits()
    assert np.max(np.abs(la - lb)) < 1e-3


def test_decode_loop_matches_teacher_forcing(c0):
    ids = list(synth.prompt_ids(0, 6))
    s = O.Session(c0)
    toks, _ = O.greedy_generate(s, ids, 5)
    seq = list(ids)
    for t in toks:
        r = O.Session(c0)
        r.prefill(seq)
        assert O.argmax(r.logits()) == t
        seq.append(t)


def test_parity_mode_equals_baseline_mode(c0):
    ids = synth.prompt_ids(0, 16)
    p = O.Session(c0, O.PARITY)
    b = O.Session(c0, O.BASELINE, 3)
    tp, lp = O.greedy_generate(p, ids, 4, record_logits=True)
    tb, lb = O.greedy_generate(b, ids, 4, record_logits=True)
    assert tp == tb
    for x, y in zip(lp, lb):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))


def test_c0_golden_tokens(c0):
    """Greedy tokens of the benchmark's tiny config, frozen when the oracle was pinned."""
    with open(os.path.join(GOLDEN, "c0_seed0.json")) as f:
        g = json.load(f)
    s = O.Session(c0)
    toks, logs = O.greedy_generate(s, np.array(g["prompt"], np.uint32), g["n_decode"], record_logits=True)
    assert toks == g["tokens"]
    np.testing.assert_allclose([float(l[t]) for l, t in zip(logs, toks)], g["top_logits"], rtol=1e-6)


def test_errors(c0):
    s = O.Session(c0)
    with pytest.raises(O.OracleError) as e:
        s.prefill(np.zeros(0, np.uint32))
    assert e.value.code == 6
    with pytest.raises(O.OracleError) as e:
        s.prefill(np.array([32000], np.uint32))
    assert e.value.code == 6
    with pytest.raises(O.OracleError) as e:
        s.prefill(np.arange(65, dtype=np.uint32))  # > context_length (64)
    assert e.value.code == 6
    s.prefill(np.arange(3, 67, dtype=np.uint32))  # exactly full
    with pytest.raises(O.OracleError) as e:
        s.decode(5)
    assert e.value.code == 8  # KVCacheFull (attention.rs:55-59)


def test_layer0_recomposed_with_brute_force_attention(c0):
    """Pins the oracle's layer composition and attention (A13/A15/A18/A22/A24/A25) against an
    independent recomposition: layer 0 of C0 rebuilt from the separately pinned ops (matmul,
    rmsnorm, rope, swiglu) around a brute-force float64 causal GQA attention. A wrong GQA head
    map, score scale, causal bound or residual wiring moves the result by O(1)."""
    m = 16
    prompt = synth.prompt_ids(0, m)
    s = O.Session(c0)
    s.set_layer_limit(1)
    s.prefill(prompt)
    want = s.hidden()
    c = c0.cfg
    H, nh, nkv, hd, F, eps = c.hidden_dim, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn_dim, c.rms_norm_eps

    def mat(name, a, k, n):
        dt, raw, k0, n0 = c0.tensor(name)
        assert (k0, n0) == (k, n)
        return O.matmul(dt, a, raw, k, n)

    def vec(name):
        dt, raw, _, _ = c0.tensor(name)
        assert dt == O.T_F32
        return raw.view(np.float32)

    dt, raw, _, _ = c0.tensor("token_embd.weight")
    per_row = H // 256 * 144
    x = np.stack([O.dequantize(dt, raw[t * per_row:(t + 1) * per_row], H // 256) for t in prompt])
    xn = np.stack([O.rmsnorm(r, vec("blk.0.attn_norm.weight"), eps) for r in x])
    q = mat("blk.0.attn_q.weight", xn, H, nh * hd)
    k = mat("blk.0.attn_k.weight", xn, H, nkv * hd)
    v = mat("blk.0.attn_v.weight", xn, H, nkv * hd)
    for p in range(m):
        q[p] = np.concatenate([O.rope(q[p, h * hd:(h + 1) * hd], 10000.0, p, hd, hd) for h in range(nh)])
        k[p] = np.concatenate([O.rope(k[p, h * hd:(h + 1) * hd], 10000.0, p, hd, hd) for h in range(nkv)])
    att = np.zeros((m, nh * hd), np.float64)
    for h in range(nh):
        kvh = h // (nh // nkv)
        qh = q[:, h * hd:(h + 1) * hd].astype(np.float64)
        kh = k[:, kvh * hd:(kvh + 1) * hd].astype(np.float64)
        vh = v[:, kvh * hd:(kvh + 1) * hd].astype(np.float64)
        sc = qh @ kh.T / np.sqrt(hd)
        sc[np.triu_indices(m, 1)] = -np.inf
        w = np.exp(sc - sc.max(axis=1, keepdims=True))
        w /= w.sum(axis=1, keepdims=True)
        att[:, h * hd:(h + 1) * hd] = w @ vh
    x1 = x + mat("blk.0.attn_output.weight", att.astype(np.float32), nh * hd, H)
    xn1 = np.stack([O.rmsnorm(r, vec("blk.0.ffn_norm.weight"), eps) for r in x1])
    g = mat("blk.0.ffn_gate.weight", xn1, H, F)
    u = mat("blk.0.ffn_up.weight", xn1, H, F)
    act = np.stack([O.swiglu(g[i], u[i]) for i in range(m)])
    got = x1 + mat("blk.0.ffn_down.weight", act, F, H)
    rel = np.linalg.norm(got.astype(np.float64) - want) / np.linalg.norm(want.astype(np.float64))
    assert rel < 1e-5, rel
