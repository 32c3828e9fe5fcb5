"""Pinning of the CPU oracle's Gemma-4 path (A14, A23 wiring, A32) on the seeded tiny Gemma-4
model ``g0``: 6 layers (2 global with head dim 128, partial rotary 32 and freq factors; 4 sliding
with head dim 64 and window 16), KV borrowing in the last 2 layers, per-layer embeddings of 32,
layer output scales in both encodings (F32 and one Q8_0 block), tied Q8_0 LM head, soft cap 30.

* whole-model recomposition from the separately pinned ops (matmul, rmsnorm, rmsnorm_no_scale,
  rope with freq factors, gelu_tanh) around a brute-force float64 windowed GQA attention
  (attention.rs:175-422, ffn.rs:16-278, gemma4_ple.rs:27-109, runtime.rs:76-116);
* prefill [t0..tN] vs prefill [t0..tN-1] + decode tN, with the prompt longer than the window
  (tests/gemma_decode_self_consistency.rs:219-320 runs the same check on a real Gemma GGUF);
* greedy loop == teacher-forced re-prefill;
* config resolution of the Gemma-4 metadata (model_config.rs:332-372, 374-444, 515-629);
* BF16 weights widen to the exact f32 of their bits (tensor_loader.rs:11-16, 39-54).
"""
import numpy as np
import pytest

import oracle as O
from inference_engine_rust_amd import synth

SPEC = synth.preset("g0")


@pytest.fixture(scope="module")
def g0_path(model_dir):
    p = str(model_dir / "g0.gguf")
    synth.write_gemma4(p, SPEC, seed=0)
    return p


@pytest.fixture(scope="module")
def g0(g0_path):
    return O.Model(g0_path)


def test_gemma_config_resolution(g0):
    c = g0.cfg
    assert c.family == 1
    assert (c.hidden_dim, c.n_layers, c.n_heads, c.n_kv_heads, c.vocab_size, c.ple_dim) == (256, 6, 4, 1, 8192, 32)
    assert c.head_dim == 128 and c.ffn_dim == 512  # maxima over layers (model_config.rs:420-444)
    assert c.unpack_qk == 0 and c.has_softcap == 1 and c.softcap == 30.0
    for li in range(SPEC.n_layers):
        sp = g0.layer_spec(li)
        swa = SPEC.is_swa(li)
        assert sp["head_dim"] == SPEC.head_dim(li)
        assert sp["sliding_window"] == (SPEC.sliding_window if swa else -1)
        assert sp["rope_theta"] == (SPEC.theta_swa if swa else SPEC.theta_global)
        assert sp["rotary_dim"] == (SPEC.rot_swa if swa else SPEC.rot_global)
    # shared-KV layers 4 (sliding) and 5 (global) borrow the last earlier layer of their kind
    assert [g0.layer_spec(li)["kv_borrow"] for li in range(6)] == [-1, -1, -1, -1, 3, 2]


def test_bf16_weights_widen_exactly(g0):
    dt, raw, k, n = g0.tensor("per_layer_model_proj.weight")
    assert dt == O.T_F32 and (k, n) == (256, 6 * 32)
    want = synth.normal(0, "per_layer_model_proj.weight", k * n, 0.0, SPEC.weight_std)
    bits = want.view(np.uint32).astype(np.uint64)
    rne = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint32) << 16
    np.testing.assert_array_equal(raw.view(np.uint32), rne)


def _vec(m, name):
    dt, raw, _, _ = m.tensor(name)
    assert dt == O.T_F32
    return raw.view(np.float32)


def _rows(m, name, ids):
    """Embedding rows of a Q8_0 [width, vocab] table (embeddings.rs:95-210)."""
    dt, raw, width, _ = m.tensor(name)
    assert dt == O.T_Q8_0
    nb = width // 32
    return np.stack([O.dequantize(dt, raw[t * nb * 34:(t + 1) * nb * 34], nb) for t in ids])


def _mat(m, name, a, k, n):
    dt, raw, k0, n0 = m.tensor(name)
    assert (k0, n0) == (k, n), name
    return O.matmul(dt, np.ascontiguousarray(a, np.float32), raw, k, n)


_gelu = np.vectorize(O.gelu_tanh, otypes=[np.float32])


def _attention(q, k, v, nh, nkv, hd, window):
    """Brute-force float64 causal GQA attention with scale 1 and an optional sliding window
    (key j visible from query p iff p - (window - 1) <= j <= p)."""
    m = q.shape[0]
    out = np.zeros((m, nh * hd), np.float64)
    p = np.arange(m)[:, None]
    j = np.arange(m)[None, :]
    mask = j <= p
    if window > 0:
        mask &= j >= p - (window - 1)
    for h in range(nh):
        kvh = h // (nh // nkv)
        sc = q[:, h * hd:(h + 1) * hd].astype(np.float64) @ k[:, kvh * hd:(kvh + 1) * hd].astype(np.float64).T
        sc = np.where(mask, sc, -np.inf)
        w = np.exp(sc - sc.max(axis=1, keepdims=True))
        w /= w.sum(axis=1, keepdims=True)
        out[:, h * hd:(h + 1) * hd] = w @ v[:, kvh * hd:(kvh + 1) * hd].astype(np.float64)
    return out.astype(np.float32)


def _layer_scale(m, li):
    dt, raw, _, _ = m.tensor(f"blk.{li}.layer_output_scale.weight")
    if dt == O.T_F32:
        return raw.view(np.float32)[0]
    return O.dequantize(dt, raw[:34], 1)[0]


def test_gemma_model_recomposed_from_pinned_ops(g0):
    """Pins the Gemma-4 wiring: a wrong PLE packing order or scale, a missing q/k/v norm, the
    post-norms applied to the wrong tensor, the layer scale applied before the PLE tail, a wrong
    borrow source, window bound, per-layer RoPE parameters or soft cap each move the logits by far
    more than the tolerance."""
    c = g0.cfg
    M = 20  # longer than the window of 16
    ids = synth.prompt_ids(0, M, c.vocab_size)
    H, nh, nkv, pd, L, eps = c.hidden_dim, c.n_heads, c.n_kv_heads, c.ple_dim, c.n_layers, c.rms_norm_eps
    x = _rows(g0, "token_embd.weight", ids) * np.float32(np.sqrt(np.float32(H)))
    x = x.astype(np.float32)
    # per-layer inputs
    proj = _mat(g0, "per_layer_model_proj.weight", x, H, L * pd) * np.float32(1.0 / np.sqrt(np.float32(H)))
    tok = _rows(g0, "per_layer_token_embd.weight", ids) * np.float32(np.sqrt(np.float32(pd)))
    pnw = _vec(g0, "per_layer_proj_norm.weight")
    packed = np.zeros((M, L * pd), np.float32)
    for p in range(M):
        for li in range(L):
            sl = slice(li * pd, (li + 1) * pd)
            packed[p, sl] = (O.rmsnorm(proj[p, sl].astype(np.float32), pnw, eps) + tok[p, sl]) * np.float32(
                1.0 / np.sqrt(np.float32(2.0)))
    kv = {}
    for li in range(L):
        sp = g0.layer_spec(li)
        hd, rot, theta, window, borrow = sp["head_dim"], sp["rotary_dim"], sp["rope_theta"], sp["sliding_window"], \
            sp["kv_borrow"]
        b = f"blk.{li}."
        xn = np.stack([O.rmsnorm(r, _vec(g0, b + "attn_norm.weight"), eps) for r in x])
        q = _mat(g0, b + "attn_q.weight", xn, H, nh * hd)
        ff = _vec(g0, b + "rope_freqs.weight") if not SPEC.is_swa(li) else None
        qn = _vec(g0, b + "attn_q_norm.weight")
        for p in range(M):
            q[p] = np.concatenate([O.rope(O.rmsnorm(q[p, h * hd:(h + 1) * hd], qn, eps), theta, p, hd, rot, ff)
                                   for h in range(nh)])
        if borrow < 0:
            k = _mat(g0, b + "attn_k.weight", xn, H, nkv * hd)
            v = _mat(g0, b + "attn_v.weight", xn, H, nkv * hd)
            kn = _vec(g0, b + "attn_k_norm.weight")
            for p in range(M):
                k[p] = np.concatenate([O.rope(O.rmsnorm(k[p, h * hd:(h + 1) * hd], kn, eps), theta, p, hd, rot, ff)
                                       for h in range(nkv)])
                v[p] = np.concatenate([O.rmsnorm_no_scale(v[p, h * hd:(h + 1) * hd], eps) for h in range(nkv)])
            kv[li] = (k, v)
        else:
            k, v = kv[borrow]
        att = _attention(q, k, v, nh, nkv, hd, window)
        ao = _mat(g0, b + "attn_output.weight", att, nh * hd, H)
        x = x + np.stack([O.rmsnorm(r, _vec(g0, b + "post_attention_norm.weight"), eps) for r in ao])
        xn = np.stack([O.rmsnorm(r, _vec(g0, b + "ffn_norm.weight"), eps) for r in x])
        g = _mat(g0, b + "ffn_gate.weight", xn, H, c.ffn_dim)
        u = _mat(g0, b + "ffn_up.weight", xn, H, c.ffn_dim)
        dn = _mat(g0, b + "ffn_down.weight", _gelu(g) * u, c.ffn_dim, H)
        x = x + np.stack([O.rmsnorm(r, _vec(g0, b + "post_ffw_norm.weight"), eps) for r in dn])
        go = _gelu(_mat(g0, b + "inp_gate.weight", x, H, pd)) * packed[:, li * pd:(li + 1) * pd]
        po = _mat(g0, b + "proj.weight", go, pd, H)
        x = x + np.stack([O.rmsnorm(r, _vec(g0, b + "post_norm.weight"), eps) for r in po])
        x = (x * _layer_scale(g0, li)).astype(np.float32)
    last = O.rmsnorm(x[-1], _vec(g0, "output_norm.weight"), eps)
    z = _mat(g0, "token_embd.weight", last[None, :], H, c.vocab_size)[0]
    want = (30.0 * np.tanh(z.astype(np.float64) / 30.0))
    s = O.Session(g0)
    s.prefill(ids)
    got = s.logits()
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < 1e-5, rel
    assert O.argmax(got) == int(np.argmax(want))


def test_gemma_prefill_vs_prefill_plus_decode(g0):
    ids = synth.prompt_ids(0, 21, SPEC.vocab)
    a = O.Session(g0)
    a.prefill(ids)
    la = a.logits()
    b = O.Session(g0)
    b.prefill(ids[:-1])
    b.decode(int(ids[-1]))
    lb = b.logits()
    assert np.max(np.abs(la - lb)) < 1e-4
    np.testing.assert_allclose(a.hidden()[-1], b.hidden()[-1], rtol=0, atol=1e-4)


def test_gemma_decode_loop_matches_teacher_forcing(g0):
    ids = list(synth.prompt_ids(0, 12, SPEC.vocab))
    s = O.Session(g0)
    toks, _ = O.greedy_generate(s, ids, 8)  # crosses the window of 16
    seq = list(ids)
    for t in toks:
        r = O.Session(g0)
        r.prefill(seq)
        assert O.argmax(r.logits()) == t
        seq.append(t)


def test_gemma_borrowing_layers_keep_no_cache_of_their_own(g0):
    s = O.Session(g0)
    s.prefill(synth.prompt_ids(0, 5, SPEC.vocab))
    assert [s.kv_len(li) for li in range(6)] == [5, 5, 5, 5, 0, 0]
