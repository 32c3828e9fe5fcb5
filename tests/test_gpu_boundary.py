"""GPU parity of the drop-in boundary's host-buffer op entries and forward-level entries against
the CPU oracle, through the C ABI (include/iek.h).

Bars: dequantize, RoPE and residual add bit-exact; argmax exact; matmul within the fp32
reordering bound of the device-pointer tests; softmax / SwiGLU / GELU within a few ulp; decode
attention within 2e-6 relative L2 of the oracle's head loop (f32 cache; the kernel sums scores and
P.V in a different order). Forward-level runs are compared with the session-level calls on the same
model (identical kernels: bit-exact) and with the oracle (the logits bar of the engine tests).
"""
import math

import numpy as np
import pytest

import oracle as O
from inference_engine_rust_amd import engine as E
from inference_engine_rust_amd import synth

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

ORC = {E.Q4K: O.T_Q4K, E.Q6K: O.T_Q6K, E.Q8_0: O.T_Q8_0, E.F32: O.T_F32}
GGML = {E.Q4K: 12, E.Q6K: 14, E.Q8_0: 8}
LOGIT_REL_L2 = 1e-3


def rel_l2(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / np.linalg.norm(np.asarray(b, np.float64)))


def _weights(dt, k, n, seed):
    be = 1 if dt == E.F32 else E.BLOCK[dt][0]
    nel = k * n
    nb = (nel + be - 1) // be
    x = synth.normal(seed, f"hw{dt}_{k}_{n}", nb * be, 0.0, 0.02)
    return x[:nel].copy() if dt == E.F32 else synth.quantize(GGML[dt], x)


# ---- host-buffer op entries ----------------------------------------------------------------------

@pytest.mark.parametrize("dt,k,n,m", [(E.Q4K, 4096, 1024, 1), (E.Q6K, 1408, 512, 7), (E.Q8_0, 2048, 96, 33),
                                      (E.F32, 256, 300, 1), (E.Q4K, 512, 1408, 130)])
def test_host_matmul_matches_oracle(gpu, dt, k, n, m):
    w = _weights(dt, k, n, 5)
    a = synth.normal(6, f"ha{k}", m * k, 0.0, 1.0).reshape(m, k)
    want = O.matmul(ORC[dt], a, w, k, n)
    got = E.host_matmul(a, w, dt, n)
    assert got.shape == (m, n)
    assert rel_l2(got, want) < 1e-5
    # the same weight already resident in HBM (on_device = 1)
    dw = torch.from_numpy(np.ascontiguousarray(w).view(np.uint8)).to("cuda")
    torch.cuda.synchronize()
    got_dev = E.host_matmul(a, dw.numel(), dt, n, on_device_ptr=dw.data_ptr())
    assert np.array_equal(got, got_dev)


def test_host_matmul_errors(gpu):
    w = _weights(E.Q4K, 256, 4, 1)
    with pytest.raises(E.EngineError) as e:
        E.host_matmul(np.ones((1, 256), np.float32), w[:-1], E.Q4K, 4)
    assert e.value.kind == "MatMul"
    with pytest.raises(E.EngineError) as e:
        E.host_matmul(np.ones((1, 256), np.float32), w, 9, 4)
    assert e.value.kind == "MatMul"


@pytest.mark.parametrize("dt", [E.Q4K, E.Q6K, E.Q8_0])
def test_host_dequantize_bit_exact(gpu, dt):
    nb = 300
    x = synth.normal(dt, "hdq", nb * E.BLOCK[dt][0], 0.0, 0.5)
    blocks = synth.quantize(GGML[dt], x)
    got = E.host_dequantize(dt, blocks, nb)
    want = O.dequantize(ORC[dt], blocks, nb)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_host_elementwise_ops(gpu):
    rng = np.random.default_rng(0)
    x = rng.standard_normal(4096).astype(np.float32)
    y = rng.standard_normal(4096).astype(np.float32)
    w = rng.standard_normal(4096).astype(np.float32)
    # rmsnorm, one row and several rows
    np.testing.assert_allclose(E.host_rmsnorm(x, w, 1e-5), O.rmsnorm(x, w, 1e-5), rtol=2e-6, atol=1e-7)
    rows = rng.standard_normal((3, 512)).astype(np.float32)
    got = E.host_rmsnorm(rows, w[:512], 1e-6)
    for r in range(3):
        np.testing.assert_allclose(got[r], O.rmsnorm(rows[r], w[:512], 1e-6), rtol=2e-6, atol=1e-7)
    # rope: bit-exact over 8 heads (the host builds the same cos/sin table as the reference)
    heads = rng.standard_normal(8 * 128).astype(np.float32)
    got = E.host_rope(heads, 8, 128, 128, 10000.0, 77)
    want = np.concatenate([O.rope(heads[h * 128:(h + 1) * 128], 10000.0, 77, 128, 128) for h in range(8)])
    assert np.array_equal(got, want)
    ff = np.linspace(1.0, 3.0, 32).astype(np.float32)
    got = E.host_rope(heads[:128], 1, 128, 64, 1e6, 5, ff)
    assert np.array_equal(got, O.rope(heads[:128], 1e6, 5, 128, 64, ff))
    # softmax / swiglu / gelu / residual
    np.testing.assert_allclose(E.host_softmax(x), O.softmax(x), rtol=4e-6, atol=1e-12)
    np.testing.assert_allclose(E.host_swiglu(x, y), O.swiglu(x, y), rtol=4e-6, atol=1e-7)
    want = np.array([O.gelu_tanh(float(v)) for v in x], np.float32)
    np.testing.assert_allclose(E.host_gelu_tanh(x), want, rtol=4e-6, atol=1e-7)
    np.testing.assert_allclose(E.host_gelu_tanh(x, y), want * y, rtol=4e-6, atol=1e-7)
    assert np.array_equal(E.host_residual_add(x, y), O.residual_add(x, y))


def test_host_argmax_and_errors(gpu):
    rng = np.random.default_rng(1)
    logits = rng.standard_normal(32000).astype(np.float32)
    logits[[17, 31000]] = 9.0  # a tie: the first index wins (sampling.rs:25-49)
    assert E.host_argmax(logits) == 17 == O.argmax(logits)
    logits[5] = np.nan
    with pytest.raises(E.EngineError) as e:
        E.host_argmax(logits)
    assert e.value.kind == "Sampling"
    with pytest.raises(E.EngineError) as e:
        E.host_softmax(np.zeros(0, np.float32))
    assert e.value.kind == "Op"
    with pytest.raises(E.EngineError) as e:
        E.host_rope(np.zeros(4, np.float32), 1, 4, 6, 10000.0, 0)
    assert e.value.kind == "Op"


# ---- decode attention ----------------------------------------------------------------------------

ATT_CASES = [  # n_heads, n_kv, head_dim, total, window
    (32, 8, 128, 1, 0), (32, 8, 128, 37, 0), (32, 8, 128, 700, 0), (32, 8, 128, 3000, 512),
    (8, 1, 256, 300, 0), (8, 1, 512, 130, 64), (8, 2, 64, 65, 0), (4, 4, 128, 64, 0), (16, 2, 256, 2100, 0),
]


def _att_inputs(n_heads, n_kv, hd, total, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(n_heads * hd).astype(np.float32)
    k = rng.standard_normal(total * n_kv * hd).astype(np.float32)
    v = rng.standard_normal(total * n_kv * hd).astype(np.float32)
    return q, k, v


@pytest.mark.parametrize("n_heads,n_kv,hd,total,window", ATT_CASES)
def test_host_attention_decode_matches_oracle(gpu, n_heads, n_kv, hd, total, window):
    q, k, v = _att_inputs(n_heads, n_kv, hd, total, total + hd)
    scale = 1.0 / math.sqrt(hd)
    got = E.host_attention_decode(q, k, v, n_heads, n_kv, hd, total, window, scale)
    want = O.attention_decode(q, k, v, n_heads, n_kv, hd, total, window if window > 0 else -1, scale)
    assert rel_l2(got, want) < 2e-6


@pytest.mark.parametrize("kv_f32", [False, True])
@pytest.mark.parametrize("n_heads,n_kv,hd,total,window", [(32, 8, 128, 520, 0), (8, 1, 256, 1500, 1024),
                                                          (8, 1, 512, 90, 0), (32, 8, 64, 4100, 0)])
def test_dev_attention_decode_matches_oracle(gpu, kv_f32, n_heads, n_kv, hd, total, window):
    """Device entry over the session layout [n_kv][max_seq_len][head_dim]; an fp16 cache is
    compared with the oracle on the fp16-rounded K/V (the rounding is the cache's, not the op's)."""
    max_len = total + 77
    q, k, v = _att_inputs(n_heads, n_kv, hd, total, 3 * total + hd)
    if not kv_f32:
        k = k.astype(np.float16).astype(np.float32)
        v = v.astype(np.float16).astype(np.float32)
    scale = 1.0 / math.sqrt(hd)
    want = O.attention_decode(q, k, v, n_heads, n_kv, hd, total, window if window > 0 else -1, scale)
    dt = np.float32 if kv_f32 else np.float16
    kc = np.full((n_kv, max_len, hd), np.nan, dt)  # rows past the live keys must never be read
    vc = np.full((n_kv, max_len, hd), np.nan, dt)
    kc[:, :total] = k.reshape(total, n_kv, hd).transpose(1, 0, 2)
    vc[:, :total] = v.reshape(total, n_kv, hd).transpose(1, 0, 2)
    dq, dk, dv = (torch.from_numpy(np.ascontiguousarray(a)).to("cuda") for a in (q, kc, vc))
    out = torch.empty(n_heads * hd, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    for _ in range(2):  # the op leaves its counters cleared for the next call
        E.attention_decode(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), E.F32 if kv_f32 else E.F16, n_heads, n_kv,
                           hd, max_len, total, window, scale, out.data_ptr(), stream)
        got = out.cpu().numpy()
        assert rel_l2(got, want) < 2e-6


def test_attention_decode_errors(gpu):
    q, k, v = _att_inputs(8, 2, 64, 4, 0)
    for args, kind in [((8, 2, 64, 0, 0), "Op"), ((8, 3, 64, 4, 0), "Op"), ((8, 2, 96, 4, 0), "Op"),
                       ((32, 2, 64, 4, 0), "Op")]:
        with pytest.raises(E.EngineError) as e:
            E.host_attention_decode(q, k, v, *args, 1.0)
        assert e.value.kind == kind
    dq = torch.zeros(8 * 64, device="cuda")
    dk = torch.zeros(2 * 16 * 64, device="cuda")
    with pytest.raises(E.EngineError) as e:
        E.attention_decode(dq.data_ptr(), dk.data_ptr(), dk.data_ptr(), E.F32, 8, 2, 64, 16, 17, 0, 1.0,
                           dq.data_ptr())
    assert e.value.kind == "KvCache"


# ---- prefill attention ---------------------------------------------------------------------------

PREFILL_ATT_CASES = [  # n_heads, n_kv, head_dim, seq, window
    (32, 8, 128, 512, 0),    # C2's layer: one 16-query tile per wave, two workgroups per CU
    (32, 8, 128, 1, 0), (32, 8, 128, 17, 0), (32, 8, 128, 200, 50),  # ragged tiles, a window
    (32, 8, 128, 4100, 1000),  # eight waves of two query tiles per staged block, a window
    (8, 2, 64, 333, 0), (8, 2, 64, 4200, 0),  # head_dim 64, both launch shapes
    (4, 4, 128, 150, 0), (16, 2, 128, 97, 0),  # one query head per KV head; eight per KV head
    (8, 1, 256, 256, 0), (8, 1, 256, 300, 100), (8, 1, 512, 130, 64),  # Gemma-4 head layouts
]


@pytest.mark.parametrize("n_heads,n_kv,hd,seq,window", PREFILL_ATT_CASES)
def test_dev_attention_prefill_matches_oracle(gpu, n_heads, n_kv, hd, seq, window):
    """The session's prefill attention kernels through the op-level entry against the oracle's
    head loop (attention.rs:364-415): within the fp16-pair operand rounding, 2e-5 relative L2
    (the pairs keep 22 significant bits; the same bar holds the C2 and C4 prefill tests)."""
    rng = np.random.default_rng(seq * 7 + hd + window)
    q = rng.standard_normal(seq * n_heads * hd).astype(np.float32)
    k = rng.standard_normal(seq * n_kv * hd).astype(np.float32)
    v = rng.standard_normal(seq * n_kv * hd).astype(np.float32)
    scale = 1.0 / math.sqrt(hd)
    want = O.attention_prefill(q, k, v, seq, n_heads, n_kv, hd, window if window > 0 else -1, scale)
    dq, dk, dv = (torch.from_numpy(a).to("cuda") for a in (q, k, v))
    out = torch.full((seq * n_heads * hd,), float("nan"), dtype=torch.float32, device="cuda")
    E.attention_prefill(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), seq, n_heads, n_kv, hd, window, scale,
                        out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    assert rel_l2(got, want) < 2e-5, rel_l2(got, want)
    # per position: the worst row stays within the bar too (a wrong mask shows in single rows)
    g, w = got.reshape(seq, -1), want.reshape(seq, -1)
    worst = max(rel_l2(g[p], w[p]) for p in range(0, seq, max(1, seq // 64)))
    assert worst < 1e-4, worst


def test_dev_attention_prefill_beyond_fp16_range_and_errors(gpu):
    """Scores from inputs past 65 504 (the fp16 pairs' range) take the f32 kernel: still the
    oracle's result; and the entry's errors."""
    n_heads, n_kv, hd, seq = 8, 2, 128, 70
    rng = np.random.default_rng(11)
    q = rng.standard_normal(seq * n_heads * hd).astype(np.float32)
    k = (rng.standard_normal(seq * n_kv * hd) * 1e-3).astype(np.float32)
    v = rng.standard_normal(seq * n_kv * hd).astype(np.float32)
    q[5 * n_heads * hd + 3] = 2.0e5  # one query value beyond the pair range
    v[9 * n_kv * hd + 7] = -1.0e6    # one value row too
    scale = 1.0 / math.sqrt(hd)
    want = O.attention_prefill(q, k, v, seq, n_heads, n_kv, hd, -1, scale)
    dq, dk, dv = (torch.from_numpy(a).to("cuda") for a in (q, k, v))
    out = torch.empty(seq * n_heads * hd, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    E.attention_prefill(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), seq, n_heads, n_kv, hd, 0, scale,
                        out.data_ptr(), stream)
    assert rel_l2(out.cpu().numpy(), want) < 1e-5
    for args in [(seq, 8, 3, hd), (0, 8, 2, hd), (seq, 8, 2, 96)]:
        with pytest.raises(E.EngineError) as e:
            E.attention_prefill(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), *args, 0, scale, out.data_ptr(), stream)
        assert e.value.kind == "Op"


# ---- forward level -------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def c0_gpu(gpu, c0_path):
    return E.LoadedModel.load(c0_path)


def test_forward_level_equals_session_level(c0_gpu):
    """embed + prefill_forward == prefill; embed(1) + decode_forward == decode_token; layer by
    layer == the whole forward (same kernels: bit-exact)."""
    prompt = synth.prompt_ids(3, 24)
    a, b, c = (E.InferenceSession(c0_gpu) for _ in range(3))
    a.prefill(prompt)
    b.embed(prompt)
    assert b.kv_len() == 0 and b.hidden().shape == (24, 512)
    b.prefill_forward()
    c.embed(prompt)
    for li in range(c0_gpu.config.n_layers):
        c.prefill_layer_block(li)
    for s in (b, c):
        assert s.kv_len() == 24
        assert np.array_equal(s.hidden(), a.hidden())
        assert np.array_equal(s.logits_last_token(), a.logits_last_token())
    for step in range(4):
        t = E.greedy_next_token(a)
        assert E.greedy_next_token(b) == t == E.greedy_next_token(c)
        a.decode_token(t)
        b.embed([t])
        b.decode_forward()
        c.embed([t])
        for li in range(c0_gpu.config.n_layers):
            c.decode_layer_block(li)
        for s in (b, c):
            assert s.kv_len() == 25 + step
            assert np.array_equal(s.hidden(), a.hidden())
            assert np.array_equal(s.logits_last_token(), a.logits_last_token())


def test_forward_level_layers_match_oracle(c0_gpu, c0_path):
    """After layer l of a layer-level prefill the state equals the oracle's prefill through l + 1
    layers; set_hidden (ForwardState::from_flat) of the embedding rows runs the same forward."""
    prompt = synth.prompt_ids(4, 12)
    om = O.Model(c0_path)
    s = E.InferenceSession(c0_gpu)
    s.embed(prompt)
    emb = s.hidden()
    for li in range(c0_gpu.config.n_layers):
        s.prefill_layer_block(li)
        r = O.Session(om)
        r.set_layer_limit(li + 1)
        r.prefill(prompt)
        assert rel_l2(s.hidden(), r.hidden()) < 1e-5, li
    t = E.InferenceSession(c0_gpu)
    t.set_hidden(emb)
    t.prefill_forward()
    assert np.array_equal(t.hidden(), s.hidden())
    r = O.Session(om)
    r.prefill(prompt)
    assert rel_l2(t.logits_last_token(), r.logits()) < LOGIT_REL_L2


def test_forward_level_errors(c0_gpu):
    s = E.InferenceSession(c0_gpu)
    s.embed(synth.prompt_ids(0, 6))
    with pytest.raises(E.EngineError) as e:
        s.prefill_layer_block(1)  # layers run in order
    assert e.value.kind == "Model"
    s.prefill_layer_block(0)
    for call in (lambda: s.decode_token(1), lambda: E.greedy_next_token(s), s.logits_last_token,
                 lambda: s.generate_greedy(2)):
        with pytest.raises(E.EngineError) as e:
            call()
        assert e.value.kind == "Model" and "in progress" in str(e.value)
    with pytest.raises(E.EngineError) as e:
        s.decode_layer_block(1)  # a six-row state is not a decode state
    assert e.value.kind == "Model"
    s.prefill_layer_block(1)
    assert s.kv_len() == 6
    s.decode_token(E.greedy_next_token(s))  # a completed layer-level forward is a normal state
    assert s.kv_len() == 7
    with pytest.raises(E.EngineError) as e:
        s.set_hidden(np.zeros((0, 512), np.float32))
    assert e.value.kind == "Model"
    with pytest.raises(E.EngineError) as e:
        s.embed([c0_gpu.config.vocab_size])
    assert e.value.kind == "Model"


def test_gemma_forward_level_matches_oracle(gpu, model_dir):
    """Gemma-4 (per-layer inputs, KV borrowing, sliding window): layer-level prefill and decode
    against the oracle, and against the session-level calls."""
    p = str(model_dir / "g0_fwd.gguf")
    synth.write_gemma4(p, synth.preset("g0"), seed=0)
    m = E.LoadedModel.load(p)
    om = O.Model(p)
    prompt = synth.prompt_ids(2, 20, 8192)
    s, a = E.InferenceSession(m), E.InferenceSession(m)
    r = O.Session(om)
    s.embed(prompt)
    for li in range(m.config.n_layers):
        s.prefill_layer_block(li)
    a.prefill(prompt)
    r.prefill(prompt)
    assert np.array_equal(s.hidden(), a.hidden())
    assert rel_l2(s.logits_last_token(), r.logits()) < LOGIT_REL_L2
    for step in range(3):
        t = O.argmax(r.logits())
        assert E.greedy_next_token(s) == t
        s.embed([t])
        for li in range(m.config.n_layers):
            s.decode_layer_block(li)
        r.decode(t)
        assert rel_l2(s.logits_last_token(), r.logits()) < LOGIT_REL_L2, step
    with pytest.raises(E.EngineError) as e:
        t = E.InferenceSession(m)
        t.set_hidden(np.zeros((2, m.config.hidden_dim), np.float32))
        t.prefill_forward()  # no per-layer inputs in a from_flat state
    assert e.value.kind == "Model"
