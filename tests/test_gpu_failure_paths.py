"""Session-level failure paths through the C ABI, against the CPU oracle.

* Non-finite logits (src/engine/sampling.rs:25-49: greedy_next_token fails with
  SamplingError::InvalidLogits): an output head whose first Q6_K superblock has d = +inf, and a
  token embedding row whose first Q4_K superblock has d = NaN, planted in the GGUF bytes. The
  greedy loop of src/main.rs:100-116 then stops at the first step whose logits are not finite;
  iek_session_generate_greedy reports IEK_ERR_SAMPLING and leaves the KV length the reference loop
  leaves. Both decode implementations run: the decode chain (a model whose widths it takes) and
  the per-launch kernels (C0, whose FFN width 1408 the chain does not take).
* The decode chain's bounded waits (kernels/chain.hip), given up on purpose through the test knob
  iek_session_set_chain_spin: every kernel exits normally, the step fails with IEK_ERR_DEVICE, and
  a reset session decodes exactly as a fresh one.
"""
import dataclasses

import numpy as np
import pytest

import oracle as O
from inference_engine_rust_amd import engine as E
from inference_engine_rust_amd import synth

pytestmark = pytest.mark.gpu

F16_INF, F16_NAN = b"\x00\x7c", b"\x00\x7e"
Q4K_BYTES, Q6K_BYTES = 144, 210
# the decode chain takes this model (hidden and FFN widths multiples of 256, one 4096-wide pass)
CHAIN_SPEC = dataclasses.replace(synth.PRESETS["c0"], name="synthetic-mistral-chain", hidden=1024, n_heads=8,
                                 n_kv_heads=2, ffn=2816, context_length=128)
SPECS = {"chain": CHAIN_SPEC, "per_launch": synth.preset("c0")}
N_PROMPT = 12


def _model(tmp_path, kind, seed=0):
    p = str(tmp_path / f"{kind}.gguf")
    synth.write_llama(p, SPECS[kind], seed=seed)
    return p


def _sessions(p):
    m = E.LoadedModel.load(p)
    return m, E.InferenceSession(m), O.Session(O.Model(p))


@pytest.mark.parametrize("kind", ["chain", "per_launch"])
def test_infinite_head_scale_fails_sampling_at_step_zero(gpu, tmp_path, kind):
    p = _model(tmp_path, kind)
    synth.patch_bytes(p, "output.weight", 208, F16_INF)  # Q6_K d of row 0's first superblock
    m, s, r = _sessions(p)
    assert (s.decode_path() >= 1) == (kind == "chain")
    prompt = synth.prompt_ids(3, N_PROMPT)
    s.prefill(prompt)
    r.prefill(prompt)
    assert not np.isfinite(r.logits()[0]) and O.argmax(r.logits()) == -2  # the oracle: InvalidLogits
    assert not np.isfinite(s.logits_last_token()[0])
    with pytest.raises(E.EngineError) as e:
        E.greedy_next_token(s)
    assert e.value.kind == "Sampling"
    with pytest.raises(E.EngineError) as e:
        s.generate_greedy(4)
    assert e.value.kind == "Sampling" and "step 0" in str(e.value)
    assert s.kv_len() == N_PROMPT  # the loop stopped before its first decode_token


@pytest.mark.parametrize("kind", ["chain", "per_launch"])
def test_nan_embedding_row_stops_the_loop_after_that_token(gpu, tmp_path, kind):
    p = _model(tmp_path, kind, seed=1)
    # the oracle's greedy tokens on the unpatched model; the planted token is the first one, from
    # the third on, that is neither in the prompt nor generated before it, taken where no earlier
    # step is a near-tie (a device that sums in another order must reach the same token k); the
    # first prompt seed that has such a step
    om = O.Model(p)
    for prompt_seed in range(4, 20):
        prompt = synth.prompt_ids(prompt_seed, N_PROMPT)
        clean, logs = O.greedy_generate(O.Session(om), prompt, 12, record_logits=True)
        gaps = [float(np.diff(np.sort(lg.astype(np.float64))[-2:])[0]) for lg in logs]
        ok = [i for i in range(2, len(clean)) if clean[i] not in set(prompt.tolist()) | set(clean[:i])]
        ks = [i for i in ok if min(gaps[: i + 1]) >= 2e-2]
        if ks:
            k = ks[0]
            break
    else:
        pytest.fail("no prompt seed in 4..19 has a step without an earlier near-tie")
    del om
    hid = SPECS[kind].hidden
    synth.patch_bytes(p, "token_embd.weight", clean[k] * (hid // 256) * Q4K_BYTES, F16_NAN)
    m, s, r = _sessions(p)
    # the oracle: the same tokens through step k; decoding token k gives non-finite logits
    r.prefill(prompt)
    for i in range(k + 1):
        assert O.argmax(r.logits()) == clean[i]
        r.decode(clean[i])
    assert O.argmax(r.logits()) == -2
    # the device's replayed loop fails at step k + 1 with the reference loop's KV length
    s.prefill(prompt)
    with pytest.raises(E.EngineError) as e:
        s.generate_greedy(k + 4)
    assert e.value.kind == "Sampling" and f"step {k + 1}" in str(e.value), str(e.value)
    assert s.kv_len() == N_PROMPT + k + 1
    assert not np.isfinite(s.logits_last_token()).all()  # the state of the reference loop: token k decoded
    # the step-by-step loop fails at the same step
    s.reset()
    s.prefill(prompt)
    for i in range(k + 1):
        t = E.greedy_next_token(s)
        assert t == clean[i], i
        s.decode_token(t)
    with pytest.raises(E.EngineError) as e:
        E.greedy_next_token(s)
    assert e.value.kind == "Sampling"


def test_chain_bounded_wait_gives_up_cleanly(gpu, tmp_path):
    p = _model(tmp_path, "chain", seed=2)
    m = E.LoadedModel.load(p)
    s, fresh = E.InferenceSession(m), E.InferenceSession(m)
    assert s.decode_path() >= 1
    prompt = synth.prompt_ids(5, N_PROMPT)
    fresh.prefill(prompt)
    t0 = E.greedy_next_token(fresh)
    fresh.decode_token(t0)
    want = fresh.logits_last_token()
    want_ids = fresh.generate_greedy(3)
    for spin in (1, 2):
        s.reset()
        s.prefill(prompt)
        s.set_chain_spin(spin)
        with pytest.raises(E.EngineError) as e:
            s.decode_token(t0)
        assert e.value.kind == "Device" and "bounded wait" in str(e.value)
        s.reset()
        s.prefill(prompt)
        with pytest.raises(E.EngineError) as e:
            s.generate_greedy(3)  # the captured step graph reads the limit at each launch
        assert e.value.kind == "Device"
        s.set_chain_spin(0)
        s.reset()
        s.prefill(prompt)
        s.decode_token(t0)
        np.testing.assert_array_equal(s.logits_last_token(), want)
        assert s.generate_greedy(3) == want_ids
