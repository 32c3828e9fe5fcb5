"""CPU checks of the drop-in boundary: libiek.so loads and exports every entry point declared in
include/iek.h; the Python mirror binds each of them; synthetic GGUFs are deterministic."""
import ctypes
import hashlib
import os
import re

from inference_engine_rust_amd import engine, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    txt = open(os.path.join(ROOT, "include", "iek.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(iek_[a-z0-9_]+)\s*\(", txt)))


def test_header_declares_entry_points():
    names = _declared()
    for n in ["iek_model_load", "iek_session_prefill", "iek_session_decode_token", "iek_session_logits_last_token",
              "iek_greedy_next_token", "iek_matmul", "iek_dequantize", "iek_attention_decode",
              "iek_session_prefill_forward", "iek_session_decode_forward", "iek_session_prefill_layer_block",
              "iek_session_decode_layer_block", "iek_dev_matmul", "iek_dev_attention_decode"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(engine.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_mirror_binds_every_symbol():
    assert set(_declared()) == set(engine.EXPORTS)
    engine.lib()  # sets argtypes for every export; raises if one is missing


def test_missing_model_file_is_model_error():
    try:
        engine.LoadedModel.load("/nonexistent/model.gguf")
    except engine.EngineError as e:
        assert e.kind == "Model"
    else:
        raise AssertionError("expected EngineError")


def test_synth_is_deterministic(tmp_path):
    spec = synth.preset("c0", n_layers=1, vocab=512)
    a, b, c = (str(tmp_path / n) for n in ("a.gguf", "b.gguf", "c.gguf"))
    synth.write_llama(a, spec, seed=7, threads=1)
    synth.write_llama(b, spec, seed=7, threads=8)
    synth.write_llama(c, spec, seed=8)
    h = [hashlib.sha256(open(p, "rb").read()).hexdigest() for p in (a, b, c)]
    assert h[0] == h[1] and h[0] != h[2]
