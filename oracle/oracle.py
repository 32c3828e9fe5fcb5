"""TEST INFRASTRUCTURE ONLY — ctypes wrapper of the CPU oracle (liboracle.so).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use this module, and
only as the checker or as the timed CPU baseline. The product never imports it.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

T_F32, T_Q4K, T_Q6K, T_Q8_0 = 0, 1, 2, 3
GGML_TO_ORC = {0: T_F32, 12: T_Q4K, 14: T_Q6K, 8: T_Q8_0}
PARITY, BASELINE, REASSOC, PAIR, F16, I8X2_ROW, I8X2_B32, I8X3_ROW = 0, 1, 2, 3, 4, 5, 6, 7

_f = ctypes.c_void_p


class OracleError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"oracle error {code}: {msg}")
        self.code = code


class Cfg(ctypes.Structure):
    _fields_ = [("family", ctypes.c_int32), ("context_length", ctypes.c_uint64), ("hidden_dim", ctypes.c_uint64),
                ("n_layers", ctypes.c_uint64), ("n_heads", ctypes.c_uint64), ("n_kv_heads", ctypes.c_uint64),
                ("head_dim", ctypes.c_uint64), ("ffn_dim", ctypes.c_uint64), ("vocab_size", ctypes.c_uint64),
                ("rope_theta", ctypes.c_float), ("rms_norm_eps", ctypes.c_float), ("unpack_qk", ctypes.c_int32),
                ("ple_dim", ctypes.c_uint64), ("has_softcap", ctypes.c_int32), ("softcap", ctypes.c_float)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        L.orc_last_error.restype = ctypes.c_char_p
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_extract_scale_min_k4.argtypes = [ctypes.c_size_t, _f, _f, _f]
        L.orc_dequantize.argtypes = [ctypes.c_int, _f, ctypes.c_size_t, _f]
        L.orc_matmul.argtypes = [ctypes.c_int, _f, ctypes.c_size_t, ctypes.c_size_t, _f, ctypes.c_size_t,
                                 ctypes.c_size_t, _f, ctypes.c_int, ctypes.c_int]
        L.orc_rmsnorm.argtypes = [_f, _f, ctypes.c_size_t, ctypes.c_float, _f]
        L.orc_rmsnorm_no_scale.argtypes = [_f, ctypes.c_size_t, ctypes.c_float]
        L.orc_rope.argtypes = [_f, ctypes.c_size_t, ctypes.c_float, ctypes.c_uint32, ctypes.c_uint32,
                               ctypes.c_uint32, _f, ctypes.c_size_t]
        L.orc_softmax.argtypes = [_f, _f, ctypes.c_size_t]
        L.orc_swiglu.argtypes = [_f, _f, _f, ctypes.c_size_t]
        L.orc_gelu_tanh.argtypes = [ctypes.c_float]
        L.orc_gelu_tanh.restype = ctypes.c_float
        L.orc_residual_add.argtypes = [_f, _f, _f, ctypes.c_size_t]
        L.orc_argmax.argtypes = [_f, ctypes.c_size_t]
        L.orc_argmax.restype = ctypes.c_long
        L.orc_sample_temperature.argtypes = [_f, ctypes.c_size_t, ctypes.c_float, ctypes.c_float]
        L.orc_sample_temperature.restype = ctypes.c_long
        u32p = ctypes.POINTER(ctypes.c_uint32)
        ip = ctypes.POINTER(ctypes.c_int)
        L.orc_model_tokenizer_prompt.argtypes = [ctypes.c_void_p, ip, ip, u32p, u32p]
        L.orc_model_tokenizer_prompt.restype = ctypes.c_int
        L.orc_unpack_qk_row.argtypes = [_f, ctypes.c_size_t, ctypes.c_size_t]
        L.orc_attention_decode.argtypes = [_f, _f, _f, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
                                           ctypes.c_size_t, ctypes.c_long, ctypes.c_float, _f]
        L.orc_attention_prefill.argtypes = [_f, _f, _f, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
                                            ctypes.c_size_t, ctypes.c_long, ctypes.c_float, _f]
        L.orc_model_load.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)]
        L.orc_model_free.argtypes = [_f]
        L.orc_model_config.argtypes = [_f, ctypes.POINTER(Cfg)]
        L.orc_model_tensor.argtypes = [_f, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p),
                                       ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_int),
                                       ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]
        L.orc_model_layer_spec.argtypes = [_f, ctypes.c_size_t, ctypes.POINTER(ctypes.c_long),
                                           ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_uint64),
                                           ctypes.POINTER(ctypes.c_long), ctypes.POINTER(ctypes.c_uint64),
                                           ctypes.POINTER(ctypes.c_uint64)]
        L.orc_session_new.argtypes = [_f, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_void_p)]
        L.orc_session_free.argtypes = [_f]
        L.orc_session_reset.argtypes = [_f]
        L.orc_session_set_layer_limit.argtypes = [_f, ctypes.c_size_t]
        L.orc_session_set_layer_limit.restype = None
        L.orc_session_prefill.argtypes = [_f, _f, ctypes.c_size_t]
        L.orc_session_decode.argtypes = [_f, ctypes.c_uint32]
        L.orc_session_logits.argtypes = [_f, _f]
        L.orc_session_hidden.argtypes = [_f, _f, ctypes.c_size_t, ctypes.POINTER(ctypes.c_uint64)]
        L.orc_session_kv_len.argtypes = [_f, ctypes.c_size_t]
        L.orc_session_kv_len.restype = ctypes.c_uint64
        L.orc_session_kv.argtypes = [_f, ctypes.c_size_t, ctypes.c_int, _f, ctypes.c_size_t]
        _lib = L
    return _lib


def _check(rc: int):
    if rc != 0:
        raise OracleError(rc, lib().orc_last_error().decode())


def _p(a: np.ndarray):
    return a.ctypes.data


def f16_to_f32(bits: int) -> float:
    return lib().orc_f16_to_f32(bits)


def extract_scale_min_k4(j: int, scales: np.ndarray) -> tuple[int, int]:
    sc = np.zeros(1, np.uint8)
    m = np.zeros(1, np.uint8)
    s = np.ascontiguousarray(scales, dtype=np.uint8)
    lib().orc_extract_scale_min_k4(j, _p(s), _p(sc), _p(m))
    return int(sc[0]), int(m[0])


def dequantize(orc_type: int, blocks: np.ndarray, nblocks: int) -> np.ndarray:
    be = 32 if orc_type == T_Q8_0 else 256
    out = np.empty(nblocks * be, np.float32)
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    _check(lib().orc_dequantize(orc_type, _p(b), nblocks, _p(out)))
    return out


def matmul(orc_type: int, a: np.ndarray, w: np.ndarray, k: int, n: int, mode: int = PARITY, threads: int = 0):
    a = np.ascontiguousarray(a, dtype=np.float32)
    m = a.size // k
    w = np.ascontiguousarray(w).view(np.uint8)
    out = np.empty((m, n), np.float32)
    _check(lib().orc_matmul(orc_type, _p(a), m, k, _p(w), w.size, n, _p(out), mode,
                            threads or (os.cpu_count() or 1)))
    return out


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    _check(lib().orc_rmsnorm(_p(x), _p(w), x.size, eps, _p(out)))
    return out


def rmsnorm_no_scale(x, eps):
    x = np.array(x, np.float32)
    _check(lib().orc_rmsnorm_no_scale(_p(x), x.size, eps))
    return x


def rope(v, base, pos, head_dim, rotary_dim, ff=None):
    v = np.array(v, np.float32)
    if ff is None:
        _check(lib().orc_rope(_p(v), v.size, base, pos, head_dim, rotary_dim, None, 0))
    else:
        ff = np.ascontiguousarray(ff, np.float32)
        _check(lib().orc_rope(_p(v), v.size, base, pos, head_dim, rotary_dim, _p(ff), ff.size))
    return v


def softmax(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    _check(lib().orc_softmax(_p(x), _p(out), x.size))
    return out


def swiglu(g, u):
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty_like(g)
    _check(lib().orc_swiglu(_p(g), _p(u), _p(out), g.size))
    return out


def gelu_tanh(x: float) -> float:
    return lib().orc_gelu_tanh(x)


def residual_add(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.empty_like(a)
    _check(lib().orc_residual_add(_p(a), _p(b), _p(out), a.size))
    return out


def argmax(logits) -> int:
    """Returns index, or -1 (EmptyLogits) / -2 (InvalidLogits)."""
    l = np.ascontiguousarray(logits, np.float32)
    return int(lib().orc_argmax(_p(l), l.size))


def sample_temperature(logits, temperature: float, r: float) -> int:
    """sample_temperature (src/engine/sampling.rs:54-79) for the uniform draw r: the index, or -1
    (EmptyLogits) / -3 (InvalidTemperature)."""
    l = np.ascontiguousarray(logits, np.float32)
    return int(lib().orc_sample_temperature(_p(l), l.size, temperature, r))


def unpack_qk_row(row, n_groups, head_dim):
    r = np.array(row, np.float32)
    _check(lib().orc_unpack_qk_row(_p(r), n_groups, head_dim))
    return r


def attention_decode(q, k, v, n_heads, n_kv, head_dim, total, sliding_window, scale):
    """Head loop of decode_attention_layer (attention.rs:608-650) over a KVCache of `total`
    positions, k and v as [total][n_kv][head_dim]; sliding_window < 0 = none."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    out = np.empty(n_heads * head_dim, np.float32)
    _check(lib().orc_attention_decode(_p(q), _p(k), _p(v), n_heads, n_kv, head_dim, total, sliding_window, scale,
                                      _p(out)))
    return out


def attention_prefill(q, k, v, seq, n_heads, n_kv, head_dim, sliding_window, scale):
    """The head loop of prefill_attention_layer (attention.rs:364-415) over the layer's own k / v
    ([seq][n_kv][head_dim]); q [seq][n_heads][head_dim] after RoPE; sliding_window < 0 = none.
    Returns [seq][n_heads][head_dim]."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    out = np.empty(seq * n_heads * head_dim, np.float32)
    _check(lib().orc_attention_prefill(_p(q), _p(k), _p(v), seq, n_heads, n_kv, head_dim, sliding_window, scale,
                                       _p(out)))
    return out


class Model:
    def __init__(self, path: str):
        h = ctypes.c_void_p()
        _check(lib().orc_model_load(path.encode(), ctypes.byref(h)))
        self.h = h
        c = Cfg()
        _check(lib().orc_model_config(self.h, ctypes.byref(c)))
        self.cfg = c

    def layer_spec(self, li: int):
        w, t, r, b, hd, fd = (ctypes.c_long(), ctypes.c_float(), ctypes.c_uint64(), ctypes.c_long(),
                              ctypes.c_uint64(), ctypes.c_uint64())
        _check(lib().orc_model_layer_spec(self.h, li, ctypes.byref(w), ctypes.byref(t), ctypes.byref(r),
                                          ctypes.byref(b), ctypes.byref(hd), ctypes.byref(fd)))
        return dict(sliding_window=w.value, rope_theta=t.value, rotary_dim=r.value, kv_borrow=b.value,
                    head_dim=hd.value, ffn_dim=fd.value)

    def tokenizer_prompt(self):
        """TokenizerPromptConfig (src/model_config.rs:8-60): (add_bos, add_eos, bos_id, eos_id)."""
        ab, ae = ctypes.c_int(), ctypes.c_int()
        b, e = ctypes.c_uint32(), ctypes.c_uint32()
        _check(lib().orc_model_tokenizer_prompt(self.h, ctypes.byref(ab), ctypes.byref(ae), ctypes.byref(b),
                                                ctypes.byref(e)))
        return bool(ab.value), bool(ae.value), int(b.value), int(e.value)

    def tensor(self, name: str):
        """(dtype, raw bytes copy, ne0, ne1) of a loaded tensor."""
        d, nb, dt, n0, n1 = (ctypes.c_void_p(), ctypes.c_size_t(), ctypes.c_int(), ctypes.c_uint64(),
                             ctypes.c_uint64())
        _check(lib().orc_model_tensor(self.h, name.encode(), ctypes.byref(d), ctypes.byref(nb), ctypes.byref(dt),
                                      ctypes.byref(n0), ctypes.byref(n1)))
        raw = np.ctypeslib.as_array((ctypes.c_uint8 * nb.value).from_address(d.value)).copy()
        return dt.value, raw, n0.value, n1.value

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_model_free(self.h)
            self.h = None


class Session:
    def __init__(self, model: Model, mode: int = PARITY, threads: int = 0):
        h = ctypes.c_void_p()
        _check(lib().orc_session_new(model.h, mode, threads, ctypes.byref(h)))
        self.h = h
        self.model = model

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, np.uint32)
        _check(lib().orc_session_prefill(self.h, _p(ids), ids.size))

    def decode(self, tok: int):
        _check(lib().orc_session_decode(self.h, int(tok)))

    def logits(self) -> np.ndarray:
        out = np.empty(self.model.cfg.vocab_size, np.float32)
        _check(lib().orc_session_logits(self.h, _p(out)))
        return out

    def hidden(self) -> np.ndarray:
        c = self.model.cfg
        buf = np.empty(c.context_length * c.hidden_dim, np.float32)
        seq = ctypes.c_uint64()
        _check(lib().orc_session_hidden(self.h, _p(buf), buf.size, ctypes.byref(seq)))
        return buf[: seq.value * c.hidden_dim].reshape(seq.value, c.hidden_dim).copy()

    def kv_len(self, layer: int) -> int:
        return int(lib().orc_session_kv_len(self.h, layer))

    def kv(self, layer: int, which_v: bool) -> np.ndarray:
        c = self.model.cfg
        n = self.kv_len(layer)
        hd = self.model.layer_spec(layer)["head_dim"]
        out = np.empty((n, c.n_kv_heads, hd), np.float32)
        _check(lib().orc_session_kv(self.h, layer, 1 if which_v else 0, _p(out), n))
        return out

    def reset(self):
        _check(lib().orc_session_reset(self.h))

    def set_layer_limit(self, n: int):
        """Timing aid: run only the first n transformer blocks per step (0 = all)."""
        lib().orc_session_set_layer_limit(self.h, n)

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_session_free(self.h)
            self.h = None


def greedy_generate(sess: Session, prompt, n_decode: int, record_logits: bool = False):
    """prefill(prompt) then n_decode x (greedy_next_token, decode_token) — main.rs:97-116 /
    bench_metrics.rs:178-182 (no EOS stop). Returns (tokens, [logits per step])."""
    sess.prefill(prompt)
    toks, logs = [], []
    for _ in range(n_decode):
        lg = sess.logits()
        t = argmax(lg)
        if t < 0:
            raise OracleError(9, "invalid logits")
        if record_logits:
            logs.append(lg)
        toks.append(t)
        sess.decode(t)
    return toks, logs
