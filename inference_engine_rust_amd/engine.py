"""Python mirror of the reference engine API over the C ABI of libiek.so (include/iek.h).

Names follow the reference crate so a port of its callers reads the same:

* ``LoadedModel.load(path)``                       — src/loaded_model.rs:23-50
* ``InferenceSession(model)`` / ``.reset()``       — src/engine/session.rs:19-42
* ``.prefill(ids)`` / ``.decode_token(id)``        — session.rs:44-69
* ``.logits_last_token()``                         — session.rs:71-74 (runtime.rs:76-116)
* ``greedy_next_token(session)``                   — src/engine/generation.rs:10-16
* ``EngineError`` with the reference's variant names (src/error.rs:5-38)

The device engine is the only implementation behind these calls: importing this module fails
loudly when libiek.so is missing, and nothing here falls back to a CPU path.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libiek.so")

KINDS = {1: "Io", 2: "Utf8", 3: "Gguf", 4: "Tensor", 5: "MatMul", 6: "Model", 7: "Tokenizer", 8: "KvCache",
         9: "Sampling", 10: "Op", 11: "Device"}

F32, Q4K, Q6K, Q8_0, F16 = 0, 1, 2, 3, 4
GGML_TO_DTYPE = {0: F32, 12: Q4K, 14: Q6K, 8: Q8_0}
BLOCK = {Q4K: (256, 144), Q6K: (256, 210), Q8_0: (32, 34)}


class EngineError(RuntimeError):
    """Status != 0 from libiek; ``kind`` is the reference's EngineError variant name."""

    def __init__(self, code: int, msg: str):
        self.code = code
        self.kind = KINDS.get(code, "Unknown")
        super().__init__(f"{self.kind}: {msg}")


class Weight(ctypes.Structure):
    """iek_weight: native block bytes of a matmul weight, in host memory or HBM."""
    _fields_ = [("dtype", ctypes.c_int32), ("data", ctypes.c_void_p), ("bytes", ctypes.c_uint64),
                ("on_device", ctypes.c_int32)]


class TokenizerPrompt(ctypes.Structure):
    """TokenizerPromptConfig (src/model_config.rs:8-60)."""
    _fields_ = [("add_bos_token", ctypes.c_int32), ("add_eos_token", ctypes.c_int32),
                ("bos_token_id", ctypes.c_uint32), ("eos_token_id", ctypes.c_uint32)]


class ModelConfig(ctypes.Structure):
    _fields_ = [("family", ctypes.c_int32), ("context_length", ctypes.c_uint64), ("hidden_dim", ctypes.c_uint64),
                ("n_layers", ctypes.c_uint64), ("n_heads", ctypes.c_uint64), ("n_kv_heads", ctypes.c_uint64),
                ("head_dim", ctypes.c_uint64), ("ffn_dim", ctypes.c_uint64), ("vocab_size", ctypes.c_uint64),
                ("rope_theta", ctypes.c_float), ("rms_norm_eps", ctypes.c_float),
                ("unpack_llama_gguf_qk", ctypes.c_int32), ("embedding_length_per_layer", ctypes.c_uint64),
                ("has_final_logit_softcapping", ctypes.c_int32), ("final_logit_softcapping", ctypes.c_float)]


_P = ctypes.c_void_p
_SZ = ctypes.c_size_t
EXPORTS = {
    "iek_last_error": ([], ctypes.c_char_p),
    "iek_model_load": ([ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(_P)], ctypes.c_int),
    "iek_model_free": ([_P], None),
    "iek_model_load_timings": ([_P, _P], ctypes.c_int),
    "iek_model_config_get": ([_P, ctypes.POINTER(ModelConfig)], ctypes.c_int),
    "iek_model_tokenizer_prompt": ([_P, ctypes.POINTER(TokenizerPrompt)], ctypes.c_int),
    "iek_model_layer_spec": ([_P, ctypes.c_uint64, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_float),
                              ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_int64),
                              ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)], ctypes.c_int),
    "iek_model_tensor": ([_P, ctypes.c_char_p, ctypes.POINTER(_P), ctypes.POINTER(ctypes.c_int),
                          ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64),
                          ctypes.POINTER(ctypes.c_uint64)], ctypes.c_int),
    "iek_session_create": ([_P, ctypes.POINTER(_P)], ctypes.c_int),
    "iek_session_free": ([_P], None),
    "iek_session_reset": ([_P], ctypes.c_int),
    "iek_session_prefill": ([_P, _P, _SZ], ctypes.c_int),
    "iek_session_decode_token": ([_P, ctypes.c_uint32], ctypes.c_int),
    "iek_session_logits_last_token": ([_P, _P, _SZ], ctypes.c_int),
    "iek_greedy_next_token": ([_P, ctypes.POINTER(ctypes.c_uint32)], ctypes.c_int),
    "iek_session_sample_temperature": ([_P, ctypes.c_float, ctypes.c_float, ctypes.POINTER(ctypes.c_uint32)],
                                       ctypes.c_int),
    "iek_session_generate_greedy": ([_P, _SZ, _P], ctypes.c_int),
    "iek_session_kv_len": ([_P, ctypes.POINTER(ctypes.c_uint64)], ctypes.c_int),
    "iek_session_decode_path": ([_P, ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
    "iek_session_set_chain_spin": ([_P, ctypes.c_uint32], ctypes.c_int),
    "iek_session_f32_prefills": ([_P, ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
    "iek_session_bench_kernel": ([_P, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                  ctypes.POINTER(ctypes.c_double)], ctypes.c_int),
    "iek_session_hidden": ([_P, _P, _SZ, ctypes.POINTER(ctypes.c_uint64)], ctypes.c_int),
    "iek_session_kv": ([_P, ctypes.c_uint64, ctypes.c_int, _P, _SZ], ctypes.c_int),
    "iek_session_embed": ([_P, _P, _SZ], ctypes.c_int),
    "iek_session_set_hidden": ([_P, _P, _SZ], ctypes.c_int),
    "iek_session_prefill_layer_block": ([_P, ctypes.c_uint64], ctypes.c_int),
    "iek_session_decode_layer_block": ([_P, ctypes.c_uint64], ctypes.c_int),
    "iek_session_prefill_forward": ([_P], ctypes.c_int),
    "iek_session_decode_forward": ([_P], ctypes.c_int),
    "iek_matmul": ([_P, _SZ, _SZ, ctypes.c_void_p, _SZ, _P], ctypes.c_int),
    "iek_dequantize": ([ctypes.c_int, _P, _SZ, _P], ctypes.c_int),
    "iek_rmsnorm": ([_P, _P, _SZ, _SZ, ctypes.c_float, _P], ctypes.c_int),
    "iek_rope": ([_P, _SZ, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float, ctypes.c_uint32, _P, _SZ],
                 ctypes.c_int),
    "iek_softmax": ([_P, _P, _SZ], ctypes.c_int),
    "iek_swiglu": ([_P, _P, _P, _SZ], ctypes.c_int),
    "iek_gelu_tanh": ([_P, _P, _P, _SZ], ctypes.c_int),
    "iek_residual_add": ([_P, _P, _P, _SZ], ctypes.c_int),
    "iek_argmax": ([_P, _SZ, ctypes.POINTER(ctypes.c_uint32)], ctypes.c_int),
    "iek_sample_temperature": ([_P, _SZ, ctypes.c_float, ctypes.c_float, ctypes.POINTER(ctypes.c_uint32)],
                               ctypes.c_int),
    "iek_attention_decode": ([_P, _P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_float, _P], ctypes.c_int),
    "iek_dev_dequantize": ([ctypes.c_int, _P, _SZ, _P, _P], ctypes.c_int),
    "iek_dev_matmul": ([_P, _SZ, _SZ, ctypes.c_int, _P, _SZ, _SZ, _P, _P], ctypes.c_int),
    "iek_dev_rmsnorm": ([_P, _P, _SZ, _SZ, ctypes.c_float, _P, _P], ctypes.c_int),
    "iek_dev_rope": ([_P, _SZ, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float, ctypes.c_uint32, _P, _SZ, _P],
                     ctypes.c_int),
    "iek_dev_softmax": ([_P, _P, _SZ, _P], ctypes.c_int),
    "iek_dev_swiglu": ([_P, _P, _P, _SZ, _P], ctypes.c_int),
    "iek_dev_gelu_tanh": ([_P, _P, _P, _SZ, _P], ctypes.c_int),
    "iek_dev_residual_add": ([_P, _P, _P, _SZ, _P], ctypes.c_int),
    "iek_dev_argmax": ([_P, _SZ, ctypes.POINTER(ctypes.c_uint32), _P], ctypes.c_int),
    "iek_dev_sample_temperature": ([_P, _SZ, ctypes.c_float, ctypes.c_float, ctypes.POINTER(ctypes.c_uint32), _P],
                                   ctypes.c_int),
    "iek_dev_attention_decode": ([_P, _P, _P, ctypes.c_int, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_float, _P, _P],
                                 ctypes.c_int),
    "iek_dev_attention_decode_noalloc": ([_P, _P, _P, ctypes.c_int, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_float, _P,
                                          _P], ctypes.c_int),
    "iek_dev_attention_prefill": ([_P, _P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_float, _P, _P], ctypes.c_int),
    "iek_device_alloc": ([_SZ, ctypes.POINTER(_P)], ctypes.c_int),
    "iek_device_free": ([_P], ctypes.c_int),
    "iek_memcpy_h2d": ([_P, _P, _SZ], ctypes.c_int),
    "iek_memcpy_d2h": ([_P, _P, _SZ], ctypes.c_int),
    "iek_synchronize": ([], ctypes.c_int),
}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: the HIP engine has not been built "
                               "(run __graft_entry__.build()); there is no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in EXPORTS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _check(rc: int) -> None:
    if rc != 0:
        raise EngineError(rc, lib().iek_last_error().decode(errors="replace"))


def _np_ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


class LoadedModel:
    """GGUF model resident in HBM (LoadedModel, src/loaded_model.rs:14-87)."""

    def __init__(self, handle, path: str):
        self._h = handle
        self.path = path
        cfg = ModelConfig()
        _check(lib().iek_model_config_get(self._h, ctypes.byref(cfg)))
        self.config = cfg

    @classmethod
    def load(cls, path: str, device: int = 0) -> "LoadedModel":
        h = ctypes.c_void_p()
        _check(lib().iek_model_load(os.fsencode(path), device, ctypes.byref(h)))
        return cls(h, path)

    def tokenizer_prompt(self) -> TokenizerPrompt:
        """LoadedModel::tokenizer_prompt (src/loaded_model.rs:80-82)."""
        t = TokenizerPrompt()
        _check(lib().iek_model_tokenizer_prompt(self._h, ctypes.byref(t)))
        return t

    def layer_spec(self, layer: int) -> dict:
        w, t, r, b, hd, fd = (ctypes.c_int64(), ctypes.c_float(), ctypes.c_uint64(), ctypes.c_int64(),
                              ctypes.c_uint64(), ctypes.c_uint64())
        _check(lib().iek_model_layer_spec(self._h, layer, ctypes.byref(w), ctypes.byref(t), ctypes.byref(r),
                                          ctypes.byref(b), ctypes.byref(hd), ctypes.byref(fd)))
        return dict(sliding_window=w.value, rope_theta=t.value, rotary_dim=r.value, kv_borrow=b.value,
                    head_dim=hd.value, ffn_dim=fd.value)

    def load_timings(self) -> dict:
        """Load-stage wall times (ms) and HBM weight bytes of this model's iek_model_load."""
        buf = (ctypes.c_double * 5)()
        _check(lib().iek_model_load_timings(self._h, ctypes.cast(buf, ctypes.c_void_p)))
        names = ["gguf_metadata_ms", "config_and_resolve_ms", "tensor_load_ms", "weights_build_ms"]
        out = {n: float(buf[i]) for i, n in enumerate(names)}
        out["hbm_bytes"] = int(ctypes.cast(ctypes.addressof(buf) + 32, ctypes.POINTER(ctypes.c_uint64))[0])
        return out

    def tensor(self, name: str) -> dict:
        """Loaded tensor lookup (GGUFData::get_tensor): device pointer, dtype, ggml dims, bytes."""
        p, dt, n0, n1, nb = (ctypes.c_void_p(), ctypes.c_int(), ctypes.c_uint64(), ctypes.c_uint64(),
                             ctypes.c_uint64())
        _check(lib().iek_model_tensor(self._h, name.encode(), ctypes.byref(p), ctypes.byref(dt), ctypes.byref(n0),
                                      ctypes.byref(n1), ctypes.byref(nb)))
        return dict(ptr=p.value, dtype=dt.value, ne0=n0.value, ne1=n1.value, bytes=nb.value)

    def close(self):
        if self._h:
            lib().iek_model_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class InferenceSession:
    """Mutable generation state (InferenceSession, src/engine/session.rs:12-75)."""

    def __init__(self, model: LoadedModel):
        self.model = model
        h = ctypes.c_void_p()
        _check(lib().iek_session_create(model._h, ctypes.byref(h)))
        self._h = h

    def reset(self) -> None:
        _check(lib().iek_session_reset(self._h))

    def prefill(self, token_ids) -> None:
        ids = np.ascontiguousarray(np.asarray(token_ids, dtype=np.uint32))
        _check(lib().iek_session_prefill(self._h, _np_ptr(ids), ids.size))

    def decode_token(self, token_id: int) -> None:
        _check(lib().iek_session_decode_token(self._h, int(token_id)))

    def logits_last_token(self) -> np.ndarray:
        out = np.empty(self.model.config.vocab_size, np.float32)
        _check(lib().iek_session_logits_last_token(self._h, _np_ptr(out), out.size))
        return out

    def generate_greedy(self, n_steps: int) -> list[int]:
        out = np.zeros(max(n_steps, 1), np.uint32)
        _check(lib().iek_session_generate_greedy(self._h, n_steps, _np_ptr(out)))
        return [int(x) for x in out[:n_steps]]

    # forward level (src/engine/runtime.rs:14-61, src/layers/block.rs:12-89): the state stays in HBM
    def embed(self, token_ids) -> None:
        ids = np.ascontiguousarray(np.asarray(token_ids, dtype=np.uint32))
        _check(lib().iek_session_embed(self._h, _np_ptr(ids), ids.size))

    def set_hidden(self, rows: np.ndarray) -> None:
        h = np.ascontiguousarray(rows, np.float32).reshape(-1, self.model.config.hidden_dim)
        _check(lib().iek_session_set_hidden(self._h, _np_ptr(h), h.shape[0]))

    def prefill_layer_block(self, layer: int) -> None:
        _check(lib().iek_session_prefill_layer_block(self._h, layer))

    def decode_layer_block(self, layer: int) -> None:
        _check(lib().iek_session_decode_layer_block(self._h, layer))

    def prefill_forward(self) -> None:
        _check(lib().iek_session_prefill_forward(self._h))

    def decode_forward(self) -> None:
        _check(lib().iek_session_decode_forward(self._h))

    def bench_kernel(self, which: int, reps: int) -> tuple[float, float]:
        """(mean us per launch, algorithmic bytes or flops per launch) of the hot kernel `which`
        (0: middle-layer decode chain launch, 1: prefill gate/up GEMM, 2: prefill down GEMM,
        3: prefill Q/K/V GEMM); resets the session."""
        us, work = ctypes.c_double(), ctypes.c_double()
        _check(lib().iek_session_bench_kernel(self._h, which, reps, ctypes.byref(us), ctypes.byref(work)))
        return us.value, work.value

    def decode_path(self) -> int:
        """0: per-launch decode kernels; 1: the decode chain (persistent phase launches)."""
        v = ctypes.c_int(0)
        _check(lib().iek_session_decode_path(self._h, ctypes.byref(v)))
        return int(v.value)

    def set_chain_spin(self, spin: int) -> None:
        """Iteration limit of the decode chain's bounded waits (0: the default); a test aid for
        the chain's failure path."""
        _check(lib().iek_session_set_chain_spin(self._h, spin))

    def f32_prefills(self) -> int:
        """How many prefills of this session ran again on f32 activations (an activation beyond
        the fp16 pair's range)."""
        v = ctypes.c_int(0)
        _check(lib().iek_session_f32_prefills(self._h, ctypes.byref(v)))
        return int(v.value)

    def kv_len(self) -> int:
        v = ctypes.c_uint64()
        _check(lib().iek_session_kv_len(self._h, ctypes.byref(v)))
        return v.value

    def hidden(self) -> np.ndarray:
        c = self.model.config
        buf = np.empty(int(c.context_length) * int(c.hidden_dim), np.float32)
        rows = ctypes.c_uint64()
        _check(lib().iek_session_hidden(self._h, _np_ptr(buf), buf.size, ctypes.byref(rows)))
        return buf[: rows.value * c.hidden_dim].reshape(rows.value, c.hidden_dim).copy()

    def kv(self, layer: int, which_v: bool) -> np.ndarray:
        c = self.model.config
        n = self.kv_len()
        hd = self.model.layer_spec(layer)["head_dim"]
        out = np.empty((c.n_kv_heads, n, hd), np.float32)
        _check(lib().iek_session_kv(self._h, layer, 1 if which_v else 0, _np_ptr(out), out.size))
        return out

    def close(self):
        if self._h:
            lib().iek_session_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def sample_temperature_next_token(session: InferenceSession, temperature: float, r: float) -> int:
    """sample_temperature (src/engine/sampling.rs:54-79) over the session's last-token logits on
    the device; r is the uniform draw in [0, 1) the reference takes from its rng."""
    v = ctypes.c_uint32()
    _check(lib().iek_session_sample_temperature(session._h, temperature, r, ctypes.byref(v)))
    return v.value


def greedy_next_token(session: InferenceSession) -> int:
    """generation::greedy_next_token (src/engine/generation.rs:10-16), argmax on the device."""
    v = ctypes.c_uint32()
    _check(lib().iek_greedy_next_token(session._h, ctypes.byref(v)))
    return v.value


# ---- op level, host buffers (numpy arrays; synchronous) ----

def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32)


def host_matmul(a, w_blocks, dtype: int, n: int, on_device_ptr: int = 0) -> np.ndarray:
    """ops::matmul (src/ops/matmul.rs:18): a [m, k] f32 times W(k, n) given as native block bytes
    (a numpy uint8/float array), or an HBM address (`on_device_ptr`) with w_blocks its byte count."""
    a = _f32(a)
    m, k = a.shape
    out = np.empty((m, n), np.float32)
    if on_device_ptr:
        w = Weight(dtype, on_device_ptr, int(w_blocks), 1)
        _check(lib().iek_matmul(_np_ptr(a), m, k, ctypes.byref(w), n, _np_ptr(out)))
    else:
        wb = np.ascontiguousarray(w_blocks).view(np.uint8)
        w = Weight(dtype, wb.ctypes.data, wb.nbytes, 0)
        _check(lib().iek_matmul(_np_ptr(a), m, k, ctypes.byref(w), n, _np_ptr(out)))
    return out


def host_dequantize(dtype: int, blocks: np.ndarray, nblocks: int) -> np.ndarray:
    b = np.ascontiguousarray(blocks).view(np.uint8)
    out = np.empty(nblocks * (32 if dtype == 3 else 256), np.float32)
    _check(lib().iek_dequantize(dtype, _np_ptr(b), nblocks, _np_ptr(out)))
    return out


def host_rmsnorm(x, w, eps: float) -> np.ndarray:
    x = _f32(x)
    w = _f32(w)
    dim = w.size
    out = np.empty_like(x)
    _check(lib().iek_rmsnorm(_np_ptr(x), _np_ptr(w), x.size // dim, dim, eps, _np_ptr(out)))
    return out


def host_rope(v, n_heads: int, head_dim: int, rotary_dim: int, base: float, pos: int, freq_factors=None):
    v = _f32(v).copy()
    if freq_factors is None:
        _check(lib().iek_rope(_np_ptr(v), n_heads, head_dim, rotary_dim, base, pos, None, 0))
    else:
        ff = _f32(freq_factors)
        _check(lib().iek_rope(_np_ptr(v), n_heads, head_dim, rotary_dim, base, pos, _np_ptr(ff), ff.size))
    return v


def host_softmax(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    _check(lib().iek_softmax(_np_ptr(x), _np_ptr(out), x.size))
    return out


def host_swiglu(g, u) -> np.ndarray:
    g, u = _f32(g), _f32(u)
    out = np.empty_like(g)
    _check(lib().iek_swiglu(_np_ptr(g), _np_ptr(u), _np_ptr(out), g.size))
    return out


def host_gelu_tanh(g, u=None) -> np.ndarray:
    g = _f32(g)
    out = np.empty_like(g)
    if u is None:
        _check(lib().iek_gelu_tanh(_np_ptr(g), None, _np_ptr(out), g.size))
    else:
        u = _f32(u)
        _check(lib().iek_gelu_tanh(_np_ptr(g), _np_ptr(u), _np_ptr(out), g.size))
    return out


def host_residual_add(a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    _check(lib().iek_residual_add(_np_ptr(a), _np_ptr(b), _np_ptr(out), a.size))
    return out


def host_sample_temperature(logits, temperature: float, r: float) -> int:
    x = _f32(logits)
    v = ctypes.c_uint32()
    _check(lib().iek_sample_temperature(_np_ptr(x), x.size, temperature, r, ctypes.byref(v)))
    return v.value


def host_argmax(logits) -> int:
    x = _f32(logits)
    v = ctypes.c_uint32()
    _check(lib().iek_argmax(_np_ptr(x), x.size, ctypes.byref(v)))
    return v.value


def host_attention_decode(q, k_cache, v_cache, n_heads: int, n_kv_heads: int, head_dim: int, total_pos: int,
                          sliding_window: int, scale: float) -> np.ndarray:
    """The attention of decode_attention_layer over the reference KVCache layout
    [total_pos][n_kv_heads][head_dim] (src/layers/attention.rs:16-24, :608-650)."""
    q, k, v = _f32(q), _f32(k_cache), _f32(v_cache)
    out = np.empty(n_heads * head_dim, np.float32)
    _check(lib().iek_attention_decode(_np_ptr(q), _np_ptr(k), _np_ptr(v), n_heads, n_kv_heads, head_dim, total_pos,
                                      sliding_window, scale, _np_ptr(out)))
    return out


# ---- op level: device pointers (ints, e.g. torch.Tensor.data_ptr()) and an optional stream ----

def dequantize(dtype: int, blocks_ptr: int, nblocks: int, out_ptr: int, stream: int = 0) -> None:
    _check(lib().iek_dev_dequantize(dtype, blocks_ptr, nblocks, out_ptr, stream or None))


def matmul(a_ptr: int, m: int, k: int, dtype: int, w_ptr: int, w_bytes: int, n: int, out_ptr: int,
           stream: int = 0) -> None:
    _check(lib().iek_dev_matmul(a_ptr, m, k, dtype, w_ptr, w_bytes, n, out_ptr, stream or None))


def rmsnorm(in_ptr: int, w_ptr: int, rows: int, dim: int, eps: float, out_ptr: int, stream: int = 0) -> None:
    _check(lib().iek_dev_rmsnorm(in_ptr, w_ptr, rows, dim, eps, out_ptr, stream or None))


def rope(v_ptr: int, n_heads: int, head_dim: int, rotary_dim: int, base: float, pos: int, freq_factors=None,
         stream: int = 0) -> None:
    if freq_factors is None:
        _check(lib().iek_dev_rope(v_ptr, n_heads, head_dim, rotary_dim, base, pos, None, 0, stream or None))
    else:
        ff = np.ascontiguousarray(freq_factors, np.float32)
        _check(lib().iek_dev_rope(v_ptr, n_heads, head_dim, rotary_dim, base, pos, _np_ptr(ff), ff.size,
                                  stream or None))


def softmax(in_ptr: int, out_ptr: int, n: int, stream: int = 0) -> None:
    _check(lib().iek_dev_softmax(in_ptr, out_ptr, n, stream or None))


def swiglu(g_ptr: int, u_ptr: int, out_ptr: int, n: int, stream: int = 0) -> None:
    _check(lib().iek_dev_swiglu(g_ptr, u_ptr, out_ptr, n, stream or None))


def gelu_tanh(g_ptr: int, u_ptr, out_ptr: int, n: int, stream: int = 0) -> None:
    _check(lib().iek_dev_gelu_tanh(g_ptr, u_ptr or None, out_ptr, n, stream or None))


def residual_add(a_ptr: int, b_ptr: int, out_ptr: int, n: int, stream: int = 0) -> None:
    _check(lib().iek_dev_residual_add(a_ptr, b_ptr, out_ptr, n, stream or None))


def sample_temperature(logits_ptr: int, n: int, temperature: float, r: float, stream: int = 0) -> int:
    v = ctypes.c_uint32()
    _check(lib().iek_dev_sample_temperature(logits_ptr, n, temperature, r, ctypes.byref(v), stream or None))
    return v.value


def argmax(logits_ptr: int, n: int, stream: int = 0) -> int:
    v = ctypes.c_uint32()
    _check(lib().iek_dev_argmax(logits_ptr, n, ctypes.byref(v), stream or None))
    return v.value


def attention_decode(q_ptr: int, k_ptr: int, v_ptr: int, kv_dtype: int, n_heads: int, n_kv_heads: int,
                     head_dim: int, max_seq_len: int, total_pos: int, sliding_window: int, scale: float,
                     out_ptr: int, stream: int = 0) -> None:
    """Decode attention over a [n_kv_heads][max_seq_len][head_dim] cache (F16 = 4 or F32 = 0)."""
    _check(lib().iek_dev_attention_decode(q_ptr, k_ptr, v_ptr, kv_dtype, n_heads, n_kv_heads, head_dim, max_seq_len,
                                          total_pos, sliding_window, scale, out_ptr, stream or None))


def attention_decode_noalloc(q_ptr: int, k_ptr: int, v_ptr: int, kv_dtype: int, n_heads: int, n_kv_heads: int,
                             head_dim: int, max_seq_len: int, total_pos: int, sliding_window: int, scale: float,
                             out_ptr: int, stream: int = 0) -> None:
    """attention_decode without any device allocation (the library's per-device scratch)."""
    _check(lib().iek_dev_attention_decode_noalloc(q_ptr, k_ptr, v_ptr, kv_dtype, n_heads, n_kv_heads, head_dim,
                                                  max_seq_len, total_pos, sliding_window, scale, out_ptr,
                                                  stream or None))


def attention_prefill(q_ptr: int, k_ptr: int, v_ptr: int, seq: int, n_heads: int, n_kv_heads: int, head_dim: int,
                      sliding_window: int, scale: float, out_ptr: int, stream: int = 0) -> None:
    """Prefill attention over the layer's own q / k / v rows (device pointers, f32)."""
    _check(lib().iek_dev_attention_prefill(q_ptr, k_ptr, v_ptr, seq, n_heads, n_kv_heads, head_dim, sliding_window,
                                           scale, out_ptr, stream or None))


def synchronize() -> None:
    _check(lib().iek_synchronize())
