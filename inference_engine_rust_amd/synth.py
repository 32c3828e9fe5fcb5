"""Seeded synthetic GGUF models (ctypes over libiek_synth.so).

The reference has no model writer and no model file is reachable offline; every model the
engine, the oracle and the bench run is produced here, deterministically from a seed.
Presets follow the configurations the benchmark is quoted on:

* ``c0``  — tiny Mistral-architecture decoder (2 layers, d 512, 8/2 heads, FFN 1408).
* ``c2``  — Mistral-7B-v0.1 architecture (32 layers, d 4096, 32/8 heads, FFN 14336).
* ``c4``  — ``c2`` with an 8704-token context for long-context decode.
* ``c3``  — Gemma-4-E2B-style decoder (35 layers, d 1536, 8/1 heads, head dim 256 on sliding
  layers and 512 on global ones, FFN 6144, per-layer embeddings of 256, vocab 262144), Q8_0.
* ``g0``  — a tiny Gemma-4-architecture model with every Gemma feature switched on (sliding
  window smaller than the prompt, KV borrowing, partial rotary with freq factors, both
  layer-scale encodings) for parity tests.

Quant recipe ("Q4_K_M-style"): Q4_K for attention and FFN gate/up and the token embedding,
Q6_K for FFN down and the output head, f32 norms. Weights are N(0, 0.02); norm weights are
1 + N(0, 0.1) so that a kernel dropping the norm scale fails parity (a builder choice).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, replace

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
SYNTH_LIB = os.path.join(_HERE, "libiek_synth.so")

GGML_F32, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K, GGML_BF16 = 0, 8, 12, 14, 30


class _Spec(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("n_layers", ctypes.c_uint32),
        ("hidden", ctypes.c_uint32),
        ("n_heads", ctypes.c_uint32),
        ("n_kv_heads", ctypes.c_uint32),
        ("ffn", ctypes.c_uint32),
        ("vocab", ctypes.c_uint32),
        ("context_length", ctypes.c_uint32),
        ("rope_theta", ctypes.c_float),
        ("rms_eps", ctypes.c_float),
        ("weight_std", ctypes.c_float),
        ("norm_std", ctypes.c_float),
        ("t_attn", ctypes.c_uint32),
        ("t_ffn_gate_up", ctypes.c_uint32),
        ("t_ffn_down", ctypes.c_uint32),
        ("t_embd", ctypes.c_uint32),
        ("t_output", ctypes.c_uint32),
        ("tied_output", ctypes.c_uint32),
        ("mix", ctypes.c_uint32),
        ("t_norm", ctypes.c_uint32),
    ]


@dataclass(frozen=True)
class LlamaSpec:
    name: str
    n_layers: int
    hidden: int
    n_heads: int
    n_kv_heads: int
    ffn: int
    vocab: int
    context_length: int
    rope_theta: float = 10000.0
    rms_eps: float = 1e-5
    weight_std: float = 0.02
    norm_std: float = 0.1
    t_attn: int = GGML_Q4_K
    t_ffn_gate_up: int = GGML_Q4_K
    t_ffn_down: int = GGML_Q6_K
    t_embd: int = GGML_Q4_K
    t_output: int = GGML_Q6_K
    tied_output: bool = False
    # per-layer attn_v / ffn_down types: 0 uniform (t_attn / t_ffn_down), 1 llama.cpp's Q4_K_M
    # rule (Q6_K in the layers it gives more bits, Q4_K elsewhere), 2 Q6_K in odd layers only
    mix: int = 0
    # RMSNorm weights: 0 F32, 1 F16, 2 F32 holding f16-rounded values (the F32 twin of 1)
    t_norm: int = 0

    @property
    def head_dim(self) -> int:
        return self.hidden // self.n_heads


PRESETS = {
    "c0": LlamaSpec("synthetic-mistral-tiny", 2, 512, 8, 2, 1408, 32000, 64),
    "c2": LlamaSpec("synthetic-mistral-7b-v0.1", 32, 4096, 32, 8, 14336, 32000, 1024),
    "c4": LlamaSpec("synthetic-mistral-7b-v0.1-long", 32, 4096, 32, 8, 14336, 32000, 8704),
    # mid-size parity model: Mistral-7B widths, 2 layers, short context
    "c2_l2": LlamaSpec("synthetic-mistral-7b-2layer", 2, 4096, 32, 8, 14336, 32000, 640),
    # c0 with a 4096-token context: long-context decode attention (multi-slice chunks) at parity size
    "c0_long": LlamaSpec("synthetic-mistral-tiny-long", 2, 512, 8, 2, 1408, 32000, 4096),
    # C4's widths and context with 2 layers: the long-prompt prefill and decode kernels at parity size
    "c4_l2": LlamaSpec("synthetic-mistral-7b-2layer-long", 2, 4096, 32, 8, 14336, 32000, 8704),
}


class _GemmaSpec(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p)] + [
        (f, ctypes.c_uint32) for f in (
            "n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim_swa", "head_dim_global", "ffn", "vocab",
            "context_length", "ple_dim", "sliding_window", "global_every", "shared_kv_layers", "rot_swa",
            "rot_global")
    ] + [(f, ctypes.c_float) for f in ("theta_swa", "theta_global", "rms_eps", "weight_std", "norm_std", "softcap")] + [
        (f, ctypes.c_uint32) for f in ("t_weights", "t_embd", "t_ple_embd", "t_ple_proj", "rope_freqs",
                                       "q8_layer_scale")
    ]


@dataclass(frozen=True)
class GemmaSpec:
    """Gemma-4-architecture model. The reference does not pin Gemma-4-E2B's dimensions; these are
    the builder's choice (recorded with the benchmark). Layer i is global when
    i % global_every == global_every - 1, otherwise sliding-window."""
    name: str
    n_layers: int
    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim_swa: int
    head_dim_global: int
    ffn: int
    vocab: int
    context_length: int
    ple_dim: int
    sliding_window: int
    global_every: int
    shared_kv_layers: int
    rot_swa: int
    rot_global: int
    theta_swa: float = 10000.0
    theta_global: float = 1000000.0
    rms_eps: float = 1e-6
    weight_std: float = 0.02
    norm_std: float = 0.1
    softcap: float = 30.0
    t_weights: int = GGML_Q8_0
    t_embd: int = GGML_Q8_0
    t_ple_embd: int = GGML_Q8_0
    t_ple_proj: int = GGML_BF16
    rope_freqs: bool = True
    q8_layer_scale: bool = True

    def is_swa(self, layer: int) -> bool:
        return layer % self.global_every != self.global_every - 1

    def head_dim(self, layer: int) -> int:
        return self.head_dim_swa if self.is_swa(layer) else self.head_dim_global


PRESETS.update({
    "c3": GemmaSpec("synthetic-gemma-4-e2b", 35, 1536, 8, 1, 256, 512, 6144, 262144, 512, 256, 512, 5, 20,
                    256, 128, rope_freqs=False, q8_layer_scale=False),
    "g0": GemmaSpec("synthetic-gemma-4-tiny", 6, 256, 4, 1, 64, 128, 512, 8192, 96, 32, 16, 3, 2, 64, 32),
    # C3's head dims (256 sliding / 512 global) and GQA group of 8 at parity size
    "g1": GemmaSpec("synthetic-gemma-4-hd512", 6, 512, 8, 1, 256, 512, 1024, 8192, 640, 64, 128, 3, 2, 256, 128),
})


def preset(name: str, **overrides):
    return replace(PRESETS[name], **overrides)


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(SYNTH_LIB):
            raise RuntimeError(f"{SYNTH_LIB} is missing: run __graft_entry__.build() first")
        L = ctypes.CDLL(SYNTH_LIB)
        L.iek_synth_write_llama.argtypes = [ctypes.c_char_p, ctypes.POINTER(_Spec), ctypes.c_uint64, ctypes.c_int]
        L.iek_synth_write_llama.restype = ctypes.c_int
        L.iek_synth_write_gemma4.argtypes = [ctypes.c_char_p, ctypes.POINTER(_GemmaSpec), ctypes.c_uint64,
                                             ctypes.c_int]
        L.iek_synth_write_gemma4.restype = ctypes.c_int
        L.iek_synth_quantize.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        L.iek_synth_quantize.restype = ctypes.c_int
        L.iek_synth_normal.argtypes = [ctypes.c_uint64, ctypes.c_char_p, ctypes.c_size_t, ctypes.c_size_t,
                                       ctypes.c_float, ctypes.c_float, ctypes.c_void_p]
        L.iek_synth_normal.restype = None
        L.iek_synth_f32_to_f16.argtypes = [ctypes.c_float]
        L.iek_synth_f32_to_f16.restype = ctypes.c_uint16
        _lib = L
    return _lib


def write_llama(path: str, spec: LlamaSpec, seed: int = 0, threads: int | None = None) -> str:
    """Write a Mistral/Llama-family GGUF for ``spec`` to ``path`` and return the path."""
    s = _Spec(spec.name.encode(), spec.n_layers, spec.hidden, spec.n_heads, spec.n_kv_heads, spec.ffn,
              spec.vocab, spec.context_length, spec.rope_theta, spec.rms_eps, spec.weight_std,
              spec.norm_std, spec.t_attn, spec.t_ffn_gate_up, spec.t_ffn_down, spec.t_embd,
              spec.t_output, 1 if spec.tied_output else 0, spec.mix, spec.t_norm)
    if threads is None:
        threads = min(16, os.cpu_count() or 1)
    rc = lib().iek_synth_write_llama(path.encode(), ctypes.byref(s), seed, threads)
    if rc != 0:
        raise OSError(f"iek_synth_write_llama({path}) failed with code {rc}")
    return path


def write_gemma4(path: str, spec: GemmaSpec, seed: int = 0, threads: int | None = None) -> str:
    """Write a Gemma-4-architecture GGUF for ``spec`` to ``path`` and return the path."""
    vals = [spec.name.encode()] + [getattr(spec, f) for f, _ in _GemmaSpec._fields_[1:]]
    vals = [int(v) if isinstance(v, bool) else v for v in vals]
    s = _GemmaSpec(*vals)
    if threads is None:
        threads = min(16, os.cpu_count() or 1)
    rc = lib().iek_synth_write_gemma4(path.encode(), ctypes.byref(s), seed, threads)
    if rc != 0:
        raise OSError(f"iek_synth_write_gemma4({path}) failed with code {rc}")
    return path


def write_model(path: str, spec, seed: int = 0, threads: int | None = None) -> str:
    """Write ``spec`` (a LlamaSpec or GemmaSpec) as GGUF."""
    if isinstance(spec, GemmaSpec):
        return write_gemma4(path, spec, seed, threads)
    return write_llama(path, spec, seed, threads)


def normal(seed: int, name: str, n: int, mean: float = 0.0, std: float = 1.0, start: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().iek_synth_normal(seed, name.encode(), start, n, mean, std, out.ctypes.data)
    return out


BLOCK = {GGML_Q4_K: (256, 144), GGML_Q6_K: (256, 210), GGML_Q8_0: (32, 34)}


def quantize(ggml_type: int, x: np.ndarray) -> np.ndarray:
    """Quantise a float array whose length is a multiple of the block size; returns raw bytes."""
    be, bb = BLOCK[ggml_type]
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    if x.size % be:
        raise ValueError(f"length {x.size} is not a multiple of {be}")
    nb = x.size // be
    out = np.empty(nb * bb, dtype=np.uint8)
    if lib().iek_synth_quantize(ggml_type, x.ctypes.data, nb, out.ctypes.data) != 0:
        raise ValueError(f"unsupported type {ggml_type}")
    return out


def prompt_ids(seed: int, n: int, vocab: int = 32000) -> np.ndarray:
    """Uniform token ids in [3, vocab) from seed+1 (the benchmark's prompt recipe)."""
    rng = np.random.default_rng(seed + 1)
    return rng.integers(3, vocab, size=n, dtype=np.int64).astype(np.uint32)


# GGUF metadata value types (the container format: gguf_types.rs:4-36)
GGUF_U8, GGUF_I8, GGUF_U16, GGUF_I16, GGUF_U32, GGUF_I32, GGUF_F32, GGUF_BOOL, GGUF_STR = range(9)
GGUF_ARR, GGUF_U64, GGUF_I64, GGUF_F64 = 9, 10, 11, 12
_SCALAR = {GGUF_U8: "<B", GGUF_I8: "<b", GGUF_U16: "<H", GGUF_I16: "<h", GGUF_U32: "<I", GGUF_I32: "<i",
           GGUF_F32: "<f", GGUF_BOOL: "<B", GGUF_U64: "<Q", GGUF_I64: "<q", GGUF_F64: "<d"}


def _skip_value(buf: bytes, o: int, t: int) -> int:
    import struct

    if t in _SCALAR:
        return o + struct.calcsize(_SCALAR[t])
    if t == GGUF_STR:
        (n,) = struct.unpack_from("<Q", buf, o)
        return o + 8 + n
    if t == GGUF_ARR:
        et, n = struct.unpack_from("<IQ", buf, o)
        o += 12
        for _ in range(n):
            o = _skip_value(buf, o, et)
        return o
    raise ValueError(f"unknown GGUF value type {t}")


def _pack_kv(key: str, t: int, value) -> bytes:
    import struct

    k = key.encode()
    out = struct.pack("<Q", len(k)) + k + struct.pack("<I", t)
    if t in _SCALAR:
        return out + struct.pack(_SCALAR[t], int(value) if t == GGUF_BOOL else value)
    if t == GGUF_STR:
        v = value.encode()
        return out + struct.pack("<Q", len(v)) + v
    raise ValueError("with_metadata writes scalar and string values only")


def with_metadata(src: str, dst: str, entries) -> str:
    """Copy the GGUF `src` to `dst` with metadata entries [(key, gguf type, value)] added (an
    existing key of the same name is replaced). Tensor infos and data are copied unchanged; the
    data section is re-aligned to general.alignment (32 by default)."""
    import struct

    buf = open(src, "rb").read()
    magic, version, n_t, n_kv = struct.unpack_from("<IIQQ", buf, 0)
    o = 24
    kvs, align = [], 32
    drop = {k for k, _, _ in entries}
    for _ in range(n_kv):
        (kl,) = struct.unpack_from("<Q", buf, o)
        key = buf[o + 8:o + 8 + kl].decode()
        (t,) = struct.unpack_from("<I", buf, o + 8 + kl)
        end = _skip_value(buf, o + 12 + kl, t)
        if key == "general.alignment" and t == GGUF_U32:
            (align,) = struct.unpack_from("<I", buf, o + 12 + kl)
        if key not in drop:
            kvs.append(buf[o:end])
        o = end
    t0 = o
    for _ in range(n_t):
        (nl,) = struct.unpack_from("<Q", buf, o)
        o += 8 + nl
        (nd,) = struct.unpack_from("<I", buf, o)
        o += 4 + 8 * nd + 4 + 8
    infos = buf[t0:o]
    data_start = (o + align - 1) // align * align
    kvs += [_pack_kv(k, t, v) for k, t, v in entries]
    head = struct.pack("<IIQQ", magic, version, n_t, len(kvs)) + b"".join(kvs) + infos
    head += b"\0" * ((-len(head)) % align)
    with open(dst, "wb") as f:
        f.write(head)
        f.write(buf[data_start:])
    return dst


def tensor_offsets(path: str) -> dict:
    """{tensor name: (absolute byte offset of its data, ggml type, dims)} of a GGUF file (the
    tensor-info table of gguf_types.rs / tensor_loader.rs: name, n_dims, dims, type, offset
    relative to the aligned data section)."""
    import struct

    with open(path, "rb") as f:
        head = f.read(1 << 20)
        while True:  # the header of a large vocabulary can exceed the first read
            try:
                return _tensor_offsets(head)
            except struct.error:
                more = f.read(len(head))
                if not more:
                    raise
                head += more


def _tensor_offsets(buf: bytes) -> dict:
    import struct

    _, _, n_t, n_kv = struct.unpack_from("<IIQQ", buf, 0)
    o, align = 24, 32
    for _ in range(n_kv):
        (kl,) = struct.unpack_from("<Q", buf, o)
        key = buf[o + 8:o + 8 + kl].decode()
        (t,) = struct.unpack_from("<I", buf, o + 8 + kl)
        if key == "general.alignment" and t == GGUF_U32:
            (align,) = struct.unpack_from("<I", buf, o + 12 + kl)
        o = _skip_value(buf, o + 12 + kl, t)
    infos = []
    for _ in range(n_t):
        (nl,) = struct.unpack_from("<Q", buf, o)
        name = buf[o + 8:o + 8 + nl].decode()
        o += 8 + nl
        (nd,) = struct.unpack_from("<I", buf, o)
        dims = list(struct.unpack_from(f"<{nd}Q", buf, o + 4))
        o += 4 + 8 * nd
        gt, off = struct.unpack_from("<IQ", buf, o)
        o += 12
        infos.append((name, off, gt, dims))
    data = (o + align - 1) // align * align
    return {n: (data + off, gt, dims) for n, off, gt, dims in infos}


def patch_bytes(path: str, tensor: str, offset: int, data: bytes) -> None:
    """Overwrite `data` at byte `offset` of tensor `tensor`'s data in the GGUF file `path` (tests
    plant non-finite block scales this way)."""
    start, _, _ = tensor_offsets(path)[tensor]
    with open(path, "r+b") as f:
        f.seek(start + offset)
        f.write(data)
