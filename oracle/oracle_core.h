// TEST INFRASTRUCTURE ONLY — the CPU oracle.
//
// A C++ restatement of the reference's CPU token loop (AntoineKhoury/inference_engine_rust,
// a Rust crate that cannot be built in this environment: no rustc/cargo, crates not vendored).
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load liboracle.so,
// and only as the checker / the timed CPU baseline. The product (libiek.so) never links it.
//
// Arithmetic rules followed everywhere: f32 ops in the reference's order, no FMA contraction
// (-ffp-contract=off), f64 block dequant as the reference writes it, glibc libm for
// expf/cosf/sinf/powf/tanhf/sqrtf (Rust std calls the platform libm on Linux).
//
// What pins each part (tests/test_oracle_known_answers.py, tests/test_oracle_model.py):
//   f16_to_f32            exhaustive over all 65536 half patterns vs the IEEE closed form
//   extract_scale_min_k4  every 6-bit (scale, min) value round-trips through the packing
//   Q4_K / Q6_K / Q8_0    positional known answers (one nonzero field at a time), f64 single
//                         rounding, quantise->dequantise round trip against the synthetic writer
//   matmul                reference known answers (matmul.rs:453-497), float64 GEMM bound,
//                         sequential-order bit test, parity mode == baseline mode bit for bit
//   rmsnorm / rope / softmax / swiglu / gelu / argmax / unpack_qk
//                         the reference's own inline known answers (file:line in each test) plus
//                         closed forms (rope running product, swiglu two-branch sigmoid)
//   sample_temperature    the reference's tests (sampling.rs:101-115: deterministic for one draw,
//                         non-positive temperature rejected), two-logit closed form, uniform
//                         logits -> floor(r n), float64 brute force of the cumulative search
//   tokenizer prompt cfg  each metadata key alone and absent, both tokenizer.ggml.model defaults
//   attention + layer     layer 0 of the tiny model recomposed from the pinned ops around a
//                         brute-force float64 causal GQA attention; prefill N+1 == prefill N +
//                         decode; greedy loop == teacher-forced re-prefill
//   Gemma-4 parts         (tests/test_oracle_gemma.py) the whole tiny Gemma-4 model recomposed from
//                         the pinned ops around a brute-force float64 windowed attention (per-layer
//                         embeddings, q/k head norms, v norm, post-norms, GeGLU, KV borrowing,
//                         layer output scale in both encodings, tied head, soft cap); prefill N+1
//                         == prefill N + decode past the window; greedy == teacher forcing; config
//                         resolution of the Gemma-4 metadata; exact BF16 widening
#pragma once
#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace orc {

// Error codes mirror the EngineError variants (src/error.rs:5-38).
enum Err : int {
  OK = 0, E_IO = 1, E_UTF8 = 2, E_GGUF = 3, E_TENSOR = 4, E_MATMUL = 5, E_MODEL = 6,
  E_TOKENIZER = 7, E_KVCACHE = 8, E_SAMPLING = 9, E_OP = 10,
};

struct Error {
  int code;
  std::string msg;
};

// ---- GGUF values (src/model_loader/gguf_types.rs:4-36) ----
enum GType : int {
  G_U8 = 0, G_I8 = 1, G_U16 = 2, G_I16 = 3, G_U32 = 4, G_I32 = 5, G_F32 = 6, G_BOOL = 7,
  G_STR = 8, G_ARR = 9, G_U64 = 10, G_I64 = 11, G_F64 = 12,
};

struct GVal {
  int type = G_U8;
  uint64_t u = 0;
  int64_t i = 0;
  double f = 0;
  float f32 = 0;
  bool b = false;
  std::string s;
  std::vector<GVal> arr;
};

// TensorType (src/core/tensor.rs:13-23)
enum TType : int { T_F32 = 0, T_Q4K = 1, T_Q6K = 2, T_Q8_0 = 3 };

struct Tensor {
  int dtype = T_F32;
  std::vector<uint8_t> buf;
  std::vector<size_t> dims;
  const float* f32() const { return reinterpret_cast<const float*>(buf.data()); }
  size_t f32_len() const { return buf.size() / 4; }
};

struct TensorInfo {
  std::string name;
  std::vector<size_t> dims;
  uint32_t type_id = 0;
  uint64_t offset = 0;
};

struct GGUF {
  uint32_t version = 0;
  std::map<std::string, GVal> kv;
  std::vector<TensorInfo> infos;
  uint64_t data_offset = 0;
  std::map<std::string, Tensor> tensors;
  const GVal* meta(const std::string& k) const {
    auto it = kv.find(k);
    return it == kv.end() ? nullptr : &it->second;
  }
  const Tensor* get(const std::string& n) const {
    auto it = tensors.find(n);
    return it == tensors.end() ? nullptr : &it->second;
  }
};

enum Family : int { MISTRAL_LLAMA = 0, GEMMA4 = 1 };

struct LayerAttentionSpec {
  long sliding_window = -1;  // -1 = None (full causal)
  float rope_theta = 10000.f;
  size_t rope_rotary_dim = 0;
};

struct LayerDims {
  size_t q_dim, kv_dim, head_dim, ffn_dim;
};

struct ModelConfig {
  int family = MISTRAL_LLAMA;
  size_t context_length = 0, hidden_dim = 0, n_layers = 0, n_heads = 0, n_kv_heads = 0;
  size_t head_dim = 0, ffn_dim = 0;
  std::vector<LayerDims> layer_dims;
  float rope_theta = 10000.f, rms_norm_eps = 0.f;
  size_t vocab_size = 0;
  bool unpack_llama_gguf_qk = false;
  std::vector<LayerAttentionSpec> layer_attention;
  float token_embedding_scale = 1.f;
  size_t embedding_length_per_layer = 0;
  float ple_combine_scale = 0.f, ple_model_proj_scale = 0.f;
  std::vector<long> kv_borrow_from;  // -1 = None
  bool has_softcap = false;
  float softcap = 0.f;
  // TokenizerPromptConfig (src/model_config.rs:8-60)
  bool add_bos_token = false, add_eos_token = false;
  uint32_t bos_token_id = 1, eos_token_id = 2;
};

struct LayerW {
  const Tensor *attn_norm = nullptr, *ffn_norm = nullptr, *attn_post_norm = nullptr,
               *ffn_post_norm = nullptr, *attn_q_norm = nullptr, *attn_k_norm = nullptr;
  const Tensor *wq = nullptr, *wk = nullptr, *wv = nullptr, *wo = nullptr;
  const Tensor *w_gate = nullptr, *w_up = nullptr, *w_down = nullptr;
  const Tensor *ple_inp_gate = nullptr, *ple_proj = nullptr, *ple_post_norm = nullptr;
  const Tensor *rope_freqs = nullptr, *layer_output_scale = nullptr;
};

struct ModelW {
  const Tensor *token_embd = nullptr, *output_norm = nullptr, *lm_head = nullptr;
  std::vector<LayerW> layers;
  const Tensor *ple_token_embd = nullptr, *ple_model_proj = nullptr, *ple_proj_norm = nullptr;
};

struct Model {
  GGUF gguf;
  ModelConfig cfg;
  ModelW w;
  std::string emb_name;
};

struct KVCache {
  std::vector<float> k, v;
  size_t current_pos = 0, max_seq_len = 0, n_kv_heads = 0, head_dim = 0;
};

struct State {
  size_t seq_len = 0, hidden_dim = 0;
  std::vector<float> hidden;
  std::vector<float> ple_packed;
  size_t ple_n_layers = 0, ple_dim = 0;
};

// Execution mode. PARITY: vectorised/threaded but bit-identical per output element.
// BASELINE: the reference's own Rayon decomposition (rows of a matmul when M*N*K >= 65536,
// heads in attention), for timing.
// REASSOC: PARITY with every matmul dot product summed as two halves of K added at the end — a
// legitimate f32 reassociation, used to measure how much the model's logits move under rounding
// differences alone (the conditioning that bounds any reordered implementation).
// PAIR: REASSOC with every activation of a multi-row matmul (the prefill's) first rounded to its
// fp16 (hi, lo) pair, hi = fp16(x), lo = fp16(x - hi): how far the device prefill's operand
// rounding alone moves a model (test infrastructure only, like REASSOC).
// F16: REASSOC with each such activation rounded to a single fp16 (the one-operand encoding).
// I8X2_ROW, I8X2_B32, I8X3_ROW: REASSOC with each such activation replaced by its int8-plane
// encoding x = s*(i1 + i2/254 [+ i3/254^2]), |i| <= 127 round to nearest, s = max|x| / 127 over
// the row (ROW) or over each aligned block of 32 (B32): the operands of an int8 matrix-core GEMM
// whose int32 dots are exact, so the encoding is the only rounding it adds. Measurement modes
// for costing prefill formulations (test infrastructure only).
enum Mode : int { PARITY = 0, BASELINE = 1, REASSOC = 2, PAIR = 3, F16 = 4, I8X2_ROW = 5, I8X2_B32 = 6, I8X3_ROW = 7 };

struct Session {
  const Model* model = nullptr;
  std::vector<KVCache> kv;
  State state;
  int mode = PARITY;
  int threads = 1;
  size_t layer_limit = 0;  // 0 = all layers; >0 runs only the first N blocks (CPU-baseline sampling)
};

}  // namespace orc
