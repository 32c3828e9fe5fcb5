/*
 * iek.h — C ABI of the MI355X-native token loop (libiek.so).
 *
 * Drop-in for the GPU side of AntoineKhoury/inference_engine_rust's greedy prefill/decode path.
 * Every entry point names the reference interface it replaces (paths relative to the reference
 * repository root). Conventions:
 *   - Every function returns an iek_status (0 = OK); iek_last_error() gives a thread-local
 *     message. Status values are the reference's EngineError variants (src/error.rs:5-38).
 *   - Engine-, forward- and op-level calls (iek_session_*, iek_matmul, iek_rmsnorm, ...) take
 *     caller-owned HOST buffers and are synchronous on return, like the reference's functions.
 *   - The iek_dev_* variants of the ops take DEVICE pointers plus an optional hipStream_t (NULL =
 *     the null stream) and are asynchronous, like any HIP launch; iek_synchronize() waits.
 *   - Handles are not thread-safe; one session per host thread. The host-buffer op entries may be
 *     called from several threads (they take turns on one staging stream per device).
 */
#ifndef IEK_H
#define IEK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum iek_status {
  IEK_OK = 0,
  IEK_ERR_IO = 1,        /* EngineError::Io */
  IEK_ERR_UTF8 = 2,      /* EngineError::Utf8 */
  IEK_ERR_GGUF = 3,      /* EngineError::Gguf */
  IEK_ERR_TENSOR = 4,    /* EngineError::Tensor */
  IEK_ERR_MATMUL = 5,    /* EngineError::MatMul */
  IEK_ERR_MODEL = 6,     /* EngineError::Model */
  IEK_ERR_TOKENIZER = 7, /* EngineError::Tokenizer */
  IEK_ERR_KV_CACHE = 8,  /* EngineError::KvCache (src/layers/attention.rs:113-126) */
  IEK_ERR_SAMPLING = 9,  /* EngineError::Sampling (src/engine/sampling.rs:8-21) */
  IEK_ERR_OP = 10,       /* EngineError::Op */
  IEK_ERR_DEVICE = 11    /* HIP runtime failure (no reference counterpart: the reference is CPU-only) */
} iek_status;

/* Tensor dtypes: the reference's TensorType (src/core/tensor.rs:13-23); IEK_F16 is the device KV
 * cache's element type (iek_dev_attention_decode). */
typedef enum iek_dtype { IEK_F32 = 0, IEK_Q4K = 1, IEK_Q6K = 2, IEK_Q8_0 = 3, IEK_F16 = 4 } iek_dtype;

typedef struct iek_model iek_model;
typedef struct iek_session iek_session;

/* ModelConfig (src/model_config.rs:102-140), fields the token loop depends on. */
typedef struct iek_model_config {
  int32_t family; /* 0 MistralLlama, 1 Gemma4 (ModelFamily, model_config.rs:62-70) */
  uint64_t context_length, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim, ffn_dim, vocab_size;
  float rope_theta, rms_norm_eps;
  int32_t unpack_llama_gguf_qk;
  uint64_t embedding_length_per_layer;
  int32_t has_final_logit_softcapping;
  float final_logit_softcapping;
} iek_model_config;

/* TokenizerPromptConfig (src/model_config.rs:8-60): BOS/EOS insertion of
 * Tokenizer::encode_with_prompt_config (src/tokenizer/backend.rs:83-96) and the EOS stop of the
 * greedy CLI (src/main.rs:100-105). From tokenizer.ggml.{add_bos_token, add_eos_token,
 * bos_token_id, eos_token_id}; when the add_* keys are absent, tokenizer.ggml.model "llama" adds
 * BOS and not EOS, any other model neither; ids default to 1 and 2. */
typedef struct iek_tokenizer_prompt {
  int32_t add_bos_token, add_eos_token;
  uint32_t bos_token_id, eos_token_id;
} iek_tokenizer_prompt;

/* Last error message of the calling thread. */
const char* iek_last_error(void);

/* ---- model ---------------------------------------------------------------------------------
 * Replaces LoadedModel::load (src/loaded_model.rs:23-50): GGUF parse (file_loader.rs:26-65),
 * ModelConfig::from_gguf (model_config.rs:143-306), ModelWeightNames::resolve/load_all
 * (names.rs:52-276), then one upload of every tensor's native blocks to HBM on `device`. */
iek_status iek_model_load(const char* gguf_path, int device, iek_model** out);
void iek_model_free(iek_model* model);
/* Wall times of iek_model_load's stages, named after the cold-start regions of
 * src/bench_metrics.rs:199-296 (run_cold_start): GGUF header + tables (read_file), ModelConfig +
 * name resolution, tensor bytes from the memory-mapped file to HBM through pinned staging
 * (names.load_all), and the derived device tables (model.weights()). hbm_bytes: weight bytes. */
typedef struct iek_load_timings {
  double gguf_metadata_ms, config_and_resolve_ms, tensor_load_ms, weights_build_ms;
  uint64_t hbm_bytes;
} iek_load_timings;
iek_status iek_model_load_timings(const iek_model* model, iek_load_timings* out);
/* LoadedModel::config (src/loaded_model.rs:51-53). */
iek_status iek_model_config_get(const iek_model* model, iek_model_config* out);
/* LoadedModel::tokenizer_prompt (src/loaded_model.rs:80-82). */
iek_status iek_model_tokenizer_prompt(const iek_model* model, iek_tokenizer_prompt* out);
/* Per-layer LayerAttentionSpec + LayerDims (model_config.rs:72-100, :484-629): window -1 = none,
 * kv_borrow -1 = none. */
iek_status iek_model_layer_spec(const iek_model* model, uint64_t layer, int64_t* sliding_window, float* rope_theta,
                                uint64_t* rotary_dim, int64_t* kv_borrow, uint64_t* head_dim, uint64_t* ffn_dim);

/* GGUFData::get_tensor (src/model_loader/gguf_types.rs:343-346): the HBM address, dtype, ggml
 * dims ([ne0, ne1], ne1 = 1 for vectors) and byte length of a loaded tensor. IEK_ERR_MODEL when
 * the name was not loaded. */
iek_status iek_model_tensor(const iek_model* model, const char* name, const void** dev_ptr, int* dtype,
                            uint64_t* ne0, uint64_t* ne1, uint64_t* bytes);

/* ---- session (src/engine/session.rs:12-75) -------------------------------------------------- */
/* InferenceSession::new: KV caches of context_length positions per layer (the reference's f32 keys and values, in HBM). */
iek_status iek_session_create(iek_model* model, iek_session** out);
void iek_session_free(iek_session* s);
/* InferenceSession::reset (session.rs:40-42). */
iek_status iek_session_reset(iek_session* s);
/* InferenceSession::prefill (session.rs:44-56) = prefill_from_tokens_loaded + prefill_forward
 * (embed.rs:104-138, runtime.rs:14-32). */
iek_status iek_session_prefill(iek_session* s, const uint32_t* token_ids, size_t n);
/* InferenceSession::decode_token (session.rs:58-69) = embedding row + decode_forward
 * (embed.rs:53-98, runtime.rs:37-61). */
iek_status iek_session_decode_token(iek_session* s, uint32_t token_id);
/* InferenceSession::logits_last_token -> final_logits_last_token (runtime.rs:76-116).
 * `out` holds at least vocab_size floats. */
iek_status iek_session_logits_last_token(iek_session* s, float* out, size_t out_len);
/* greedy_next_token (src/engine/generation.rs:10-16) with argmax on the device
 * (sampling.rs:25-49: first maximal index; IEK_ERR_SAMPLING on any non-finite logit). */
iek_status iek_greedy_next_token(iek_session* s, uint32_t* out_token);
/* sample_temperature (src/engine/sampling.rs:54-79) on the session's last-token logits, on the
 * device: softmax(logits / temperature), then the first index whose cumulative probability
 * exceeds r, the caller's uniform draw in [0, 1) (the reference's rng.gen_range(0.0..1.0)).
 * IEK_ERR_SAMPLING for an empty vocabulary or a temperature that is not finite and positive;
 * IEK_ERR_OP for r outside [0, 1). NaN or +inf among the scaled logits gives the last index, as
 * the reference's NaN probabilities do. */
iek_status iek_session_sample_temperature(iek_session* s, float temperature, float r, uint32_t* out_token);
/* n iterations of { id = greedy_next_token; decode_token(id) } — the loop of src/main.rs:100-116
 * and EngineBench::run_decode_throughput (src/bench_metrics.rs:178-182) — replayed as one
 * captured decode-step graph; token ids never leave the device until the end. */
iek_status iek_session_generate_greedy(iek_session* s, size_t n_steps, uint32_t* out_ids);
/* KVCache::current_pos (attention.rs:49-52). */
iek_status iek_session_kv_len(const iek_session* s, uint64_t* out);
/* Which decode implementation the session runs (no reference counterpart; a diagnostic): 0 = one
 * launch per matvec and attention, 1 = the decode chain (Q/K/V, O, gate/up and down as phases of
 * persistent launches, two launches per layer) with row items and phase barriers (the default),
 * 2 = the same chain with 16-row tile items and per-superblock readiness (IEK_CHAIN=2 in the
 * environment at session creation selects it). All compute the same function. */
iek_status iek_session_decode_path(const iek_session* s, int* out);
/* No reference counterpart; a test aid for the decode chain's failure path. Sets the iteration
 * limit of the chain's bounded waits (each ~64 clocks; 0 restores the default, ~0.1-0.2 s). With a
 * small limit the next chain step gives its waits up: every kernel still exits normally, the call
 * fails with IEK_ERR_DEVICE, and the session state is undefined until iek_session_reset.
 * IEK_ERR_OP when the session does not decode through the chain. */
iek_status iek_session_set_chain_spin(iek_session* s, uint32_t spin);
/* No reference counterpart; a diagnostic. The prefill GEMMs and attention run on the matrix cores
 * with each f32 activation held as an fp16 (hi, lo) pair. When a value (or a per-32 sum of a GEMM
 * input) is beyond that pair's range (|x| > 65504), the prefill (session or layer level) runs again
 * on f32 activations, so that any finite f32 the reference takes is taken. *out: how many prefills
 * of this session have done so. */
iek_status iek_session_f32_prefills(const iek_session* s, int* out);
/* No reference counterpart; a measurement aid for the roofline figures. Times `reps` back-to-back
 * launches of one hot kernel on the session's stream between two HIP events, launch i on layer
 * i % n (so that consecutive launches stream different weights from HBM): which = 0, the decode
 * chain launch of layer pair (k-1, k) (layer k-1's O, gate/up and down phases, layer k's Q/K/V;
 * needs a state and the chain decode path); which = 1, the prefill gate/up GEMM over the last
 * prefill's rows (Mistral/Llama, a prefill state of >= 2 rows); which = 2, the prefill down
 * projection + residual; which = 3, the prefill Q/K/V GEMM (same conditions as 1). *avg_us: mean
 * duration per launch (a split-K GEMM's reduction pass included); *work: algorithmic bytes (0) or
 * flops (1-3) per launch, averaged over the layers. The session is reset afterwards. */
iek_status iek_session_bench_kernel(iek_session* s, int which, int reps, double* avg_us, double* work);
/* Hidden rows of the current ForwardState ([rows, hidden], src/engine/state.rs:7-175). */
iek_status iek_session_hidden(iek_session* s, float* out, size_t cap, uint64_t* rows);
/* KVCache::get_k_slice/get_v_slice for every stored position (attention.rs:77-110), widened to
 * f32 as [n_kv][kv_len][head_dim]. */
iek_status iek_session_kv(iek_session* s, uint64_t layer, int which_v, float* out, size_t cap);

/* ---- forward level (src/engine/runtime.rs, src/layers/block.rs) ---------------------------
 * The session's ForwardState ([rows, hidden], src/engine/state.rs:7-175) stays in HBM; read it
 * with iek_session_hidden and the logits of its last row with iek_session_logits_last_token
 * (final_logits_last_token, runtime.rs:76-116). A layer-level forward runs layers 0, 1, ...,
 * n_layers - 1 in order (IEK_ERR_MODEL for another layer); after the last one the KV length grows
 * by the state's rows. While one is part way, iek_session_decode_token, iek_greedy_next_token,
 * iek_session_generate_greedy and iek_session_logits_last_token fail with IEK_ERR_MODEL. */
/* prefill_from_tokens_loaded (src/engine/embed.rs:104-138): state = the ids' embedding rows (and,
 * for Gemma-4, their per-layer inputs, gemma4_ple.rs:27-109); n = 1 is the decode-token state of
 * prefill_state_for_single_token_loaded (embed.rs:53-98). */
iek_status iek_session_embed(iek_session* s, const uint32_t* token_ids, size_t n);
/* ForwardState::from_flat (state.rs:107-113): state = `rows` x hidden_dim floats, without
 * per-layer inputs (Gemma-4 layers with per-layer embeddings then fail with IEK_ERR_MODEL). */
iek_status iek_session_set_hidden(iek_session* s, const float* hidden, size_t rows);
/* prefill_layer_block (src/layers/block.rs:12-47) of layer `layer` over every row of the state:
 * prefill_attention_with_norm (attention.rs:696-824) + prefill_ffn_with_norm (ffn.rs:66-167) +
 * the Gemma-4 tails (ffn.rs:170-278); K/V rows go to the layer's cache at kv_len, kv_len + 1, ... */
iek_status iek_session_prefill_layer_block(iek_session* s, uint64_t layer);
/* decode_layer_block (block.rs:50-89) on a one-row state (IEK_ERR_MODEL otherwise), RoPE at kv_len. */
iek_status iek_session_decode_layer_block(iek_session* s, uint64_t layer);
/* prefill_forward (runtime.rs:14-32): every layer's prefill block over the state. */
iek_status iek_session_prefill_forward(iek_session* s);
/* decode_forward (runtime.rs:37-61): every layer's decode block; the state must have one row. */
iek_status iek_session_decode_forward(iek_session* s);

/* ---- op level, host buffers (synchronous) -------------------------------------------------- */
/* A matmul weight: native block bytes in ggml layout (element (k, n) at flat k + n*K), as the
 * reference's Tensor holds them (src/core/tensor.rs:8-23). on_device = 0: `data` is host memory,
 * uploaded per call; on_device = 1: `data` is an HBM address (e.g. from iek_model_tensor). */
typedef struct iek_weight {
  int32_t dtype; /* iek_dtype: F32, Q4K, Q6K or Q8_0 */
  const void* data;
  uint64_t bytes;
  int32_t on_device;
} iek_weight;
/* matmul (src/ops/matmul.rs:18-415): out[m, n] = sum_k a[m, k] * W(k, n). IEK_ERR_MATMUL for an
 * unsupported dtype or when w->bytes < div_ceil(K*N, block) * block_bytes. */
iek_status iek_matmul(const float* a, size_t m, size_t k, const iek_weight* w, size_t n, float* out);
/* dequantize_{q4k,q6k,q8_0}_block over n consecutive blocks (quant_k_handler.rs:21-135). */
iek_status iek_dequantize(int dtype, const void* blocks, size_t nblocks, float* out);
/* rmsnorm over `rows` rows of `dim` (src/ops/rmsnorm.rs:25-50). */
iek_status iek_rmsnorm(const float* in, const float* weight, size_t rows, size_t dim, float eps, float* out);
/* rope (src/ops/rope.rs:11-59) in place on n_heads contiguous heads of head_dim at position `pos`;
 * freq_factors may be NULL. IEK_ERR_OP: rotary_dim > head_dim, an odd rotary span, or fewer
 * freq_factors than pairs. */
iek_status iek_rope(float* vec, size_t n_heads, uint32_t head_dim, uint32_t rotary_dim, float base, uint32_t pos,
                    const float* freq_factors, size_t ff_len);
/* softmax (src/ops/softmax.rs:3-28); IEK_ERR_OP when n == 0. */
iek_status iek_softmax(const float* in, float* out, size_t n);
/* swiglu (src/ops/swiglu.rs:24-36): out = silu(gate) * up. */
iek_status iek_swiglu(const float* gate, const float* up, float* out, size_t n);
/* out = gelu_tanh(gate) * up, or gelu_tanh(gate) when up is NULL (src/ops/gelu.rs:5-18). */
iek_status iek_gelu_tanh(const float* gate, const float* up, float* out, size_t n);
/* residual_add (src/ops/residual_add.rs:3-12). */
iek_status iek_residual_add(const float* a, const float* b, float* out, size_t n);
/* argmax_index / sample_greedy (src/engine/sampling.rs:25-49): first maximal index;
 * IEK_ERR_SAMPLING when n == 0 or any logit is non-finite. */
iek_status iek_argmax(const float* logits, size_t n, uint32_t* out_index);
/* sample_temperature (src/engine/sampling.rs:54-79) over host logits; r is the caller's uniform
 * draw in [0, 1). Errors as iek_session_sample_temperature. */
iek_status iek_sample_temperature(const float* logits, size_t n, float temperature, float r, uint32_t* out_index);
/* The attention of decode_attention_layer (src/layers/attention.rs:608-650) for one new token,
 * its K/V already appended: for every query head h (KV head h / (n_heads / n_kv_heads)),
 * out[h] = softmax(scale * q[h] . K[j]) . V[j] over positions j in [j_min, total_pos), j_min =
 * total_pos - sliding_window when 0 < sliding_window < total_pos, else 0. k_cache and v_cache are
 * the reference KVCache's buffers (attention.rs:16-24): [total_pos][n_kv_heads][head_dim] f32.
 * Supported: head_dim 64, 128, 256 or 512 and n_heads / n_kv_heads <= 8 (IEK_ERR_OP otherwise);
 * total_pos == 0 is IEK_ERR_OP (the reference's empty softmax). */
iek_status iek_attention_decode(const float* q, const float* k_cache, const float* v_cache, size_t n_heads,
                                size_t n_kv_heads, size_t head_dim, size_t total_pos, size_t sliding_window,
                                float scale, float* out);

/* ---- op level, device pointers (asynchronous on `stream`) ---------------------------------
 * Same functions and errors as the host entries above; operands live in HBM. */
iek_status iek_dev_dequantize(int dtype, const void* blocks, size_t nblocks, float* out, void* stream);
/* w: w_bytes of native blocks in HBM; w_dtype an iek_dtype (F32, Q4K, Q6K, Q8_0). */
iek_status iek_dev_matmul(const float* a, size_t m, size_t k, int w_dtype, const void* w, size_t w_bytes, size_t n,
                          float* out, void* stream);
iek_status iek_dev_rmsnorm(const float* in, const float* weight, size_t rows, size_t dim, float eps, float* out,
                           void* stream);
/* freq_factors: HOST pointer or NULL. Waits for the stream before returning. */
iek_status iek_dev_rope(float* vec, size_t n_heads, uint32_t head_dim, uint32_t rotary_dim, float base, uint32_t pos,
                        const float* freq_factors, size_t ff_len, void* stream);
iek_status iek_dev_softmax(const float* in, float* out, size_t n, void* stream);
iek_status iek_dev_swiglu(const float* gate, const float* up, float* out, size_t n, void* stream);
iek_status iek_dev_gelu_tanh(const float* gate, const float* up, float* out, size_t n, void* stream);
iek_status iek_dev_residual_add(const float* a, const float* b, float* out, size_t n, void* stream);
/* Waits for the stream; *out_index is a host location. */
iek_status iek_dev_argmax(const float* logits, size_t n, uint32_t* out_index, void* stream);
/* Waits for the stream; *out_index is a host location. */
iek_status iek_dev_sample_temperature(const float* logits, size_t n, float temperature, float r, uint32_t* out_index,
                                      void* stream);
/* iek_attention_decode over the session's cache layout: k_cache / v_cache are
 * [n_kv_heads][max_seq_len][head_dim] of kv_dtype (IEK_F16 or IEK_F32) with positions
 * [0, total_pos) filled; total_pos <= max_seq_len (IEK_ERR_KV_CACHE otherwise). The partial
 * buffers are allocated per call; waits for the stream before returning. */
iek_status iek_dev_attention_decode(const float* q, const void* k_cache, const void* v_cache, int kv_dtype,
                                    size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t max_seq_len,
                                    size_t total_pos, size_t sliding_window, float scale, float* out, void* stream);
/* The head loop of prefill_attention_layer (src/layers/attention.rs:364-415) over the layer's own
 * K / V: q [seq][n_heads][head_dim] (RoPE applied), k and v [seq][n_kv_heads][head_dim], f32 in
 * HBM; for every position p and query head h (KV head h / (n_heads / n_kv_heads)),
 * out[p][h] = softmax(scale * q[p][h] . k[j]) . v[j] over j in [j_min, p], j_min = p -
 * (sliding_window - 1) when 0 < sliding_window, else 0. Runs the session's prefill kernels (fp16
 * (hi, lo) operand pairs on the matrix cores; an input beyond the pairs' range reruns on f32).
 * Supported: head_dim 64, 128, 256 or 512 (IEK_ERR_OP otherwise); seq == 0 is IEK_ERR_OP. Allocates
 * its scratch per call; waits for the stream before returning. */
iek_status iek_dev_attention_prefill(const float* q, const float* k, const float* v, size_t seq, size_t n_heads,
                                     size_t n_kv_heads, size_t head_dim, size_t sliding_window, float scale, float* out,
                                     void* stream);
/* No counterpart in the reference. For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): iek_dev_attention_decode
 * with the same arguments, results and errors, but its partials, arrival counters and position live
 * in a 16 MiB scratch array the library holds per device until the process ends; it calls no
 * allocator and does not wait for the stream. Limit: n_heads * ceil(max_seq_len / 64) *
 * (head_dim + 2) * 4 bytes <= 16 MiB - 4 KiB (e.g. 32 heads of 128 up to 32K keys), IEK_ERR_OP
 * beyond. Every call on a device shares that device's scratch: calls that overlap on one GPU (two
 * streams, or two threads) race and must be ordered by the caller. */
iek_status iek_dev_attention_decode_noalloc(const float* q, const void* k_cache, const void* v_cache, int kv_dtype,
                                            size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t max_seq_len,
                                            size_t total_pos, size_t sliding_window, float scale, float* out,
                                            void* stream);

/* ---- device memory helpers for FFI callers without a HIP binding ---------------------------- */
iek_status iek_device_alloc(size_t bytes, void** out);
iek_status iek_device_free(void* p);
iek_status iek_memcpy_h2d(void* dst, const void* src, size_t bytes);
iek_status iek_memcpy_d2h(void* dst, const void* src, size_t bytes);
iek_status iek_synchronize(void);

#ifdef __cplusplus
}
#endif
#endif /* IEK_H */
