// extern "C" surface of libiek.so (declared in include/iek.h).
#include <cmath>
#include <cstring>
#include <memory>
#include <mutex>
#include <vector>

#include "../../include/iek.h"
#include "session.h"

namespace iek {

static thread_local std::string g_err;

void fail(int code, const std::string& msg) { throw Error{code, msg}; }

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) throw Error{ST_DEVICE, std::string(what) + ": " + hipGetErrorString(e)};
}

}  // namespace iek

using namespace iek;

struct iek_model {
  std::unique_ptr<Model> m;
};
struct iek_session {
  std::unique_ptr<Session> s;
};

#define IEK_API_TRY(...)                     \
  try {                                      \
    __VA_ARGS__;                             \
    return IEK_OK;                           \
  } catch (const Error& e) {                 \
    g_err = e.msg;                           \
    return (iek_status)e.code;               \
  } catch (const std::bad_alloc&) {          \
    g_err = "host allocation failed";        \
    return IEK_ERR_DEVICE;                   \
  } catch (const std::exception& e) {        \
    g_err = e.what();                        \
    return IEK_ERR_OP;                       \
  }

static hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

static void after_launch() { IEK_HIP(hipGetLastError()); }

static size_t block_elems(int dt) { return dt == DT_Q8_0 ? 32 : 256; }
static size_t block_bytes(int dt) { return dt == DT_Q4K ? 144 : dt == DT_Q6K ? 210 : 34; }

extern "C" {

const char* iek_last_error(void) { return g_err.c_str(); }

iek_status iek_model_load(const char* path, int device, iek_model** out) {
  IEK_API_TRY({
    if (!path || !out) fail(ST_OP, "null argument");
    auto* h = new iek_model();
    try {
      h->m.reset(load_model(path, device));
    } catch (...) {
      delete h;
      throw;
    }
    *out = h;
  })
}

void iek_model_free(iek_model* m) { delete m; }

iek_status iek_model_load_timings(const iek_model* m, iek_load_timings* o) {
  IEK_API_TRY({
    const LoadTimings& t = m->m->timings;
    o->gguf_metadata_ms = t.gguf_metadata_ms;
    o->config_and_resolve_ms = t.config_and_resolve_ms;
    o->tensor_load_ms = t.tensor_load_ms;
    o->weights_build_ms = t.weights_build_ms;
    o->hbm_bytes = (uint64_t)m->m->blob_bytes;
  })
}

iek_status iek_model_config_get(const iek_model* m, iek_model_config* o) {
  IEK_API_TRY({
    const Config& c = m->m->cfg;
    o->family = c.family;
    o->context_length = c.context_length;
    o->hidden_dim = c.hidden;
    o->n_layers = c.n_layers;
    o->n_heads = c.n_heads;
    o->n_kv_heads = c.n_kv_heads;
    o->head_dim = c.head_dim;
    o->ffn_dim = c.ffn_dim;
    o->vocab_size = c.vocab;
    o->rope_theta = c.rope_theta;
    o->rms_norm_eps = c.rms_eps;
    o->unpack_llama_gguf_qk = c.unpack_qk;
    o->embedding_length_per_layer = c.ple_dim;
    o->has_final_logit_softcapping = c.has_softcap;
    o->final_logit_softcapping = c.softcap;
  })
}

iek_status iek_model_tokenizer_prompt(const iek_model* m, iek_tokenizer_prompt* o) {
  IEK_API_TRY({
    const Config& c = m->m->cfg;
    o->add_bos_token = c.add_bos;
    o->add_eos_token = c.add_eos;
    o->bos_token_id = c.bos_id;
    o->eos_token_id = c.eos_id;
  })
}

iek_status iek_model_layer_spec(const iek_model* m, uint64_t li, int64_t* window, float* theta, uint64_t* rot,
                                int64_t* borrow, uint64_t* hd, uint64_t* fd) {
  IEK_API_TRY({
    const Config& c = m->m->cfg;
    if (li >= (uint64_t)c.n_layers) fail(ST_MODEL, "layer index out of range");
    const LayerSpec& L = c.layers[li];
    *window = L.window;
    *theta = L.rope_theta;
    *rot = L.rotary_dim;
    *borrow = L.kv_borrow;
    *hd = L.head_dim;
    *fd = L.ffn_dim;
  })
}

iek_status iek_model_tensor(const iek_model* m, const char* name, const void** dev_ptr, int* dtype, uint64_t* ne0,
                            uint64_t* ne1, uint64_t* bytes) {
  IEK_API_TRY({
    auto it = m->m->by_name.find(name ? name : "");
    if (it == m->m->by_name.end()) fail(ST_MODEL, std::string("tensor '") + (name ? name : "") + "' not loaded");
    const DevTensor& t = *it->second;
    *dev_ptr = t.dev;
    *dtype = t.dtype;
    *ne0 = t.dims.empty() ? 1 : t.dims[0];
    *ne1 = t.dims.size() > 1 ? t.dims[1] : 1;
    *bytes = t.bytes;
  })
}

iek_status iek_session_create(iek_model* m, iek_session** out) {
  IEK_API_TRY({
    auto* h = new iek_session();
    try {
      h->s.reset(new Session(m->m.get()));
    } catch (...) {
      delete h;
      throw;
    }
    *out = h;
  })
}

void iek_session_free(iek_session* s) { delete s; }

iek_status iek_session_reset(iek_session* s) { IEK_API_TRY(s->s->reset()) }

iek_status iek_session_prefill(iek_session* s, const uint32_t* ids, size_t n) {
  IEK_API_TRY({
    if (n > (size_t)INT32_MAX) fail(ST_MODEL, "prefill: token length exceeds context length");
    s->s->prefill(ids, (int)n);
  })
}

iek_status iek_session_decode_token(iek_session* s, uint32_t id) { IEK_API_TRY(s->s->decode_token(id)) }

iek_status iek_session_logits_last_token(iek_session* s, float* out, size_t n) {
  IEK_API_TRY(s->s->logits_last_token(out, (int)std::min<size_t>(n, INT32_MAX)))
}

iek_status iek_greedy_next_token(iek_session* s, uint32_t* out) { IEK_API_TRY(*out = s->s->greedy_next_token()) }

iek_status iek_session_sample_temperature(iek_session* s, float temperature, float r, uint32_t* out) {
  IEK_API_TRY(*out = s->s->sample_temperature(temperature, r))
}

iek_status iek_session_generate_greedy(iek_session* s, size_t n, uint32_t* out) {
  IEK_API_TRY({
    if (n > (size_t)INT32_MAX) fail(ST_KVCACHE, "KVCache is Full");
    s->s->generate_greedy((int)n, out);
  })
}

iek_status iek_session_kv_len(const iek_session* s, uint64_t* out) { IEK_API_TRY(*out = (uint64_t)s->s->kv_len()) }

iek_status iek_session_decode_path(const iek_session* s, int* out) { IEK_API_TRY(*out = s->s->decode_path()) }
iek_status iek_session_set_chain_spin(iek_session* s, uint32_t spin) { IEK_API_TRY(s->s->set_chain_spin(spin)) }
iek_status iek_session_f32_prefills(const iek_session* s, int* out) { IEK_API_TRY(*out = s->s->f32_prefills()) }

iek_status iek_session_bench_kernel(iek_session* s, int which, int reps, double* avg_us, double* work) {
  IEK_API_TRY(*avg_us = s->s->bench_kernel(which, reps, work))
}

iek_status iek_session_hidden(iek_session* s, float* out, size_t cap, uint64_t* rows) {
  IEK_API_TRY({
    int r = 0;
    s->s->copy_hidden(out, cap, &r);
    *rows = (uint64_t)r;
  })
}

iek_status iek_session_kv(iek_session* s, uint64_t layer, int which_v, float* out, size_t cap) {
  IEK_API_TRY(s->s->copy_kv((int)layer, which_v != 0, out, cap))
}

// ---- forward level ----
iek_status iek_session_embed(iek_session* s, const uint32_t* ids, size_t n) {
  IEK_API_TRY({
    if (n > (size_t)INT32_MAX) fail(ST_MODEL, "prefill: token length exceeds context length");
    s->s->embed(ids, (int)n);
  })
}

iek_status iek_session_set_hidden(iek_session* s, const float* hidden, size_t rows) {
  IEK_API_TRY({
    if (rows > (size_t)INT32_MAX) fail(ST_MODEL, "ForwardState: seq_len * hidden_dim overflow");
    s->s->set_hidden(hidden, (int)rows);
  })
}

iek_status iek_session_prefill_layer_block(iek_session* s, uint64_t layer) {
  IEK_API_TRY(s->s->prefill_layer((int)std::min<uint64_t>(layer, INT32_MAX)))
}

iek_status iek_session_decode_layer_block(iek_session* s, uint64_t layer) {
  IEK_API_TRY(s->s->decode_layer((int)std::min<uint64_t>(layer, INT32_MAX)))
}

iek_status iek_session_prefill_forward(iek_session* s) {
  IEK_API_TRY({
    const int L = s->s->n_layers();
    s->s->check_no_layer_forward();
    for (int li = 0; li < L; ++li) s->s->prefill_layer(li);
  })
}

iek_status iek_session_decode_forward(iek_session* s) {
  IEK_API_TRY({
    const int L = s->s->n_layers();
    s->s->check_no_layer_forward();
    for (int li = 0; li < L; ++li) s->s->decode_layer(li);
  })
}

// ---- op level, device pointers (asynchronous on the caller's stream) ----
static void matmul_dev(const float* a, size_t m, size_t k, int dt, const void* w, size_t w_bytes, size_t n, float* out,
                       hipStream_t st) {
  if (dt < DT_F32 || dt > DT_Q8_0) fail(ST_MATMUL, "unsupported matmul dtype");
  size_t need = dt == DT_F32 ? k * n * 4 : (k * n + block_elems(dt) - 1) / block_elems(dt) * block_bytes(dt);
  if (w_bytes < need) fail(ST_MATMUL, "weight buffer is smaller than expected");
  if (m == 0 || n == 0) return;
  if (m > (size_t)INT32_MAX || k > (size_t)INT32_MAX || n > (size_t)INT32_MAX) fail(ST_MATMUL, "dims too large");
  if (m == 1) {
    MvSegDesc sd{w, out, nullptr, (int)n};
    launch_matvec(dt, &sd, 1, a, (int)k, 0, st);
  } else {
    launch_gemm(dt, w, a, (int)m, (int)k, (int)n, out, nullptr, st);
  }
  after_launch();
}

// The (cos, sin) table of rope (src/ops/rope.rs:11-59) for `pos`, built on the host in f32 like
// the reference: theta starts at pos and is multiplied by base^(-2/rotary_dim) per pair.
static std::vector<float> rope_table(uint32_t head_dim, uint32_t rotary_dim, float base, uint32_t pos, const float* ff,
                                     size_t ff_len) {
  if (rotary_dim > head_dim)
    fail(ST_OP, "RoPE rotary_dim " + std::to_string(rotary_dim) + " > head_dim " + std::to_string(head_dim));
  uint32_t end = std::min(rotary_dim, head_dim);
  if (end % 2 != 0) fail(ST_OP, "RoPE rotary span must be even");
  uint32_t np = end / 2;
  if (ff && ff_len < np) fail(ST_OP, "RoPE freq_factors len < num_pairs");
  std::vector<float> cs((size_t)np * 2);
  float theta_scale = powf(base, -2.0f / (float)rotary_dim);
  float theta = (float)pos;
  for (uint32_t kk = 0; kk < np; ++kk) {
    float f = (ff && ff[kk] != 0.0f) ? ff[kk] : 1.0f;
    float angle = theta / f;
    cs[2 * kk] = cosf(angle);
    cs[2 * kk + 1] = sinf(angle);
    theta *= theta_scale;
  }
  return cs;
}

// argmax over device logits with a 32-byte device scratch (key, flag, flags, token); waits for
// the stream and returns the index, IEK_ERR_SAMPLING on a non-finite logit.
static uint32_t argmax_dev(const float* logits, size_t n, unsigned long long* scratch, hipStream_t st) {
  int* flag = reinterpret_cast<int*>(scratch + 1);
  int* flags = reinterpret_cast<int*>(scratch + 2);
  uint32_t* tok = reinterpret_cast<uint32_t*>(scratch + 3);
  uint32_t host = 0;
  int hflag = 0;
  launch_fill_u64(scratch, 0ull, 4, st);
  launch_argmax(logits, (int)n, scratch, flag, nullptr, st);
  launch_argmax_finish(scratch, flag, tok, nullptr, flags, nullptr, st);
  after_launch();
  IEK_HIP(hipMemcpyAsync(&host, tok, 4, hipMemcpyDeviceToHost, st));
  IEK_HIP(hipMemcpyAsync(&hflag, flags, 4, hipMemcpyDeviceToHost, st));
  IEK_HIP(hipStreamSynchronize(st));
  if (hflag) fail(ST_SAMPLING, "invalid logits for argmax (empty or non-finite)");
  return host;
}

// Checks of the decode attention op; returns the partial-buffer floats it needs.
static size_t attention_check(size_t n_heads, size_t n_kv, size_t hd, size_t max_len, size_t total) {
  if (n_kv == 0 || n_heads == 0 || n_heads % n_kv != 0 || n_heads / n_kv > 8)
    fail(ST_OP, "attention: GQA group must divide the heads and be at most 8");
  if (hd != 64 && hd != 128 && hd != 256 && hd != 512) fail(ST_OP, "attention: head_dim must be 64, 128, 256 or 512");
  if (total == 0) fail(ST_OP, "softmax: empty input");
  if (total > max_len)
    fail(ST_KVCACHE, "KV cache position " + std::to_string(total - 1) + " is out of bounds (max_seq_len is " +
                         std::to_string(max_len) + ")");
  if (max_len > (size_t)INT32_MAX / 2 || n_heads > 4096) fail(ST_OP, "attention: dims too large");
  return attn_decode_part_floats((int)n_heads, (int)hd, (int)max_len);
}

// counters (2 * n_kv ints) cleared and the position (total - 1) set by small kernels, so the
// sequence is safe under stream capture; the kernel leaves the counters zero again.
static void attention_launch(const float* q, const void* kc, const void* vc, bool kv_f32, size_t n_heads, size_t n_kv,
                             size_t hd, size_t max_len, size_t total, size_t window, float scale, float* out,
                             float* part, int* cnt, int* pos, hipStream_t st) {
  const int win = window >= total ? 0 : (int)window;  // a window covering every key is no window
  launch_fill_i32(cnt, 0, 2 * (int)n_kv, st);
  launch_set_int(pos, (int)(total - 1), st);
  launch_attn_decode(q, kc, vc, kv_f32, out, part, cnt, (int)n_heads, (int)n_kv, (int)hd, (int)max_len, pos, win,
                     scale, (int)max_len, st);
  after_launch();
}

iek_status iek_dev_dequantize(int dt, const void* blocks, size_t nblocks, float* out, void* stream) {
  IEK_API_TRY({
    if (dt != DT_Q4K && dt != DT_Q6K && dt != DT_Q8_0) fail(ST_TENSOR, "dequantize: not a block dtype");
    launch_dequant(dt, blocks, nblocks, out, as_stream(stream));
    after_launch();
  })
}

iek_status iek_dev_matmul(const float* a, size_t m, size_t k, int dt, const void* w, size_t w_bytes, size_t n,
                          float* out, void* stream) {
  IEK_API_TRY(matmul_dev(a, m, k, dt, w, w_bytes, n, out, as_stream(stream)))
}

iek_status iek_dev_rmsnorm(const float* in, const float* w, size_t rows, size_t dim, float eps, float* out,
                           void* stream) {
  IEK_API_TRY({
    launch_rmsnorm(in, w, (int)rows, (int)dim, eps, out, as_stream(stream));
    after_launch();
  })
}

iek_status iek_dev_rope(float* vec, size_t n_heads, uint32_t head_dim, uint32_t rotary_dim, float base, uint32_t pos,
                        const float* ff, size_t ff_len, void* stream) {
  IEK_API_TRY({
    std::vector<float> cs = rope_table(head_dim, rotary_dim, base, pos, ff, ff_len);
    float* d = nullptr;
    hipStream_t st = as_stream(stream);
    IEK_HIP(hipMalloc(&d, std::max<size_t>(cs.size() * 4, 4)));
    try {
      IEK_HIP(hipMemcpyAsync(d, cs.data(), cs.size() * 4, hipMemcpyHostToDevice, st));
      launch_rope_rows(vec, 1, (int)(n_heads * head_dim), (int)n_heads, (int)head_dim, 0, d, (int)(cs.size() / 2), st);
      after_launch();
      IEK_HIP(hipStreamSynchronize(st));
    } catch (...) {
      (void)hipFree(d);
      throw;
    }
    IEK_HIP(hipFree(d));
  })
}

iek_status iek_dev_softmax(const float* in, float* out, size_t n, void* stream) {
  IEK_API_TRY({
    if (n == 0) fail(ST_OP, "softmax: empty input");
    launch_softmax(in, out, (int)n, as_stream(stream));
    after_launch();
  })
}

iek_status iek_dev_swiglu(const float* g, const float* u, float* out, size_t n, void* stream) {
  IEK_API_TRY({
    launch_swiglu(g, u, out, n, as_stream(stream));
    after_launch();
  })
}

iek_status iek_dev_gelu_tanh(const float* g, const float* u, float* out, size_t n, void* stream) {
  IEK_API_TRY({
    launch_gelu_mul(g, u, out, n, as_stream(stream));
    after_launch();
  })
}

iek_status iek_dev_residual_add(const float* a, const float* b, float* out, size_t n, void* stream) {
  IEK_API_TRY({
    launch_residual_add(a, b, out, n, as_stream(stream));
    after_launch();
  })
}

iek_status iek_dev_argmax(const float* logits, size_t n, uint32_t* out_index, void* stream) {
  IEK_API_TRY({
    if (n == 0) fail(ST_SAMPLING, "logits slice is empty");
    unsigned long long* key = nullptr;
    IEK_HIP(hipMalloc(&key, 64));
    try {
      *out_index = argmax_dev(logits, n, key, as_stream(stream));
    } catch (...) {
      (void)hipFree(key);
      throw;
    }
    IEK_HIP(hipFree(key));
  })
}

// sample_temperature over device logits into a 4-byte device word, then to the host
static uint32_t sample_dev(const float* logits, size_t n, float temperature, float r, uint32_t* word, hipStream_t st) {
  if (n > (size_t)INT32_MAX) fail(ST_OP, "sample_temperature: too many logits");
  launch_sample_temperature(logits, (int)n, temperature, r, word, st);
  after_launch();
  uint32_t host = 0;
  IEK_HIP(hipMemcpyAsync(&host, word, 4, hipMemcpyDeviceToHost, st));
  IEK_HIP(hipStreamSynchronize(st));
  return host;
}

iek_status iek_dev_sample_temperature(const float* logits, size_t n, float temperature, float r, uint32_t* out_index,
                                      void* stream) {
  IEK_API_TRY({
    if (n == 0) fail(ST_SAMPLING, "logits slice is empty");
    uint32_t* word = nullptr;
    IEK_HIP(hipMalloc(&word, 64));
    try {
      *out_index = sample_dev(logits, n, temperature, r, word, as_stream(stream));
    } catch (...) {
      (void)hipFree(word);
      throw;
    }
    IEK_HIP(hipFree(word));
  })
}

iek_status iek_dev_attention_decode(const float* q, const void* k_cache, const void* v_cache, int kv_dtype,
                                    size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t max_seq_len,
                                    size_t total_pos, size_t sliding_window, float scale, float* out, void* stream) {
  IEK_API_TRY({
    if (kv_dtype != IEK_F16 && kv_dtype != IEK_F32) fail(ST_OP, "attention: KV cache dtype must be F16 or F32");
    const size_t pf = attention_check(n_heads, n_kv_heads, head_dim, max_seq_len, total_pos);
    hipStream_t st = as_stream(stream);
    char* scratch = nullptr;
    const size_t cnt_off = (pf * 4 + 255) / 256 * 256;
    IEK_HIP(hipMalloc(&scratch, cnt_off + (2 * n_kv_heads + 1) * 4));
    try {
      int* cnt = reinterpret_cast<int*>(scratch + cnt_off);
      attention_launch(q, k_cache, v_cache, kv_dtype == IEK_F32, n_heads, n_kv_heads, head_dim, max_seq_len, total_pos,
                       sliding_window, scale, out, reinterpret_cast<float*>(scratch), cnt, cnt + 2 * n_kv_heads, st);
      IEK_HIP(hipStreamSynchronize(st));  // the scratch is freed below
    } catch (...) {
      (void)hipFree(scratch);
      throw;
    }
    IEK_HIP(hipFree(scratch));
  })
}

iek_status iek_dev_attention_prefill(const float* q, const float* k, const float* v, size_t seq, size_t n_heads,
                                     size_t n_kv_heads, size_t head_dim, size_t sliding_window, float scale, float* out,
                                     void* stream) {
  IEK_API_TRY({
    if (n_kv_heads == 0 || n_heads == 0 || n_heads % n_kv_heads != 0)
      fail(ST_OP, "attention: the KV heads must divide the query heads");
    if (head_dim != 64 && head_dim != 128 && head_dim != 256 && head_dim != 512)
      fail(ST_OP, "attention: head_dim must be 64, 128, 256 or 512");
    if (seq == 0) fail(ST_OP, "softmax: empty input");
    if (seq > (1u << 20) || n_heads > 4096 || sliding_window > (size_t)INT32_MAX) fail(ST_OP, "attention: dims too large");
    const int M = (int)seq, nh = (int)n_heads, nkv = (int)n_kv_heads, hd = (int)head_dim;
    const int win = sliding_window >= seq ? 0 : (int)sliding_window;  // a window covering every key is no window
    hipStream_t st = as_stream(stream);
    // the K / V^T fp16 planes of the shared-K/V kernel (head_dim up to 256), then the range flag
    const size_t halves = hd <= 256 ? attn_prefill_scratch_halves(M, nkv, hd) : 0;
    const size_t ovf_off = (halves * 2 + 255) / 256 * 256;
    char* scratch = nullptr;
    IEK_HIP(hipMalloc(&scratch, ovf_off + 256));
    try {
      int* ovf = reinterpret_cast<int*>(scratch + ovf_off);
      launch_fill_i32(ovf, 0, 1, st);
      launch_attn_prefill(q, k, v, out, M, nh, nkv, hd, win, scale, st, halves ? scratch : nullptr, halves, false, ovf);
      int flagged = 0;
      IEK_HIP(hipMemcpyAsync(&flagged, ovf, sizeof(int), hipMemcpyDeviceToHost, st));
      IEK_HIP(hipStreamSynchronize(st));
      // an input beyond the fp16 pair's range: the f32 kernel, as the session's prefill reruns
      if (flagged) {
        launch_attn_prefill_f32(q, k, v, out, M, nh, nkv, hd, win, scale, st);
        IEK_HIP(hipStreamSynchronize(st));
      }
    } catch (...) {
      (void)hipFree(scratch);
      throw;
    }
    IEK_HIP(hipFree(scratch));
  })
}

iek_status iek_dev_attention_decode_noalloc(const float* q, const void* k_cache, const void* v_cache, int kv_dtype,
                                            size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t max_seq_len,
                                            size_t total_pos, size_t sliding_window, float scale, float* out,
                                            void* stream) {
  IEK_API_TRY({
    if (kv_dtype != IEK_F16 && kv_dtype != IEK_F32) fail(ST_OP, "attention: KV cache dtype must be F16 or F32");
    const size_t pf = attention_check(n_heads, n_kv_heads, head_dim, max_seq_len, total_pos);
    const size_t part_cap = NOALLOC_SCRATCH_BYTES - NOALLOC_COUNTER_BYTES;
    if (pf * 4 > part_cap)
      fail(ST_OP, "attention (no-alloc): partials of " + std::to_string(pf * 4) + " bytes exceed the " +
                      std::to_string(part_cap) + "-byte scratch (n_heads * ceil(max_seq_len / 64) * (head_dim + 2) "
                      "floats); use iek_dev_attention_decode");
    if ((2 * n_kv_heads + 1) * 4 > NOALLOC_COUNTER_BYTES) fail(ST_OP, "attention (no-alloc): too many KV heads");
    char* base = static_cast<char*>(noalloc_scratch(as_stream(stream)));
    int* cnt = reinterpret_cast<int*>(base);
    float* part = reinterpret_cast<float*>(base + NOALLOC_COUNTER_BYTES);
    attention_launch(q, k_cache, v_cache, kv_dtype == IEK_F32, n_heads, n_kv_heads, head_dim, max_seq_len, total_pos,
                     sliding_window, scale, out, part, cnt, cnt + 2 * n_kv_heads, as_stream(stream));
  })
}

}  // extern "C"

// ---- op level, host buffers (synchronous) ----
// Device staging of the host-buffer entries: per device one stream and one grow-only buffer, held
// until the process ends. A call holds the lock from its first upload to its final wait, so calls
// from several threads take turns.
namespace {
struct Stage {
  hipStream_t st = nullptr;
  char* buf = nullptr;
  size_t cap = 0;
};
std::mutex g_stage_mu;
Stage g_stage[64];

class HostCall {
 public:
  // `sizes`: the byte sizes of the call's device buffers, each placed at a 256-byte boundary
  explicit HostCall(std::initializer_list<size_t> sizes) : lock_(g_stage_mu) {
    int dev = 0;
    IEK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) fail(ST_DEVICE, "device index out of range");
    Stage& s = g_stage[dev];
    if (!s.st) IEK_HIP(hipStreamCreateWithFlags(&s.st, hipStreamNonBlocking));
    size_t total = 0;
    for (size_t b : sizes) {
      off_.push_back(total);
      total += (b + 255) / 256 * 256;
    }
    if (total > s.cap) {
      if (s.buf) IEK_HIP(hipFree(s.buf));
      s.buf = nullptr;
      s.cap = 0;
      IEK_HIP(hipMalloc(&s.buf, total));
      s.cap = total;
    }
    st = s.st;
    base_ = s.buf;
  }
  template <class T>
  T* ptr(int i) const {
    return reinterpret_cast<T*>(base_ + off_[i]);
  }
  template <class T>
  T* up(int i, const void* host, size_t bytes) const {
    if (bytes) IEK_HIP(hipMemcpyAsync(base_ + off_[i], host, bytes, hipMemcpyHostToDevice, st));
    return ptr<T>(i);
  }
  void down(void* host, const void* dev, size_t bytes) const {
    if (bytes) IEK_HIP(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, st));
  }
  void finish() const {
    after_launch();
    IEK_HIP(hipStreamSynchronize(st));
  }
  hipStream_t st = nullptr;

 private:
  std::unique_lock<std::mutex> lock_;
  std::vector<size_t> off_;
  char* base_ = nullptr;
};
// out = f(a, b) for the elementwise entries, staged through three buffers of n floats
template <class F>
void host_binary(const float* a, const float* b, float* out, size_t n, F launch) {
  if (n == 0) return;
  HostCall hc({n * 4, b ? n * 4 : 0, n * 4});
  const float* da = hc.up<float>(0, a, n * 4);
  const float* db = b ? hc.up<float>(1, b, n * 4) : nullptr;
  launch(da, db, hc.ptr<float>(2), hc.st);
  hc.down(out, hc.ptr<float>(2), n * 4);
  hc.finish();
}

}  // namespace

extern "C" {

iek_status iek_dequantize(int dt, const void* blocks, size_t nblocks, float* out) {
  IEK_API_TRY({
    if (dt != DT_Q4K && dt != DT_Q6K && dt != DT_Q8_0) fail(ST_TENSOR, "dequantize: not a block dtype");
    if (nblocks == 0) return IEK_OK;
    const size_t in_b = nblocks * block_bytes(dt), out_b = nblocks * block_elems(dt) * 4;
    HostCall hc({in_b, out_b});
    const void* d = hc.up<char>(0, blocks, in_b);
    launch_dequant(dt, d, nblocks, hc.ptr<float>(1), hc.st);
    hc.down(out, hc.ptr<float>(1), out_b);
    hc.finish();
  })
}

iek_status iek_matmul(const float* a, size_t m, size_t k, const iek_weight* w, size_t n, float* out) {
  IEK_API_TRY({
    if (!w) fail(ST_MATMUL, "null weight");
    const int dt = w->dtype;
    if (dt < DT_F32 || dt > DT_Q8_0) fail(ST_MATMUL, "unsupported matmul dtype");
    const size_t a_b = m * k * 4, o_b = m * n * 4, w_b = w->on_device ? 0 : w->bytes;
    HostCall hc({a_b, w_b, o_b});
    const float* da = hc.up<float>(0, a, a_b);
    const void* dw = w->on_device ? w->data : hc.up<char>(1, w->data, w_b);
    matmul_dev(da, m, k, dt, dw, w->bytes, n, hc.ptr<float>(2), hc.st);
    hc.down(out, hc.ptr<float>(2), o_b);
    hc.finish();
  })
}

iek_status iek_rmsnorm(const float* in, const float* w, size_t rows, size_t dim, float eps, float* out) {
  IEK_API_TRY({
    if (rows == 0 || dim == 0) return IEK_OK;
    const size_t n = rows * dim * 4;
    HostCall hc({n, dim * 4, n});
    const float* di = hc.up<float>(0, in, n);
    const float* dw = hc.up<float>(1, w, dim * 4);
    launch_rmsnorm(di, dw, (int)rows, (int)dim, eps, hc.ptr<float>(2), hc.st);
    hc.down(out, hc.ptr<float>(2), n);
    hc.finish();
  })
}

iek_status iek_rope(float* vec, size_t n_heads, uint32_t head_dim, uint32_t rotary_dim, float base, uint32_t pos,
                    const float* ff, size_t ff_len) {
  IEK_API_TRY({
    std::vector<float> cs = rope_table(head_dim, rotary_dim, base, pos, ff, ff_len);
    const size_t n = n_heads * head_dim * 4;
    if (n == 0 || cs.empty()) return IEK_OK;
    HostCall hc({n, cs.size() * 4});
    float* dv = hc.up<float>(0, vec, n);
    const float* dcs = hc.up<float>(1, cs.data(), cs.size() * 4);
    launch_rope_rows(dv, 1, (int)(n_heads * head_dim), (int)n_heads, (int)head_dim, 0, dcs, (int)(cs.size() / 2),
                     hc.st);
    hc.down(vec, dv, n);
    hc.finish();
  })
}

iek_status iek_softmax(const float* in, float* out, size_t n) {
  IEK_API_TRY({
    if (n == 0) fail(ST_OP, "softmax: empty input");
    HostCall hc({n * 4, n * 4});
    const float* di = hc.up<float>(0, in, n * 4);
    launch_softmax(di, hc.ptr<float>(1), (int)n, hc.st);
    hc.down(out, hc.ptr<float>(1), n * 4);
    hc.finish();
  })
}

iek_status iek_swiglu(const float* g, const float* u, float* out, size_t n) {
  IEK_API_TRY({
    if (!u) fail(ST_OP, "swiglu: null up");
    host_binary(g, u, out, n, [&](const float* a, const float* b, float* o, hipStream_t st) {
      launch_swiglu(a, b, o, n, st);
    });
  })
}

iek_status iek_gelu_tanh(const float* g, const float* u, float* out, size_t n) {
  IEK_API_TRY(host_binary(g, u, out, n, [&](const float* a, const float* b, float* o, hipStream_t st) {
    launch_gelu_mul(a, b, o, n, st);
  }))
}

iek_status iek_residual_add(const float* a, const float* b, float* out, size_t n) {
  IEK_API_TRY({
    if (!b) fail(ST_OP, "residual_add: null residual");
    host_binary(a, b, out, n, [&](const float* x, const float* r, float* o, hipStream_t st) {
      launch_residual_add(x, r, o, n, st);
    });
  })
}

iek_status iek_argmax(const float* logits, size_t n, uint32_t* out_index) {
  IEK_API_TRY({
    if (n == 0) fail(ST_SAMPLING, "logits slice is empty");
    HostCall hc({n * 4, 64});
    const float* dl = hc.up<float>(0, logits, n * 4);
    *out_index = argmax_dev(dl, n, hc.ptr<unsigned long long>(1), hc.st);
  })
}

iek_status iek_sample_temperature(const float* logits, size_t n, float temperature, float r, uint32_t* out_index) {
  IEK_API_TRY({
    if (n == 0) fail(ST_SAMPLING, "logits slice is empty");
    HostCall hc({n * 4, 64});
    const float* dl = hc.up<float>(0, logits, n * 4);
    *out_index = sample_dev(dl, n, temperature, r, hc.ptr<uint32_t>(1), hc.st);
  })
}

iek_status iek_attention_decode(const float* q, const float* k_cache, const float* v_cache, size_t n_heads,
                                size_t n_kv_heads, size_t head_dim, size_t total_pos, size_t sliding_window,
                                float scale, float* out) {
  IEK_API_TRY({
    const size_t pf = attention_check(n_heads, n_kv_heads, head_dim, total_pos, total_pos);
    // KVCache rows [pos][n_kv][head_dim] -> the kernel's [n_kv][pos][head_dim]
    const size_t kvn = total_pos * n_kv_heads * head_dim;
    std::vector<float> kt(kvn), vt(kvn);
    for (size_t p = 0; p < total_pos; ++p)
      for (size_t h = 0; h < n_kv_heads; ++h) {
        const size_t src = (p * n_kv_heads + h) * head_dim, dst = (h * total_pos + p) * head_dim;
        std::memcpy(&kt[dst], k_cache + src, head_dim * 4);
        std::memcpy(&vt[dst], v_cache + src, head_dim * 4);
      }
    const size_t qn = n_heads * head_dim * 4;
    HostCall hc({qn, kvn * 4, kvn * 4, qn, pf * 4, (2 * n_kv_heads + 1) * 4});
    const float* dq = hc.up<float>(0, q, qn);
    const float* dk = hc.up<float>(1, kt.data(), kvn * 4);
    const float* dv = hc.up<float>(2, vt.data(), kvn * 4);
    int* cnt = hc.ptr<int>(5);
    attention_launch(dq, dk, dv, true, n_heads, n_kv_heads, head_dim, total_pos, total_pos, sliding_window, scale,
                     hc.ptr<float>(3), hc.ptr<float>(4), cnt, cnt + 2 * n_kv_heads, hc.st);
    hc.down(out, hc.ptr<float>(3), qn);
    hc.finish();
  })
}

iek_status iek_device_alloc(size_t bytes, void** out) { IEK_API_TRY(IEK_HIP(hipMalloc(out, std::max<size_t>(bytes, 1)))) }
iek_status iek_device_free(void* p) { IEK_API_TRY(IEK_HIP(hipFree(p))) }
iek_status iek_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  IEK_API_TRY(IEK_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice)))
}
iek_status iek_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  IEK_API_TRY(IEK_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost)))
}
iek_status iek_synchronize(void) { IEK_API_TRY(IEK_HIP(hipDeviceSynchronize())) }

}  // extern "C"
