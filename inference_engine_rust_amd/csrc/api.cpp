// extern "C" surface of libiek.so (declared in include/iek.h).
#include <cmath>
#include <cstring>
#include <memory>
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

iek_status iek_session_generate_greedy(iek_session* s, size_t n, uint32_t* out) {
  IEK_API_TRY({
    if (n > (size_t)INT32_MAX) fail(ST_KVCACHE, "KVCache is Full");
    s->s->generate_greedy((int)n, out);
  })
}

iek_status iek_session_kv_len(const iek_session* s, uint64_t* out) { IEK_API_TRY(*out = (uint64_t)s->s->kv_len()) }

iek_status iek_session_decode_path(const iek_session* s, int* out) { IEK_API_TRY(*out = s->s->decode_path()) }

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

// ---- op level ----
iek_status iek_dequantize(int dt, const void* blocks, size_t nblocks, float* out, void* stream) {
  IEK_API_TRY({
    if (dt != DT_Q4K && dt != DT_Q6K && dt != DT_Q8_0) fail(ST_TENSOR, "dequantize: not a block dtype");
    launch_dequant(dt, blocks, nblocks, out, as_stream(stream));
    after_launch();
  })
}

iek_status iek_matmul(const float* a, size_t m, size_t k, int dt, const void* w, size_t w_bytes, size_t n, float* out,
                      void* stream) {
  IEK_API_TRY({
    if (dt < DT_F32 || dt > DT_Q8_0) fail(ST_MATMUL, "unsupported matmul dtype");
    size_t need = dt == DT_F32 ? k * n * 4 : (k * n + block_elems(dt) - 1) / block_elems(dt) * block_bytes(dt);
    if (w_bytes < need) fail(ST_MATMUL, "weight buffer is smaller than expected");
    if (m == 0 || n == 0) return IEK_OK;
    if (m > (size_t)INT32_MAX || k > (size_t)INT32_MAX || n > (size_t)INT32_MAX) fail(ST_MATMUL, "dims too large");
    hipStream_t st = as_stream(stream);
    if (m == 1) {
      MvSegDesc sd{w, out, nullptr, (int)n};
      launch_matvec(dt, &sd, 1, a, (int)k, 0, st);
    } else {
      launch_gemm(dt, w, a, (int)m, (int)k, (int)n, out, nullptr, st);
    }
    after_launch();
  })
}

iek_status iek_rmsnorm(const float* in, const float* w, size_t rows, size_t dim, float eps, float* out, void* stream) {
  IEK_API_TRY({
    launch_rmsnorm(in, w, (int)rows, (int)dim, eps, out, as_stream(stream));
    after_launch();
  })
}

iek_status iek_rope(float* vec, size_t n_heads, uint32_t head_dim, uint32_t rotary_dim, float base, uint32_t pos,
                    const float* ff, size_t ff_len, void* stream) {
  IEK_API_TRY({
    if (rotary_dim > head_dim) fail(ST_OP, "RoPE rotary_dim " + std::to_string(rotary_dim) + " > head_dim " +
                                               std::to_string(head_dim));
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
    float* d = nullptr;
    hipStream_t st = as_stream(stream);
    IEK_HIP(hipMalloc(&d, std::max<size_t>(cs.size() * 4, 4)));
    try {
      IEK_HIP(hipMemcpyAsync(d, cs.data(), cs.size() * 4, hipMemcpyHostToDevice, st));
      launch_rope_rows(vec, 1, (int)(n_heads * head_dim), (int)n_heads, (int)head_dim, 0, d, (int)np, st);
      after_launch();
      IEK_HIP(hipStreamSynchronize(st));
    } catch (...) {
      (void)hipFree(d);
      throw;
    }
    IEK_HIP(hipFree(d));
  })
}

iek_status iek_softmax(const float* in, float* out, size_t n, void* stream) {
  IEK_API_TRY({
    if (n == 0) fail(ST_OP, "softmax: empty input");
    launch_softmax(in, out, (int)n, as_stream(stream));
    after_launch();
  })
}

iek_status iek_swiglu(const float* g, const float* u, float* out, size_t n, void* stream) {
  IEK_API_TRY({
    launch_swiglu(g, u, out, n, as_stream(stream));
    after_launch();
  })
}

iek_status iek_gelu_tanh(const float* g, const float* u, float* out, size_t n, void* stream) {
  IEK_API_TRY({
    launch_gelu_mul(g, u, out, n, as_stream(stream));
    after_launch();
  })
}

iek_status iek_residual_add(const float* a, const float* b, float* out, size_t n, void* stream) {
  IEK_API_TRY({
    launch_residual_add(a, b, out, n, as_stream(stream));
    after_launch();
  })
}

iek_status iek_argmax(const float* logits, size_t n, uint32_t* out_index, void* stream) {
  IEK_API_TRY({
    if (n == 0) fail(ST_SAMPLING, "logits slice is empty");
    hipStream_t st = as_stream(stream);
    unsigned long long* key = nullptr;
    IEK_HIP(hipMalloc(&key, 64));
    int* flag = reinterpret_cast<int*>(key + 1);
    int* flags = reinterpret_cast<int*>(key + 2);
    uint32_t* tok = reinterpret_cast<uint32_t*>(key + 3);
    uint32_t host[2] = {0, 0};
    int hflag = 0;
    try {
      launch_fill_u64(key, 0ull, 4, st);
      launch_argmax(logits, (int)n, key, flag, nullptr, st);
      launch_argmax_finish(key, flag, tok, nullptr, flags, nullptr, st);
      after_launch();
      IEK_HIP(hipMemcpyAsync(host, tok, 4, hipMemcpyDeviceToHost, st));
      IEK_HIP(hipMemcpyAsync(&hflag, flags, 4, hipMemcpyDeviceToHost, st));
      IEK_HIP(hipStreamSynchronize(st));
    } catch (...) {
      (void)hipFree(key);
      throw;
    }
    IEK_HIP(hipFree(key));
    if (hflag) fail(ST_SAMPLING, "invalid logits for argmax (empty or non-finite)");
    *out_index = host[0];
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
