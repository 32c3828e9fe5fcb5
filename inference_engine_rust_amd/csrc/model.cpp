// GGUF loading, ModelConfig resolution and the one-time upload of native quant blocks to HBM.
//
// Semantics follow the reference loader and config code so that the device engine sees exactly
// the model the reference would run:
//   src/model_loader/file_loader.rs:11-65   header, KV table, tensor table, aligned data offset
//   src/model_loader/reader.rs:94-157       value encodings (bool must be 0/1, nested arrays)
//   src/model_loader/tensor_loader.rs:27-88 raw block bytes, BF16 -> F32, div_ceil byte lengths
// One extension: F16 tensors (ggml type 1), which the reference rejects (tensor.rs:87-97), are
// widened to F32 at load like BF16; their values are exactly representable, so a model with F16
// norms or embeddings runs as the same model stored in F32.
//   src/model_config.rs:143-730             family detection, dims, attention specs, QK unpack
//   src/model_weights/names.rs:52-336       tensor-name fallbacks, tied LM head
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "model.h"

namespace iek {

namespace {

struct FileReader {
  FILE* f = nullptr;
  uint64_t pos = 0;
  ~FileReader() {
    if (f) fclose(f);
  }
  void read(void* dst, size_t n) {
    if (n && fread(dst, 1, n, f) != n) fail(ST_IO, "failed to fill whole buffer");
    pos += n;
  }
  template <class T>
  T get() {
    T v;
    read(&v, sizeof(T));
    return v;
  }
  std::string str() {
    uint64_t n = get<uint64_t>();
    if (n > (1ull << 32)) fail(ST_GGUF, "string length out of range");
    std::string s(n, '\0');
    read(&s[0], n);
    return s;
  }
};

uint32_t value_type(uint32_t code) {
  if (code > 12) fail(ST_GGUF, "unknown value type code " + std::to_string(code));
  return code;
}

MetaValue read_value(FileReader& r, uint32_t t) {
  MetaValue v;
  v.type = t;
  switch (t) {
    case 0: v.u = r.get<uint8_t>(); break;
    case 1: v.i = r.get<int8_t>(); break;
    case 2: v.u = r.get<uint16_t>(); break;
    case 3: v.i = r.get<int16_t>(); break;
    case 4: v.u = r.get<uint32_t>(); break;
    case 5: v.i = r.get<int32_t>(); break;
    case 6: v.f32 = r.get<float>(); v.f = v.f32; break;
    case 7: {
      uint8_t b = r.get<uint8_t>();
      if (b > 1) fail(ST_GGUF, "invalid GGUF bool byte (expected 0 or 1, got " + std::to_string(b) + ")");
      v.b = b == 1;
      break;
    }
    case 8: v.s = r.str(); break;
    case 9: {
      uint32_t et = value_type(r.get<uint32_t>());
      uint64_t n = r.get<uint64_t>();
      for (uint64_t i = 0; i < n; ++i) v.arr.push_back(read_value(r, et));
      break;
    }
    case 10: v.u = r.get<uint64_t>(); break;
    case 11: v.i = r.get<int64_t>(); break;
    case 12: v.f = r.get<double>(); break;
  }
  return v;
}

bool as_usize(const MetaValue& v, size_t* out) {
  switch (v.type) {
    case 0: case 2: case 4: case 10: *out = (size_t)v.u; return true;
    case 1: case 3: case 5: case 11:
      if (v.i < 0) return false;
      *out = (size_t)v.i;
      return true;
  }
  return false;
}

bool usize_opt(const GgufFile& g, const std::string& k, size_t* out) {
  const MetaValue* v = g.meta(k);
  if (!v) return false;
  if (v->type == 9) return !v->arr.empty() && as_usize(v->arr[0], out);
  return as_usize(*v, out);
}

size_t usize_alt(const GgufFile& g, std::initializer_list<const char*> keys) {
  size_t v;
  for (auto k : keys)
    if (usize_opt(g, k, &v)) return v;
  fail(ST_MODEL, std::string("missing integer metadata; tried keys [") + *keys.begin() + ", ...]");
}

bool f32_opt(const GgufFile& g, const std::string& k, float* out) {
  const MetaValue* v = g.meta(k);
  if (!v) return false;
  if (v->type == 6) { *out = v->f32; return true; }
  if (v->type == 12) { *out = (float)v->f; return true; }
  return false;
}

// get_bool (src/model_config.rs:704-709): a GGUF bool only.
bool bool_opt(const GgufFile& g, const std::string& k, bool* out) {
  const MetaValue* v = g.meta(k);
  if (!v || v->type != 7) return false;
  *out = v->b;
  return true;
}

// get_u32 (src/model_config.rs:711-723): any integer type whose value fits u32; no arrays.
bool u32_opt(const GgufFile& g, const std::string& k, uint32_t* out) {
  const MetaValue* v = g.meta(k);
  if (!v) return false;
  switch (v->type) {
    case 0: case 2: case 4: case 10:
      if (v->u > 0xFFFFFFFFull) return false;
      *out = (uint32_t)v->u;
      return true;
    case 1: case 3: case 5: case 11:
      if (v->i < 0 || v->i > 0xFFFFFFFFll) return false;
      *out = (uint32_t)v->i;
      return true;
  }
  return false;
}

std::string str_meta(const GgufFile& g, const std::string& k) {
  const MetaValue* v = g.meta(k);
  return (v && v->type == 8) ? v->s : std::string();
}

std::string lower(std::string s) {
  for (auto& c : s) c = (char)tolower((unsigned char)c);
  return s;
}

bool contains(const std::string& s, const char* t) { return s.find(t) != std::string::npos; }

bool env_bool(const char* name, bool* out) {
  const char* v = getenv(name);
  if (!v) return false;
  std::string s = lower(v);
  if (s == "1" || s == "true") { *out = true; return true; }
  if (s == "0" || s == "false") { *out = false; return true; }
  return false;
}

}  // namespace

GgufFile read_gguf(const std::string& path) {
  FileReader r;
  r.f = fopen(path.c_str(), "rb");
  if (!r.f) fail(ST_IO, "cannot open " + path);
  GgufFile g;
  char magic[4];
  r.read(magic, 4);  // read but not validated, as in file_loader.rs:31
  g.version = r.get<uint32_t>();
  uint64_t nt = r.get<uint64_t>(), nkv = r.get<uint64_t>();
  for (uint64_t i = 0; i < nkv; ++i) {
    std::string key = r.str();
    uint32_t t = value_type(r.get<uint32_t>());
    g.kv[key] = read_value(r, t);
  }
  for (uint64_t i = 0; i < nt; ++i) {
    TensorMeta t;
    t.name = r.str();
    uint32_t nd = r.get<uint32_t>();
    for (uint32_t d = 0; d < nd; ++d) t.dims.push_back((size_t)r.get<uint64_t>());
    t.ggml_type = r.get<uint32_t>();
    t.offset = r.get<uint64_t>();
    g.tensors.push_back(std::move(t));
  }
  uint64_t align = 32;
  const MetaValue* a = g.meta("general.alignment");
  if (a && a->type == 4 && a->u > 0 && (a->u & (a->u - 1)) == 0) align = a->u;
  g.data_offset = (r.pos + align - 1) & ~(align - 1);
  return g;
}

Config config_from_gguf(const GgufFile& g) {
  Config c;
  c.context_length = (int)usize_alt(g, {"llama.context_length", "gemma4.context_length"});
  c.hidden = (int)usize_alt(g, {"llama.embedding_length", "gemma4.embedding_length"});
  c.n_layers = (int)usize_alt(g, {"llama.block_count", "gemma4.block_count"});
  c.n_heads = (int)usize_alt(g, {"llama.attention.head_count", "gemma4.attention.head_count"});
  size_t v;
  c.n_kv_heads = (usize_opt(g, "llama.attention.head_count_kv", &v) || usize_opt(g, "gemma4.attention.head_count_kv", &v))
                     ? (int)v
                     : c.n_heads;
  int ffn_meta = (int)usize_alt(g, {"llama.feed_forward_length", "gemma4.feed_forward_length"});
  float f;
  c.rope_theta = (f32_opt(g, "llama.rope.theta", &f) || f32_opt(g, "gemma4.rope.freq_base", &f)) ? f : 10000.0f;
  if (!(f32_opt(g, "llama.attention.layer_norm_rms_epsilon", &f) ||
        f32_opt(g, "gemma4.attention.layer_norm_rms_epsilon", &f)))
    fail(ST_MODEL, "missing float metadata; tried keys [llama.attention.layer_norm_rms_epsilon, ...]");
  c.rms_eps = f;
  if (usize_opt(g, "llama.vocab_size", &v) || usize_opt(g, "gemma4.vocab_size", &v)) {
    c.vocab = (int)v;
  } else {
    const MetaValue* t = g.meta("tokenizer.ggml.tokens");
    if (!t) fail(ST_MODEL, "missing metadata key 'tokenizer.ggml.tokens'");
    if (t->type != 9) fail(ST_MODEL, "metadata key 'tokenizer.ggml.tokens' is not an array");
    c.vocab = (int)t->arr.size();
  }
  if (c.n_heads <= 0 || c.n_kv_heads <= 0) fail(ST_MODEL, "head counts must be positive");
  int hd;
  size_t kd;
  if (usize_opt(g, "gemma4.attention.key_length", &kd) && (int)kd * c.n_heads == c.hidden) hd = (int)kd;
  else if (c.hidden % c.n_heads != 0) fail(ST_MODEL, "hidden_dim not divisible by n_heads");
  else hd = c.hidden / c.n_heads;
  if (c.n_heads % c.n_kv_heads != 0) fail(ST_MODEL, "GQA requires n_heads divisible by n_kv_heads");

  // detect_model_family (model_config.rs:461-482)
  std::string arch = lower(str_meta(g, "general.architecture")), name = lower(str_meta(g, "general.name"));
  c.family = (contains(arch, "gemma4") || contains(arch, "gemma-4") || contains(name, "gemma-4") ||
              contains(name, "gemma4") || g.meta("gemma4.attention.sliding_window_pattern"))
                 ? FAM_GEMMA4
                 : FAM_MISTRAL_LLAMA;
  bool b;
  if (env_bool("INFERENCE_ENGINE_GGUF_QK_UNPACK", &b)) {
    c.unpack_qk = b;
  } else {
    const char* no = getenv("INFERENCE_ENGINE_GGUF_NO_QK_UNPACK");
    std::string ns = no ? lower(no) : "";
    if (no && (ns == "1" || ns == "true")) c.unpack_qk = false;
    else c.unpack_qk = c.family == FAM_GEMMA4 ? false : !(contains(name, "mistral") || contains(name, "gemma"));
  }
  // infer_layer_dims (model_config.rs:374-444)
  c.layers.resize(c.n_layers);
  if (c.n_layers <= 0) fail(ST_MODEL, "layer_dims empty");
  for (int i = 0; i < c.n_layers; ++i) {
    LayerSpec& L = c.layers[i];
    if (c.family == FAM_MISTRAL_LLAMA) {
      L.q_dim = c.n_heads * hd;
      L.kv_dim = c.n_kv_heads * hd;
      L.head_dim = hd;
      L.ffn_dim = ffn_meta;
    } else {
      std::string p = "blk." + std::to_string(i) + ".";
      auto kn = [&](const std::string& n, size_t* k, size_t* nn) {
        const TensorMeta* t = g.tensor(n);
        if (!t) fail(ST_MODEL, "missing tensor metadata '" + n + "'");
        if (t->dims.size() < 2) fail(ST_MODEL, "tensor '" + n + "': expected 2 dimensions");
        *k = t->dims[0];
        *nn = t->dims[1];
      };
      size_t kq, qd, kk, kvd, kg, fd;
      kn(p + "attn_q.weight", &kq, &qd);
      kn(p + "attn_k.weight", &kk, &kvd);
      kn(p + "ffn_gate.weight", &kg, &fd);
      if ((int)kq != c.hidden || (int)kk != c.hidden || (int)kg != c.hidden)
        fail(ST_MODEL, "layer " + std::to_string(i) + ": unexpected attn/FFN input dim");
      if (qd % c.n_heads || kvd % c.n_kv_heads) fail(ST_MODEL, "layer " + std::to_string(i) + ": head split");
      if (qd / c.n_heads != kvd / c.n_kv_heads) fail(ST_MODEL, "Q head dim != KV head dim");
      L.q_dim = (int)qd;
      L.kv_dim = (int)kvd;
      L.head_dim = (int)(qd / c.n_heads);
      L.ffn_dim = (int)fd;
    }
  }
  c.head_dim = hd;
  c.ffn_dim = ffn_meta;
  if (c.family == FAM_GEMMA4) {
    c.head_dim = 0;
    c.ffn_dim = 0;
    for (auto& L : c.layers) {
      c.head_dim = std::max(c.head_dim, L.head_dim);
      c.ffn_dim = std::max(c.ffn_dim, L.ffn_dim);
    }
  }
  int hd0 = c.layers[0].head_dim;
  if (hd0 <= 0 || hd0 % 2) fail(ST_MODEL, "layer attention: head_dim must be positive and even");
  if (c.family == FAM_MISTRAL_LLAMA) {
    // Dense family: full causal attention on every layer (model_config.rs:505-507).
    for (auto& L : c.layers) {
      L.window = -1;
      L.rope_theta = c.rope_theta;
      L.rotary_dim = hd0;
    }
  } else {
    const MetaValue* pat = g.meta("gemma4.attention.sliding_window_pattern");
    if (!pat) fail(ST_MODEL, "Gemma 4 GGUF missing gemma4.attention.sliding_window_pattern");
    if (pat->type != 9) fail(ST_MODEL, "gemma4.attention.sliding_window_pattern has wrong type");
    if ((int)pat->arr.size() != c.n_layers) fail(ST_MODEL, "sliding_window_pattern length != n_layers");
    size_t window;
    if (!usize_opt(g, "gemma4.attention.sliding_window", &window) && !usize_opt(g, "llama.attention.sliding_window", &window))
      fail(ST_MODEL, "Gemma 4 GGUF missing sliding window size");
    if (window == 0) fail(ST_MODEL, "Gemma 4 sliding window size must be > 0");
    size_t rl, rg;
    if (!usize_opt(g, "gemma4.rope.dimension_count_swa", &rl) && !usize_opt(g, "gemma4.attention.rotary_dim_local", &rl) &&
        !usize_opt(g, "llama.rope.dimension_count", &rl))
      rl = (size_t)hd0;
    if (!usize_opt(g, "gemma4.rope.dimension_count", &rg) && !usize_opt(g, "gemma4.attention.rotary_dim_global", &rg))
      rg = rl;
    float tl, tg;
    if (!f32_opt(g, "gemma4.rope.freq_base_swa", &tl) && !f32_opt(g, "gemma4.rope.local_theta", &tl)) tl = c.rope_theta;
    if (!f32_opt(g, "gemma4.rope.freq_base", &tg) && !f32_opt(g, "gemma4.rope.global_theta", &tg)) tg = c.rope_theta;
    for (int i = 0; i < c.n_layers; ++i) {
      const MetaValue& it = pat->arr[i];
      bool swa;
      if (it.type == 7) swa = it.b;
      else if (it.type == 0 || it.type == 4) swa = it.u != 0;
      else if (it.type == 1 || it.type == 5) swa = it.i != 0;
      else fail(ST_MODEL, "gemma4.attention.sliding_window_pattern must be bool[] (or integer 0/1)");
      LayerSpec& L = c.layers[i];
      size_t rd = std::min(swa ? rl : rg, (size_t)L.head_dim);
      if (rd == 0) rd = (size_t)L.head_dim;
      if (rd % 2) rd -= 1;
      L.rotary_dim = (int)rd;
      L.window = swa ? (int)window : -1;
      L.rope_theta = swa ? tl : tg;
    }
  }
  if (c.family == FAM_GEMMA4) {
    size_t pd;
    c.ple_dim = usize_opt(g, "gemma4.embedding_length_per_layer_input", &pd) ? (int)pd : 0;
    c.embed_scale = sqrtf((float)c.hidden);
    if (c.ple_dim > 0) {
      c.ple_combine_scale = 1.0f / sqrtf(2.0f);
      c.ple_proj_scale = 1.0f / sqrtf((float)c.hidden);
    }
    size_t ns = 0;
    if (!usize_opt(g, "gemma4.attention.shared_kv_layers", &ns)) ns = 0;
    if (ns > 0) {
      if ((int)ns > c.n_layers) fail(ST_MODEL, "gemma4 attention.shared_kv_layers exceeds block_count");
      int first = c.n_layers - (int)ns;
      if (first == 0) fail(ST_MODEL, "gemma4: shared_kv_layers == block_count is unsupported (no KV source layer)");
      for (int li = first; li < c.n_layers; ++li) {
        bool want = c.layers[li].window >= 0;
        int src = -1;
        for (int s = first - 1; s >= 0; --s)
          if ((c.layers[s].window >= 0) == want) {
            src = s;
            break;
          }
        if (src < 0) fail(ST_MODEL, "Gemma 4: no KV-borrow source for layer " + std::to_string(li));
        c.layers[li].kv_borrow = src;
      }
    }
  }
  if (f32_opt(g, "gemma4.final_logit_softcapping", &f) && f > 0.0f && std::isfinite(f)) {
    c.has_softcap = true;
    c.softcap = f;
  }
  // TokenizerPromptConfig::from_gguf (src/model_config.rs:35-60): llama.cpp's implicit defaults
  // for a SentencePiece ("llama") vocabulary are add BOS, no EOS; keys override them
  const bool spm = str_meta(g, "tokenizer.ggml.model") == "llama";
  c.add_bos = spm;
  c.add_eos = false;
  bool_opt(g, "tokenizer.ggml.add_bos_token", &c.add_bos);
  bool_opt(g, "tokenizer.ggml.add_eos_token", &c.add_eos);
  if (!u32_opt(g, "tokenizer.ggml.bos_token_id", &c.bos_id)) c.bos_id = 1;
  if (!u32_opt(g, "tokenizer.ggml.eos_token_id", &c.eos_id)) c.eos_id = 2;
  return c;
}

// ---- weights ----
namespace {

std::string resolve(const GgufFile& g, std::initializer_list<std::string> cands, bool required = true) {
  for (auto& c : cands)
    if (g.tensor(c)) return c;
  if (required) fail(ST_MODEL, "none of the candidate tensor names were found: [" + *cands.begin() + ", ...]");
  return "";
}

int dtype_of(uint32_t ggml) {
  switch (ggml) {
    case 0: case 1: case 30: return DT_F32;
    case 12: return DT_Q4K;
    case 14: return DT_Q6K;
    case 8: return DT_Q8_0;
  }
  if (ggml > 40 || ggml == 4 || ggml == 5 || (ggml > 30 && ggml < 34) || (ggml > 35 && ggml < 39))
    fail(ST_GGUF, "unknown GGML type id: " + std::to_string(ggml));
  fail(ST_TENSOR, "unsupported GGML type for inference: " + std::to_string(ggml));
}

size_t byte_len(int dt, size_t n) {
  switch (dt) {
    case DT_Q4K: return (n + 255) / 256 * 144;
    case DT_Q6K: return (n + 255) / 256 * 210;
    case DT_Q8_0: return (n + 31) / 32 * 34;
    default: return n * 4;
  }
}

}  // namespace

Model::~Model() {
  for (auto& t : rope_tables)
    if (t.dev) (void)hipFree(t.dev);
  if (blob) (void)hipFree(blob);
  if (blob_r) (void)hipFree(blob_r);
}

static double ms_since(std::chrono::steady_clock::time_point t0) {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

// Read-only mapping of the whole GGUF file (the tensor bytes are copied out of it once).
struct FileMap {
  const uint8_t* p = nullptr;
  size_t n = 0;
  explicit FileMap(const std::string& path) {
    int fd = open(path.c_str(), O_RDONLY);
    if (fd < 0) fail(ST_IO, "cannot open " + path);
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
      close(fd);
      fail(ST_IO, "cannot stat " + path);
    }
    n = (size_t)sb.st_size;
    void* a = n ? mmap(nullptr, n, PROT_READ, MAP_PRIVATE, fd, 0) : nullptr;
    close(fd);
    if (n && a == MAP_FAILED) fail(ST_IO, "cannot map " + path);
    p = static_cast<const uint8_t*>(a);
    if (n) madvise(a, n, MADV_SEQUENTIAL);
  }
  ~FileMap() {
    if (p) munmap(const_cast<uint8_t*>(p), n);
  }
  const uint8_t* at(uint64_t off, size_t bytes) const {
    if (off > n || bytes > n - off) fail(ST_IO, "failed to fill whole buffer");
    return p + off;
  }
};

Model* load_model(const std::string& path, int device) {
  FILE* probe = fopen(path.c_str(), "rb");
  if (!probe) fail(ST_MODEL, "model file not found: " + path);
  fclose(probe);
  std::unique_ptr<Model> m(new Model());
  m->device = device;
  m->path = path;
  auto t0 = std::chrono::steady_clock::now();
  GgufFile g = read_gguf(path);
  m->timings.gguf_metadata_ms = ms_since(t0);
  t0 = std::chrono::steady_clock::now();
  m->cfg = config_from_gguf(g);
  const Config& c = m->cfg;

  // Name resolution (names.rs:52-222): the same candidates, the same tied-head fallback.
  struct Want {
    DevTensor* dst;
    std::string name;
  };
  std::vector<Want> wants;
  auto want = [&](DevTensor* d, const std::string& n) {
    if (!n.empty()) wants.push_back({d, n});
  };
  want(&m->token_embd, resolve(g, {"token_embd.weight", "tok_embeddings.weight", "embeddings.weight"}));
  want(&m->output_norm, resolve(g, {"output_norm.weight", "norm.weight"}));
  std::string head = resolve(g, {"output.weight", "lm_head.weight"}, false);
  if (head.empty()) {
    if (g.tensor("token_embd.weight")) head = "token_embd.weight";
    else fail(ST_MODEL, "LM head: none of output.weight, lm_head.weight, token_embd.weight (tied) found");
  }
  want(&m->lm_head, head);
  m->layers.resize(c.n_layers);
  for (int i = 0; i < c.n_layers; ++i) {
    std::string p = "blk." + std::to_string(i) + ".";
    LayerTensors& L = m->layers[i];
    if (c.family == FAM_GEMMA4) {
      want(&L.attn_post_norm, resolve(g, {p + "post_attention_norm.weight"}));
      want(&L.ffn_post_norm, resolve(g, {p + "post_ffw_norm.weight"}));
      if (c.ple_dim > 0) {
        want(&L.ple_gate, resolve(g, {p + "inp_gate.weight"}));
        want(&L.ple_proj, resolve(g, {p + "proj.weight"}));
        want(&L.ple_post_norm, resolve(g, {p + "post_norm.weight"}));
      }
    }
    want(&L.attn_norm, resolve(g, {p + "attn_norm.weight", p + "attention_norm.weight"}));
    want(&L.ffn_norm, resolve(g, {p + "ffn_norm.weight", p + "feed_forward_norm.weight"}));
    want(&L.wq, resolve(g, {p + "attn_q.weight", p + "wq.weight"}));
    want(&L.wk, resolve(g, {p + "attn_k.weight", p + "wk.weight"}));
    want(&L.wv, resolve(g, {p + "attn_v.weight", p + "wv.weight"}));
    want(&L.wo, resolve(g, {p + "attn_output.weight", p + "wo.weight"}));
    want(&L.gate, resolve(g, {p + "ffn_gate.weight", p + "w1.weight"}));
    want(&L.up, resolve(g, {p + "ffn_up.weight", p + "w3.weight"}));
    want(&L.down, resolve(g, {p + "ffn_down.weight", p + "w2.weight"}));
    want(&L.q_norm, resolve(g, {p + "attn_q_norm.weight"}, false));
    want(&L.k_norm, resolve(g, {p + "attn_k_norm.weight"}, false));
    want(&L.rope_freqs, resolve(g, {p + "rope_freqs.weight", p + "rope_freqs"}, false));
    want(&L.out_scale, resolve(g, {p + "layer_output_scale.weight"}, false));
  }
  if (c.family == FAM_GEMMA4 && c.ple_dim > 0) {
    want(&m->ple_token_embd, resolve(g, {"per_layer_token_embd.weight"}));
    want(&m->ple_model_proj, resolve(g, {"per_layer_model_proj.weight"}));
    want(&m->ple_proj_norm, resolve(g, {"per_layer_proj_norm.weight"}));
  }

  m->timings.config_and_resolve_ms = ms_since(t0);
  t0 = std::chrono::steady_clock::now();

  // Layout: every distinct tensor once, each at a 256-byte aligned offset of one HBM blob.
  struct Slot {
    const TensorMeta* meta;
    int dtype;
    size_t nelem, file_bytes, dev_bytes, off;
  };
  std::map<std::string, size_t> slot_of;
  std::vector<Slot> slots;
  size_t total = 0;
  for (auto& w : wants) {
    if (slot_of.count(w.name)) continue;
    const TensorMeta* t = g.tensor(w.name);
    Slot s{t, dtype_of(t->ggml_type), 1, 0, 0, 0};
    for (size_t d : t->dims) s.nelem *= d;
    s.file_bytes = (t->ggml_type == 30 || t->ggml_type == 1) ? s.nelem * 2 : byte_len(s.dtype, s.nelem);
    s.dev_bytes = byte_len(s.dtype, s.nelem);
    s.off = total;
    total += (s.dev_bytes + 255) & ~size_t(255);
    slot_of[w.name] = slots.size();
    slots.push_back(s);
  }
  IEK_HIP(hipSetDevice(device));
  m->blob_bytes = total;
  IEK_HIP(hipMalloc(&m->blob, std::max<size_t>(total, 256)));

  // Stream tensors in file order out of the mapped file through two pinned staging buffers: the
  // copy of chunk i + 1 into one overlaps the DMA of chunk i from the other.
  std::vector<size_t> order(slots.size());
  for (size_t i = 0; i < order.size(); ++i) order[i] = i;
  std::sort(order.begin(), order.end(), [&](size_t a, size_t b) { return slots[a].meta->offset < slots[b].meta->offset; });
  FileMap fm(path);
  std::vector<std::vector<float>> host_f32(slots.size());
  const size_t CH = 64u << 20;
  void* stage[2] = {nullptr, nullptr};
  hipStream_t st;
  IEK_HIP(hipStreamCreate(&st));
  hipEvent_t ev[2] = {nullptr, nullptr};
  bool ev_used[2] = {false, false};
  int cur = 0;
  auto cleanup = [&]() {
    (void)hipStreamSynchronize(st);
    for (int i = 0; i < 2; ++i) {
      if (ev[i]) (void)hipEventDestroy(ev[i]);
      if (stage[i]) (void)hipHostFree(stage[i]);
    }
    (void)hipStreamDestroy(st);
  };
  try {
    IEK_HIP(hipHostMalloc(&stage[0], CH));
    IEK_HIP(hipHostMalloc(&stage[1], CH));
    IEK_HIP(hipEventCreate(&ev[0]));
    IEK_HIP(hipEventCreate(&ev[1]));
    for (size_t oi : order) {
      Slot& s = slots[oi];
      const uint8_t* src = fm.at(g.data_offset + s.meta->offset, s.file_bytes);
      bool small_f32 = s.dtype == DT_F32 && s.nelem <= (1u << 20);
      const uint32_t gt = s.meta->ggml_type;
      if (gt == 30 || gt == 1) {  // BF16 (tensor_loader.rs:11-16) or F16 -> F32 widening
        std::vector<float> wide(s.nelem);
        for (size_t e = 0; e < s.nelem; ++e) {
          uint16_t h;
          memcpy(&h, src + 2 * e, 2);
          if (gt == 30) {
            uint32_t bits = (uint32_t)h << 16;
            memcpy(&wide[e], &bits, 4);
          } else {
            wide[e] = __half2float(__ushort_as_half(h));
          }
        }
        IEK_HIP(hipMemcpy((char*)m->blob + s.off, wide.data(), s.nelem * 4, hipMemcpyHostToDevice));
        if (small_f32) host_f32[oi] = std::move(wide);
        continue;
      }
      if (small_f32) {
        host_f32[oi].resize(s.nelem);
        memcpy(host_f32[oi].data(), src, s.nelem * 4);
      }
      size_t done = 0;
      while (done < s.file_bytes) {
        size_t n = std::min(CH, s.file_bytes - done);
        if (ev_used[cur]) IEK_HIP(hipEventSynchronize(ev[cur]));
        memcpy(stage[cur], src + done, n);
        IEK_HIP(hipMemcpyAsync((char*)m->blob + s.off + done, stage[cur], n, hipMemcpyHostToDevice, st));
        IEK_HIP(hipEventRecord(ev[cur], st));
        ev_used[cur] = true;
        done += n;
        cur ^= 1;
      }
    }
  } catch (...) {
    cleanup();
    throw;
  }
  cleanup();
  m->timings.tensor_load_ms = ms_since(t0);
  t0 = std::chrono::steady_clock::now();

  for (auto& w : wants) {
    const Slot& s = slots[slot_of[w.name]];
    DevTensor& d = *w.dst;
    d.dtype = s.dtype;
    d.dims = s.meta->dims;
    d.bytes = s.dev_bytes;
    d.dev = (char*)m->blob + s.off;
    d.host_f32 = host_f32[slot_of[w.name]];
    m->by_name[w.name] = &d;
  }

  // Regrouped copies of the matrices the decode matvec streams, laid out for 16-byte lane loads:
  // every Q6_K projection (ffn_down, and attn_v in Q4_K_M files) and LM head (DT_Q6K_R), and
  // every Q8_0 projection and a Q8_0 LM head (DT_Q8_0_R). Same bytes, rearranged; the native blocks stay in place for every other consumer
  // (prefill GEMM, embedding lookups, op-level entry points).
  {
    std::vector<DevTensor*> rg;
    auto consider = [&](DevTensor& t) {
      if (!t.present() || t.dims.size() != 2 || t.dims[0] % 256 != 0) return;
      if (t.dtype != DT_Q6K && t.dtype != DT_Q8_0) return;
      for (DevTensor* o : rg)
        if (o == &t) return;
      rg.push_back(&t);
    };
    for (auto& L : m->layers)
      for (DevTensor* t : {&L.wq, &L.wk, &L.wv, &L.wo, &L.gate, &L.up, &L.down, &L.ple_gate, &L.ple_proj})
        if (t->dtype == DT_Q6K || t->dtype == DT_Q8_0) consider(*t);
    consider(m->lm_head);
    size_t total_r = 0;
    std::vector<size_t> off_r;
    for (DevTensor* t : rg) {
      off_r.push_back(total_r);
      const size_t rb = t->dtype == DT_Q6K ? q6r_row_bytes(t->dims[0] / 256) : q8r_row_bytes(t->dims[0] / 32);
      total_r += (rb * t->dims[1] + 255) / 256 * 256;
    }
    if (total_r) {
      IEK_HIP(hipMalloc(&m->blob_r, total_r));
      for (size_t i = 0; i < rg.size(); ++i) {
        DevTensor* t = rg[i];
        t->dev_r = (char*)m->blob_r + off_r[i];
        if (t->dtype == DT_Q6K) {
          t->dtype_r = DT_Q6K_R;
          launch_repack_q6k(t->dev, (int)t->dims[0], (int)t->dims[1], t->dev_r, nullptr);
        } else {
          t->dtype_r = DT_Q8_0_R;
          launch_repack_q80(t->dev, (int)t->dims[0], (int)t->dims[1], t->dev_r, nullptr);
        }
      }
      IEK_HIP(hipDeviceSynchronize());
    }
  }

  // Shape checks the reference performs lazily (rmsnorm/matmul length checks).
  auto need_len = [&](const DevTensor& t, size_t n, const char* what) {
    if (t.dtype != DT_F32) fail(ST_TENSOR, std::string(what) + ": dtype is not F32");
    size_t e = 1;
    for (size_t d : t.dims) e *= d;
    if (e != n) fail(ST_MODEL, std::string(what) + " weights len != hidden_dim");
  };
  need_len(m->output_norm, c.hidden, "output_norm");
  for (int i = 0; i < c.n_layers; ++i) {
    LayerTensors& L = m->layers[i];
    need_len(L.attn_norm, c.hidden, "attn_norm");
    need_len(L.ffn_norm, c.hidden, "ffn_norm");
    if (L.out_scale.present()) {
      L.has_out_scale = true;
      if (L.out_scale.dtype == DT_F32) {
        if (L.out_scale.host_f32.empty()) fail(ST_MODEL, "layer_output_scale: empty F32 tensor");
        L.out_scale_value = L.out_scale.host_f32[0];
      } else if (L.out_scale.dtype == DT_Q8_0) {
        uint8_t blk[34];
        IEK_HIP(hipMemcpy(blk, L.out_scale.dev, 34, hipMemcpyDeviceToHost));
        uint16_t h = (uint16_t)(blk[0] | (blk[1] << 8));
        __half hh = __ushort_as_half(h);
        L.out_scale_value = __half2float(hh) * (float)(int8_t)blk[2];
      } else {
        fail(ST_MODEL, "layer_output_scale: unsupported dtype for scalar");
      }
    }
  }

  // RoPE (cos, sin) tables, one per distinct (theta, rotary_dim, freq_factors) and covering every
  // position < context_length. Angles follow rope.rs:40-57 exactly: theta_0 = pos and
  // theta *= base^(-2/n_rot) in f32, angle = theta / ff, libm cosf/sinf.
  for (int i = 0; i < c.n_layers; ++i) {
    const LayerSpec& S = c.layers[i];
    LayerTensors& L = m->layers[i];
    const void* ffk = L.rope_freqs.present() ? L.rope_freqs.dev : nullptr;
    int found = -1;
    for (size_t t = 0; t < m->rope_tables.size(); ++t)
      if (m->rope_tables[t].theta == S.rope_theta && m->rope_tables[t].rotary_dim == S.rotary_dim &&
          m->rope_tables[t].ff_key == ffk)
        found = (int)t;
    if (found < 0) {
      const int np = S.rotary_dim / 2;
      const std::vector<float>* ff = ffk ? &L.rope_freqs.host_f32 : nullptr;
      if (ff && ff->size() < (size_t)np) fail(ST_OP, "RoPE freq_factors len < num_pairs");
      std::vector<float> tab((size_t)c.context_length * np * 2);
      const float theta_scale = powf(S.rope_theta, -2.0f / (float)S.rotary_dim);
      for (int pos = 0; pos < c.context_length; ++pos) {
        float theta = (float)pos;
        for (int k = 0; k < np; ++k) {
          float fk = (ff && (*ff)[k] != 0.0f) ? (*ff)[k] : 1.0f;
          float angle = theta / fk;
          tab[((size_t)pos * np + k) * 2] = cosf(angle);
          tab[((size_t)pos * np + k) * 2 + 1] = sinf(angle);
          theta *= theta_scale;
        }
      }
      RopeTable rt{S.rope_theta, S.rotary_dim, ffk, nullptr};
      IEK_HIP(hipMalloc(&rt.dev, std::max<size_t>(tab.size() * 4, 4)));
      IEK_HIP(hipMemcpy(rt.dev, tab.data(), tab.size() * 4, hipMemcpyHostToDevice));
      m->rope_tables.push_back(rt);
      found = (int)m->rope_tables.size() - 1;
    }
    L.rope_table = found;
  }
  m->timings.weights_build_ms = ms_since(t0);
  return m.release();
}

}  // namespace iek
