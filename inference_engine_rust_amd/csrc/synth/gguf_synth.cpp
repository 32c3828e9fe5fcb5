// Seeded synthetic GGUF writer with ggml-layout K-quant / Q8_0 quantisers.
//
// The reference ships no writer or quantiser, and no model file is available offline, so every
// model the engine runs here comes from this generator. Block layouts are the ones the
// reference's dequantisers read (src/ops/quant/quant_k_handler.rs:10-18, :38-135):
//   Q4_K  144 B: f16 d | f16 dmin | scales[12] (6-bit sc/m packed as get_scale_min_k4) | qs[128]
//   Q6_K  210 B: ql[128] | qh[64] | int8 scales[16] | f16 d
//   Q8_0   34 B: f16 d | int8 q[32]
// Values: counter-based normal stream keyed by (seed, tensor name): element i of a tensor depends
// only on (seed, name, i), so multi-threaded generation is deterministic.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <thread>
#include <vector>

namespace {

uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ULL;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
  return x ^ (x >> 31);
}

uint64_t fnv1a(const std::string& s) {
  uint64_t h = 1469598103934665603ULL;
  for (unsigned char c : s) {
    h ^= c;
    h *= 1099511628211ULL;
  }
  return h;
}

// Standard normal pair via Box–Muller from two 53-bit uniforms in (0, 1].
inline void normal_pair(uint64_t key, uint64_t idx, double* z0, double* z1) {
  uint64_t a = splitmix64(key ^ (idx * 2 + 0x243F6A8885A308D3ULL));
  uint64_t b = splitmix64(key ^ (idx * 2 + 1 + 0x13198A2E03707344ULL));
  double u1 = ((a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
  double u2 = (b >> 11) * (1.0 / 9007199254740992.0);
  double r = std::sqrt(-2.0 * std::log(u1));
  double t = 6.283185307179586476925 * u2;
  *z0 = r * std::cos(t);
  *z1 = r * std::sin(t);
}

// Fill out[0..n) with mean + std * N(0,1) for elements [start, start+n) of the stream `key`.
// Elements 2i and 2i+1 are the two outputs of Box–Muller pair i.
void gen_normal(uint64_t key, size_t start, size_t n, float mean, float stdv, float* out) {
  size_t i = 0;
  while (i < n) {
    size_t e = start + i;
    double z0, z1;
    normal_pair(key, e / 2, &z0, &z1);
    if ((e & 1) == 0) {
      out[i++] = (float)(mean + stdv * z0);
      if (i < n) out[i++] = (float)(mean + stdv * z1);
    } else {
      out[i++] = (float)(mean + stdv * z1);
    }
  }
}

// f32 -> IEEE half, round to nearest even (handles subnormals, overflow -> inf).
uint16_t f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000;
  uint32_t mant = x & 0x7FFFFF;
  int exp = (int)((x >> 23) & 0xFF);
  if (exp == 0xFF) return (uint16_t)(sign | 0x7C00 | (mant ? 0x200 : 0));
  int e = exp - 127 + 15;
  if (e >= 0x1F) return (uint16_t)(sign | 0x7C00);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    mant |= 0x800000;
    int shift = 14 - e;
    uint32_t half = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1);
    uint32_t mid = 1u << (shift - 1);
    if (rem > mid || (rem == mid && (half & 1))) half++;
    return (uint16_t)(sign | half);
  }
  uint32_t half = ((uint32_t)e << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1FFF;
  if (rem > 0x1000 || (rem == 0x1000 && (half & 1))) half++;
  return (uint16_t)(sign | half);
}

float f16_to_f32(uint16_t h) {
  uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 0x1F, m = h & 0x3FF;
  float v;
  if (e == 0) v = std::ldexp((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = std::ldexp((float)(m | 0x400), (int)e - 25);
  uint32_t bits;
  memcpy(&bits, &v, 4);
  bits |= sign;
  memcpy(&v, &bits, 4);
  return v;
}

inline int nearest(float x) { return (int)std::lrintf(x); }

// Q4_K: per 32-value sub-block an affine (scale, min) pair, both 6-bit multiples of f16 d / dmin.
void quantize_q4k(const float* x, uint8_t* b) {
  float scales[8], mins[8];
  for (int j = 0; j < 8; ++j) {
    float mn = x[32 * j], mx = x[32 * j];
    for (int l = 1; l < 32; ++l) {
      mn = std::min(mn, x[32 * j + l]);
      mx = std::max(mx, x[32 * j + l]);
    }
    float m = mn < 0 ? -mn : 0.0f;  // dequant is d*sc*q - dmin*m, so m >= 0 carries -min
    scales[j] = (mx + m) / 15.0f;
    mins[j] = m;
  }
  float ms = 0, mm = 0;
  for (int j = 0; j < 8; ++j) {
    ms = std::max(ms, scales[j]);
    mm = std::max(mm, mins[j]);
  }
  uint16_t dh = f32_to_f16(ms / 63.0f), mh = f32_to_f16(mm / 63.0f);
  float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
  uint8_t sc[8], mq[8];
  for (int j = 0; j < 8; ++j) {
    sc[j] = (uint8_t)(d > 0 ? std::min(63, std::max(0, nearest(scales[j] / d))) : 0);
    mq[j] = (uint8_t)(dmin > 0 ? std::min(63, std::max(0, nearest(mins[j] / dmin))) : 0);
  }
  memcpy(b, &dh, 2);
  memcpy(b + 2, &mh, 2);
  uint8_t* s = b + 4;
  for (int j = 0; j < 4; ++j) {
    s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
    s[j + 4] = (uint8_t)((mq[j] & 63) | ((mq[j + 4] >> 4) << 6));
    s[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mq[j + 4] & 0xF) << 4));
  }
  uint8_t q[256];
  for (int j = 0; j < 8; ++j) {
    float ds = d * (float)sc[j], dm = dmin * (float)mq[j];
    for (int l = 0; l < 32; ++l) {
      int v = ds > 0 ? nearest((x[32 * j + l] + dm) / ds) : 0;
      q[32 * j + l] = (uint8_t)std::min(15, std::max(0, v));
    }
  }
  uint8_t* qs = b + 16;
  for (int g = 0; g < 4; ++g)
    for (int l = 0; l < 32; ++l) qs[32 * g + l] = (uint8_t)(q[64 * g + l] | (q[64 * g + 32 + l] << 4));
}

// Q6_K: per 16-value sub-block an int8 scale; q in [-32, 31].
void quantize_q6k(const float* x, uint8_t* b) {
  float sub[16];
  float amax_all = 0;
  for (int j = 0; j < 16; ++j) {
    float am = 0, v = 0;
    for (int l = 0; l < 16; ++l) {
      float a = std::fabs(x[16 * j + l]);
      if (a > am) {
        am = a;
        v = x[16 * j + l];
      }
    }
    sub[j] = v / -32.0f;  // the extreme value maps to q = -32
    amax_all = std::max(amax_all, std::fabs(sub[j]));
  }
  uint16_t dh = f32_to_f16(amax_all / 127.0f);
  float d = f16_to_f32(dh);
  int8_t sc[16];
  for (int j = 0; j < 16; ++j) sc[j] = (int8_t)(d > 0 ? std::min(127, std::max(-128, nearest(sub[j] / d))) : 0);
  uint8_t q[256];
  for (int e = 0; e < 256; ++e) {
    float ds = d * (float)sc[e / 16];
    int v = ds != 0 ? nearest(x[e] / ds) : 0;
    q[e] = (uint8_t)(std::min(31, std::max(-32, v)) + 32);
  }
  uint8_t *ql = b, *qh = b + 128;
  for (int h = 0; h < 2; ++h)
    for (int l = 0; l < 32; ++l) {
      const uint8_t* qq = q + 128 * h;
      uint8_t q1 = qq[l], q2 = qq[l + 32], q3 = qq[l + 64], q4 = qq[l + 96];
      ql[64 * h + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
      ql[64 * h + l + 32] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
      qh[32 * h + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
    }
  memcpy(b + 192, sc, 16);
  memcpy(b + 208, &dh, 2);
}

void quantize_q8_0(const float* x, uint8_t* b) {
  float am = 0;
  for (int l = 0; l < 32; ++l) am = std::max(am, std::fabs(x[l]));
  uint16_t dh = f32_to_f16(am / 127.0f);
  float d = f16_to_f32(dh);
  memcpy(b, &dh, 2);
  for (int l = 0; l < 32; ++l) b[2 + l] = (uint8_t)(int8_t)(d > 0 ? std::min(127, std::max(-127, nearest(x[l] / d))) : 0);
}

// T_F32_H: stored as F32, values rounded to f16 first (the F32 twin of a T_F16 tensor)
enum { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q4K = 12, T_Q6K = 14, T_BF16 = 30, T_F32_H = 1001 };

size_t block_elems(int t) { return t == T_Q8_0 ? 32 : 256; }
size_t block_bytes(int t) { return t == T_Q4K ? 144 : t == T_Q6K ? 210 : 34; }
size_t tensor_bytes(int t, size_t n) {
  if (t == T_F32 || t == T_F32_H) return n * 4;
  if (t == T_BF16 || t == T_F16) return n * 2;
  return (n + block_elems(t) - 1) / block_elems(t) * block_bytes(t);
}

void parallel_chunks(size_t n, int threads, const std::function<void(size_t, size_t)>& f) {
  if (threads <= 1 || n < 1024) {
    f(0, n);
    return;
  }
  std::vector<std::thread> th;
  size_t per = (n + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    size_t a = t * per, e = std::min(n, a + per);
    if (a >= e) break;
    th.emplace_back(f, a, e);
  }
  for (auto& x : th) x.join();
}

// Generate one tensor's on-disk bytes.
std::vector<uint8_t> make_tensor(uint64_t seed, const std::string& name, int type, size_t nelem, float mean,
                                 float stdv, int threads) {
  uint64_t key = splitmix64(seed ^ fnv1a(name));
  std::vector<uint8_t> out(tensor_bytes(type, nelem));
  if (type == T_F32) {
    std::vector<float> v(nelem);
    parallel_chunks(nelem, threads, [&](size_t a, size_t e) { gen_normal(key, a, e - a, mean, stdv, v.data() + a); });
    memcpy(out.data(), v.data(), nelem * 4);
    return out;
  }
  if (type == T_F16 || type == T_F32_H) {  // IEEE half, round to nearest even
    parallel_chunks(nelem, threads, [&](size_t a, size_t e) {
      std::vector<float> v(e - a);
      gen_normal(key, a, e - a, mean, stdv, v.data());
      for (size_t i = a; i < e; ++i) {
        const uint16_t h = f32_to_f16(v[i - a]);
        if (type == T_F16) {
          memcpy(out.data() + 2 * i, &h, 2);
        } else {
          const float w = f16_to_f32(h);
          memcpy(out.data() + 4 * i, &w, 4);
        }
      }
    });
    return out;
  }
  if (type == T_BF16) {  // round to nearest even on the upper 16 bits
    parallel_chunks(nelem, threads, [&](size_t a, size_t e) {
      std::vector<float> v(e - a);
      gen_normal(key, a, e - a, mean, stdv, v.data());
      for (size_t i = a; i < e; ++i) {
        uint32_t x;
        memcpy(&x, &v[i - a], 4);
        uint16_t h = (uint16_t)((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
        memcpy(out.data() + 2 * i, &h, 2);
      }
    });
    return out;
  }
  size_t be = block_elems(type), bb = block_bytes(type), nb = (nelem + be - 1) / be;
  parallel_chunks(nb, threads, [&](size_t a, size_t e) {
    float buf[256];
    for (size_t blk = a; blk < e; ++blk) {
      size_t s0 = blk * be, cnt = std::min(be, nelem - s0);
      gen_normal(key, s0, cnt, mean, stdv, buf);
      for (size_t i = cnt; i < be; ++i) buf[i] = 0.0f;  // tail of a partial last block
      uint8_t* dst = out.data() + blk * bb;
      if (type == T_Q4K) quantize_q4k(buf, dst);
      else if (type == T_Q6K) quantize_q6k(buf, dst);
      else quantize_q8_0(buf, dst);
    }
  });
  return out;
}

// ---- minimal GGUF v3 writer ----
struct KV {
  std::string key;
  uint32_t type;
  std::vector<uint8_t> payload;
};
struct TI {
  std::string name;
  std::vector<uint64_t> dims;
  uint32_t type;
  float mean, stdv;
};

void put_str(std::vector<uint8_t>& o, const std::string& s) {
  uint64_t n = s.size();
  o.insert(o.end(), (uint8_t*)&n, (uint8_t*)&n + 8);
  o.insert(o.end(), s.begin(), s.end());
}
template <class T>
void put(std::vector<uint8_t>& o, T v) {
  o.insert(o.end(), (uint8_t*)&v, (uint8_t*)&v + sizeof(T));
}
KV kv_u32(const std::string& k, uint32_t v) {
  KV x{k, 4, {}};
  put(x.payload, v);
  return x;
}
KV kv_f32(const std::string& k, float v) {
  KV x{k, 6, {}};
  put(x.payload, v);
  return x;
}
KV kv_str(const std::string& k, const std::string& v) {
  KV x{k, 8, {}};
  put_str(x.payload, v);
  return x;
}
KV kv_bool_arr(const std::string& k, const std::vector<bool>& v) {
  KV x{k, 9, {}};
  put<uint32_t>(x.payload, 7);
  put<uint64_t>(x.payload, v.size());
  for (bool b : v) put<uint8_t>(x.payload, b ? 1 : 0);
  return x;
}

// Header + tensor data for `tis` (offsets aligned to 32 like general.alignment).
int write_gguf(const char* path, const std::vector<KV>& kvs, const std::vector<TI>& tis, uint64_t seed, int threads) {
  std::vector<uint8_t> head;
  head.insert(head.end(), {'G', 'G', 'U', 'F'});
  put<uint32_t>(head, 3);
  put<uint64_t>(head, tis.size());
  put<uint64_t>(head, kvs.size());
  for (auto& k : kvs) {
    put_str(head, k.key);
    put<uint32_t>(head, k.type);
    head.insert(head.end(), k.payload.begin(), k.payload.end());
  }
  uint64_t off = 0;
  std::vector<uint64_t> offs;
  for (auto& t : tis) {
    put_str(head, t.name);
    put<uint32_t>(head, (uint32_t)t.dims.size());
    for (auto d : t.dims) put<uint64_t>(head, d);
    put<uint32_t>(head, t.type == T_F32_H ? (uint32_t)T_F32 : t.type);
    put<uint64_t>(head, off);
    offs.push_back(off);
    size_t n = 1;
    for (auto d : t.dims) n *= d;
    off += tensor_bytes((int)t.type, n);
    off = (off + 31) & ~uint64_t(31);
  }
  while (head.size() % 32) head.push_back(0);
  FILE* f = fopen(path, "wb");
  if (!f) return 1;
  if (fwrite(head.data(), 1, head.size(), f) != head.size()) {
    fclose(f);
    return 2;
  }
  uint64_t written = 0;
  for (size_t i = 0; i < tis.size(); ++i) {
    auto& t = tis[i];
    size_t n = 1;
    for (auto d : t.dims) n *= d;
    std::vector<uint8_t> data = make_tensor(seed, t.name, (int)t.type, n, t.mean, t.stdv, threads);
    std::vector<uint8_t> pad(offs[i] - written, 0);
    if (!pad.empty() && fwrite(pad.data(), 1, pad.size(), f) != pad.size()) {
      fclose(f);
      return 2;
    }
    if (fwrite(data.data(), 1, data.size(), f) != data.size()) {
      fclose(f);
      return 2;
    }
    written = offs[i] + data.size();
  }
  if (fclose(f) != 0) return 3;
  return 0;
}

}  // namespace

extern "C" {

// Model spec for the generator. Types are ggml ids (0 F32, 8 Q8_0, 12 Q4_K, 14 Q6_K).
struct iek_synth_spec {
  const char* name;         // general.name ("...mistral..." keeps Q/K un-permute off)
  uint32_t n_layers, hidden, n_heads, n_kv_heads, ffn, vocab, context_length;
  float rope_theta, rms_eps, weight_std, norm_std;
  uint32_t t_attn, t_ffn_gate_up, t_ffn_down, t_embd, t_output;
  uint32_t tied_output;     // 1: no output.weight (LM head reuses token_embd)
  // Per-layer attn_v / ffn_down types. 0: t_attn / t_ffn_down everywhere. 1: llama.cpp's Q4_K_M
  // rule: Q6_K in the layers it gives more bits (i < n/8, i >= 7n/8, (i - n/8) % 3 == 2), Q4_K in
  // the others. 2: Q6_K in odd layers, Q4_K in even ones (small test models).
  uint32_t mix;
  uint32_t t_norm;          // RMSNorm weights: 0 F32, 1 F16, 2 F32 holding f16-rounded values
};

static bool more_bits(uint32_t mix, uint32_t i, uint32_t n) {
  if (mix == 2) return i % 2 == 1;
  return i < n / 8 || i >= 7 * n / 8 || (i >= n / 8 && (i - n / 8) % 3 == 2);
}

// Writes a Mistral/Llama-family GGUF. Returns 0 on success, nonzero on I/O failure.
int iek_synth_write_llama(const char* path, const iek_synth_spec* sp, uint64_t seed, int threads) {
  const iek_synth_spec& s = *sp;
  uint32_t hd = s.hidden / s.n_heads;
  std::vector<KV> kvs = {
      kv_str("general.architecture", "llama"),
      kv_str("general.name", s.name),
      kv_u32("general.alignment", 32),
      kv_u32("llama.context_length", s.context_length),
      kv_u32("llama.embedding_length", s.hidden),
      kv_u32("llama.block_count", s.n_layers),
      kv_u32("llama.attention.head_count", s.n_heads),
      kv_u32("llama.attention.head_count_kv", s.n_kv_heads),
      kv_u32("llama.feed_forward_length", s.ffn),
      kv_f32("llama.attention.layer_norm_rms_epsilon", s.rms_eps),
      kv_u32("llama.vocab_size", s.vocab),
      kv_f32("llama.rope.theta", s.rope_theta),
      kv_u32("llama.rope.dimension_count", hd),
  };
  std::vector<TI> tis;
  float ws = s.weight_std, ns = s.norm_std;
  tis.push_back({"token_embd.weight", {s.hidden, s.vocab}, s.t_embd, 0.f, ws});
  for (uint32_t l = 0; l < s.n_layers; ++l) {
    std::string p = "blk." + std::to_string(l) + ".";
    const uint32_t t_v = s.mix ? (more_bits(s.mix, l, s.n_layers) ? T_Q6K : T_Q4K) : s.t_attn;
    const uint32_t t_down = s.mix ? (more_bits(s.mix, l, s.n_layers) ? T_Q6K : T_Q4K) : s.t_ffn_down;
    const uint32_t t_n = s.t_norm == 1 ? T_F16 : (s.t_norm == 2 ? T_F32_H : T_F32);
    tis.push_back({p + "attn_norm.weight", {s.hidden}, t_n, 1.f, ns});
    tis.push_back({p + "attn_q.weight", {s.hidden, s.n_heads * hd}, s.t_attn, 0.f, ws});
    tis.push_back({p + "attn_k.weight", {s.hidden, s.n_kv_heads * hd}, s.t_attn, 0.f, ws});
    tis.push_back({p + "attn_v.weight", {s.hidden, s.n_kv_heads * hd}, t_v, 0.f, ws});
    tis.push_back({p + "attn_output.weight", {s.n_heads * hd, s.hidden}, s.t_attn, 0.f, ws});
    tis.push_back({p + "ffn_norm.weight", {s.hidden}, t_n, 1.f, ns});
    tis.push_back({p + "ffn_gate.weight", {s.hidden, s.ffn}, s.t_ffn_gate_up, 0.f, ws});
    tis.push_back({p + "ffn_up.weight", {s.hidden, s.ffn}, s.t_ffn_gate_up, 0.f, ws});
    tis.push_back({p + "ffn_down.weight", {s.ffn, s.hidden}, t_down, 0.f, ws});
  }
  tis.push_back({"output_norm.weight", {s.hidden}, s.t_norm == 1 ? T_F16 : (s.t_norm == 2 ? T_F32_H : T_F32), 1.f, ns});
  if (!s.tied_output) tis.push_back({"output.weight", {s.hidden, s.vocab}, s.t_output, 0.f, ws});
  return write_gguf(path, kvs, tis, seed, threads);
}

// Gemma-4-architecture spec. Layer i is a sliding-window layer unless (i % global_every) ==
// global_every - 1; sliding layers use head_dim_swa, global layers head_dim_global (per-layer
// dims are read back from the Q/K weight shapes, model_config.rs:374-444). The last
// shared_kv_layers layers borrow K/V from an earlier layer of the same kind (model_config.rs:332-372).
struct iek_synth_gemma_spec {
  const char* name;
  uint32_t n_layers, hidden, n_heads, n_kv_heads, head_dim_swa, head_dim_global, ffn, vocab, context_length;
  uint32_t ple_dim, sliding_window, global_every, shared_kv_layers, rot_swa, rot_global;
  float theta_swa, theta_global, rms_eps, weight_std, norm_std, softcap;
  uint32_t t_weights;       // projections (ggml type)
  uint32_t t_embd;          // token_embd (also the tied LM head)
  uint32_t t_ple_embd;      // per_layer_token_embd
  uint32_t t_ple_proj;      // per_layer_model_proj (F32 or BF16)
  uint32_t rope_freqs;      // 1: global layers carry rope_freqs (factors in [1, 2))
  uint32_t q8_layer_scale;  // 1: odd layers store layer_output_scale as one Q8_0 block
};

int iek_synth_write_gemma4(const char* path, const iek_synth_gemma_spec* sp, uint64_t seed, int threads) {
  const iek_synth_gemma_spec& s = *sp;
  const uint32_t ge = s.global_every ? s.global_every : 1;
  std::vector<bool> swa(s.n_layers);
  for (uint32_t i = 0; i < s.n_layers; ++i) swa[i] = (i % ge) != ge - 1;
  std::vector<KV> kvs = {
      kv_str("general.architecture", "gemma4"),
      kv_str("general.name", s.name),
      kv_u32("general.alignment", 32),
      kv_u32("gemma4.context_length", s.context_length),
      kv_u32("gemma4.embedding_length", s.hidden),
      kv_u32("gemma4.block_count", s.n_layers),
      kv_u32("gemma4.attention.head_count", s.n_heads),
      kv_u32("gemma4.attention.head_count_kv", s.n_kv_heads),
      kv_u32("gemma4.feed_forward_length", s.ffn),
      kv_f32("gemma4.attention.layer_norm_rms_epsilon", s.rms_eps),
      kv_u32("gemma4.vocab_size", s.vocab),
      kv_f32("gemma4.rope.freq_base", s.theta_global),
      kv_f32("gemma4.rope.freq_base_swa", s.theta_swa),
      kv_u32("gemma4.rope.dimension_count", s.rot_global),
      kv_u32("gemma4.rope.dimension_count_swa", s.rot_swa),
      kv_u32("gemma4.attention.sliding_window", s.sliding_window),
      kv_bool_arr("gemma4.attention.sliding_window_pattern", swa),
      kv_u32("gemma4.attention.shared_kv_layers", s.shared_kv_layers),
      kv_u32("gemma4.embedding_length_per_layer_input", s.ple_dim),
      kv_f32("gemma4.final_logit_softcapping", s.softcap),
  };
  std::vector<TI> tis;
  const float ws = s.weight_std, ns = s.norm_std;
  const uint32_t pack = s.n_layers * s.ple_dim;
  tis.push_back({"token_embd.weight", {s.hidden, s.vocab}, s.t_embd, 0.f, ws});
  if (s.ple_dim) {
    tis.push_back({"per_layer_token_embd.weight", {pack, s.vocab}, s.t_ple_embd, 0.f, ws});
    tis.push_back({"per_layer_model_proj.weight", {s.hidden, pack}, s.t_ple_proj, 0.f, ws});
    tis.push_back({"per_layer_proj_norm.weight", {s.ple_dim}, T_F32, 1.f, ns});
  }
  for (uint32_t l = 0; l < s.n_layers; ++l) {
    const std::string p = "blk." + std::to_string(l) + ".";
    const uint32_t hd = swa[l] ? s.head_dim_swa : s.head_dim_global;
    const uint32_t qd = s.n_heads * hd, kvd = s.n_kv_heads * hd;
    tis.push_back({p + "attn_norm.weight", {s.hidden}, T_F32, 1.f, ns});
    tis.push_back({p + "attn_q.weight", {s.hidden, qd}, s.t_weights, 0.f, ws});
    tis.push_back({p + "attn_k.weight", {s.hidden, kvd}, s.t_weights, 0.f, ws});
    tis.push_back({p + "attn_v.weight", {s.hidden, kvd}, s.t_weights, 0.f, ws});
    tis.push_back({p + "attn_q_norm.weight", {hd}, T_F32, 1.f, ns});
    tis.push_back({p + "attn_k_norm.weight", {hd}, T_F32, 1.f, ns});
    tis.push_back({p + "attn_output.weight", {qd, s.hidden}, s.t_weights, 0.f, ws});
    tis.push_back({p + "post_attention_norm.weight", {s.hidden}, T_F32, 1.f, ns});
    tis.push_back({p + "ffn_norm.weight", {s.hidden}, T_F32, 1.f, ns});
    tis.push_back({p + "ffn_gate.weight", {s.hidden, s.ffn}, s.t_weights, 0.f, ws});
    tis.push_back({p + "ffn_up.weight", {s.hidden, s.ffn}, s.t_weights, 0.f, ws});
    tis.push_back({p + "ffn_down.weight", {s.ffn, s.hidden}, s.t_weights, 0.f, ws});
    tis.push_back({p + "post_ffw_norm.weight", {s.hidden}, T_F32, 1.f, ns});
    if (s.ple_dim) {
      tis.push_back({p + "inp_gate.weight", {s.hidden, s.ple_dim}, s.t_weights, 0.f, ws});
      tis.push_back({p + "proj.weight", {s.ple_dim, s.hidden}, s.t_weights, 0.f, ws});
      tis.push_back({p + "post_norm.weight", {s.hidden}, T_F32, 1.f, ns});
    }
    if (s.rope_freqs && !swa[l]) tis.push_back({p + "rope_freqs.weight", {s.rot_global / 2}, T_F32, 1.5f, 0.25f});
    if (s.q8_layer_scale && (l & 1))
      tis.push_back({p + "layer_output_scale.weight", {32}, T_Q8_0, 1.f, 0.05f});
    else
      tis.push_back({p + "layer_output_scale.weight", {1}, T_F32, 1.f, 0.05f});
  }
  tis.push_back({"output_norm.weight", {s.hidden}, T_F32, 1.f, ns});
  return write_gguf(path, kvs, tis, seed, threads);
}

// Quantise `nblocks` blocks of float input (type 8/12/14) — used by tests to build weights.
int iek_synth_quantize(int type, const float* x, size_t nblocks, uint8_t* out) {
  size_t be = block_elems(type), bb = block_bytes(type);
  for (size_t b = 0; b < nblocks; ++b) {
    if (type == T_Q4K) quantize_q4k(x + b * be, out + b * bb);
    else if (type == T_Q6K) quantize_q6k(x + b * be, out + b * bb);
    else if (type == T_Q8_0) quantize_q8_0(x + b * be, out + b * bb);
    else return 1;
  }
  return 0;
}

// Deterministic N(mean, std) stream, exposed so tests can make seeded activations.
void iek_synth_normal(uint64_t seed, const char* name, size_t start, size_t n, float mean, float stdv, float* out) {
  gen_normal(splitmix64(seed ^ fnv1a(name)), start, n, mean, stdv, out);
}

uint16_t iek_synth_f32_to_f16(float f) { return f32_to_f16(f); }

}  // extern "C"
