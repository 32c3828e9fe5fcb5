// Session forward passes. Layer order and numerics follow the reference's layer code:
//   prefill_layer_block / decode_layer_block     src/layers/block.rs:12-89
//   mistral_*_attention_with_norm                src/layers/attention.rs:713-890
//   prefill_attention_layer / decode_attention   src/layers/attention.rs:175-655
//   mistral_prefill_ffn_with_norm / prefill_ffn  src/layers/ffn.rs:16-117
//   final_logits_last_token                      src/engine/runtime.rs:76-116
//   Gemma-4: head norms, post-norms, GeGLU, PLE  attention.rs:277-308,424-455; ffn.rs:120-278;
//                                                src/layers/gemma4_ple.rs:27-109; embed.rs:53-149
#include "session.h"

#include <functional>
#include <mutex>

#include "kernels/chain.h"
#include "kernels/mv_args.h"

#include <cmath>
#include <cstring>

namespace iek {

namespace {

template <class T>
T* dev_alloc(size_t n) {
  void* p = nullptr;
  IEK_HIP(hipMalloc(&p, std::max<size_t>(n * sizeof(T), 16)));
  return static_cast<T*>(p);
}

void dev_free(void* p) {
  if (p) (void)hipFree(p);
}

// A chain launch waits on its own workgroups across the whole GPU, so it needs every compute unit
// to itself: two sessions' chain steps overlapping on one device would each get part of the CUs,
// and their bounded waits would run out. Sessions on one device therefore take turns: a step's
// work waits on its stream for the previous chain step of any session on the device (an event per
// device), and records that event when its own work is enqueued. Work from another process on the
// same GPU is not ordered by this; a chain step it starves fails with IEK_ERR_DEVICE.
struct ChainOrder {
  std::mutex mu;
  hipEvent_t last = nullptr;
};
ChainOrder g_chain_order[64];

class ChainTurn {
 public:
  ChainTurn(int dev, hipStream_t st, bool on) : st_(st) {
    if (!on) return;
    if (dev < 0 || dev >= 64) fail(ST_DEVICE, "device index out of range");
    o_ = &g_chain_order[dev];
    lock_ = std::unique_lock<std::mutex>(o_->mu);
    if (!o_->last) IEK_HIP(hipEventCreateWithFlags(&o_->last, hipEventDisableTiming));
    else IEK_HIP(hipStreamWaitEvent(st, o_->last, 0));
  }
  ~ChainTurn() {
    if (o_) (void)hipEventRecord(o_->last, st_);
  }

 private:
  ChainOrder* o_ = nullptr;
  std::unique_lock<std::mutex> lock_;
  hipStream_t st_;
};

}  // namespace

Session::Session(Model* m) : m_(m) {
  const Config& c = m->cfg;
  gemma_ = c.family == FAM_GEMMA4;
  IEK_HIP(hipSetDevice(m->device));
  IEK_HIP(hipStreamCreateWithFlags(&st_, hipStreamNonBlocking));
  ctx_ = c.context_length;
  H_ = c.hidden;
  // KV cache (fp16): per layer K and V as [n_kv][ctx][head_dim] (kv_caches_for_config,
  // attention.rs:129-135, sizes every cache to context_length).
  // A layer that borrows another layer's KV (Gemma-4 shared-KV layers, model_config.rs:332-372)
  // never appends to its own cache; it gets none and aliases its source's.
  // The cache keeps the reference's f32 keys and values (KVCache, attention.rs:16-24). Rounding
  // them to fp16 is not within the logits bar: applied to the reference's own CPU path (the oracle
  // with fp16-rounded K and V), it moves the decode logits of the 32-layer Mistral-7B-shaped model
  // by 2.4e-3 relative L2 (K alone 2.1e-3, V alone 1.3e-3) and of the 2-layer one by 7e-4; Gemma-4
  // (q/k head norms, score scale 1) moves by ~1e-2.
  kv_f32_ = true;
  const size_t esz = kv_f32_ ? 4 : 2;
  size_t total = 0;
  for (auto& L : c.layers)
    if (L.kv_borrow < 0) total += 2 * (size_t)c.n_kv_heads * ctx_ * L.head_dim;
  IEK_HIP(hipMalloc(&kv_blob_, std::max<size_t>(total * esz, 16)));
  // zeroed once for determinism of copies; no kernel lets a row past the live keys reach a result
  IEK_HIP(hipMemset(kv_blob_, 0, std::max<size_t>(total * esz, 16)));
  char* p = static_cast<char*>(kv_blob_);
  for (int li = 0; li < c.n_layers; ++li) {
    const LayerSpec& L = c.layers[li];
    if (L.kv_borrow >= 0) {
      if (L.kv_borrow >= li || c.layers[L.kv_borrow].head_dim != L.head_dim)
        fail(ST_MODEL, "borrow source KV shape mismatch");
      kc_.push_back(kc_[L.kv_borrow]);
      vc_.push_back(vc_[L.kv_borrow]);
      continue;
    }
    size_t per = (size_t)c.n_kv_heads * ctx_ * L.head_dim * esz;
    kc_.push_back(p);
    vc_.push_back(p + per);
    p += 2 * per;
  }
  int qmax = 0, kvmax = 0, fmax = 0, hdmax = 0;
  for (auto& L : c.layers) {
    qmax = std::max(qmax, L.q_dim);
    kvmax = std::max(kvmax, L.kv_dim);
    fmax = std::max(fmax, L.ffn_dim);
    hdmax = std::max(hdmax, L.head_dim);
  }
  xdec_ = dev_alloc<float>(H_);
  xdec2_ = dev_alloc<float>(H_);
  xdec_save_ = dev_alloc<float>(H_);
  xndec_ = dev_alloc<float>(std::max(H_, qmax));
  qd_ = dev_alloc<float>(qmax);
  kd_ = dev_alloc<float>(kvmax);
  vd_ = dev_alloc<float>(kvmax);
  attd_ = dev_alloc<float>(qmax);
  actd_ = dev_alloc<float>(fmax);
  tmpd_ = dev_alloc<float>(std::max(qmax, fmax));
  logits_ = dev_alloc<float>(c.vocab);
  const int nsplit = (ctx_ + 63) / 64;
  part_ = dev_alloc<float>((size_t)c.n_heads * nsplit * (hdmax + 2));
  d_pos_ = dev_alloc<int>(1);
  d_step_ = dev_alloc<int>(1);
  d_flags_ = dev_alloc<int>(ctx_ + 1);
  d_tok_ = dev_alloc<uint32_t>(1);
  d_ids_ = dev_alloc<uint32_t>(ctx_);
  d_gen_ = dev_alloc<uint32_t>(ctx_ + 1);
  d_key_ = dev_alloc<unsigned long long>(1);
  d_flag_ = dev_alloc<int>(1);
  d_cnt_ = dev_alloc<int>(2 * c.n_kv_heads);  // per (KV head, query-head group) arrival counters
  d_ovf_ = dev_alloc<int>(1);
  IEK_HIP(hipHostMalloc(reinterpret_cast<void**>(&h_ovf_), sizeof(int), hipHostMallocDefault));
  if (gemma_ && c.ple_dim > 0) {
    const size_t pack = (size_t)c.n_layers * c.ple_dim;
    ple_tokd_ = dev_alloc<float>(pack);
    ple_projd_ = dev_alloc<float>(pack);
    ple_packd_ = dev_alloc<float>(pack);
  }
  launch_fill_u64(d_key_, 0ull, 1, st_);
  launch_fill_i32(d_flag_, 0, 1, st_);
  launch_fill_i32(d_cnt_, 0, 2 * c.n_kv_heads, st_);
  launch_fill_i32(d_ovf_, 0, 1, st_);
  prepare_chain();
  reset();
}

Session::~Session() {
  if (st_) (void)hipStreamSynchronize(st_);
  if (step_exec_) (void)hipGraphExecDestroy(step_exec_);
  if (step_graph_) (void)hipGraphDestroy(step_graph_);
  if (st_) (void)hipStreamSynchronize(st_);
  for (void* p : {(void*)x_, (void*)xn_, (void*)q_, (void*)k_, (void*)v_, (void*)att_, (void*)g_, (void*)u_,
                  (void*)act_, (void*)tmp_, (void*)xdec_, (void*)xndec_, (void*)qd_, (void*)kd_, (void*)vd_,
                  (void*)attd_, (void*)actd_, (void*)logits_, (void*)part_, (void*)tmpd_, (void*)d_pos_,
                  (void*)d_step_, (void*)d_flags_, (void*)d_tok_, (void*)d_ids_, (void*)d_gen_, (void*)d_key_,
                  (void*)d_flag_, (void*)d_cnt_, (void*)xs_, (void*)xsum_, kv_blob_, (void*)ple_tok_,
                  (void*)ple_proj_, (void*)ple_pack_, (void*)ple_tokd_, (void*)ple_projd_, (void*)ple_packd_,
                  (void*)xdec2_, (void*)xdec_save_, chain_blob_, (void*)d_chain_cnt_, (void*)d_chain_err_,
                  (void*)d_ovf_, (void*)x_save_})
    dev_free(p);
  if (h_ovf_) (void)hipHostFree(h_ovf_);
  if (st_) (void)hipStreamDestroy(st_);
}

void Session::sync() {
  IEK_HIP(hipGetLastError());
  IEK_HIP(hipStreamSynchronize(st_));
}

// Whether a prefill kernel flagged an input beyond the fp16 pair's range since d_ovf_ was cleared
// (waits for the stream).
bool Session::overflowed() {
  IEK_HIP(hipMemcpyAsync(h_ovf_, d_ovf_, sizeof(int), hipMemcpyDeviceToHost, st_));
  sync();
  return *h_ovf_ != 0;
}

void Session::reset() {
  launch_set_int(d_pos_, 0, st_);
  pos_ = 0;
  state_rows_ = 0;
  state_prefill_ = false;
  state_ple_ = false;
  layer_cursor_ = 0;
  sync();
}

void Session::ensure_rows(int rows) {
  if (rows <= rows_cap_) return;
  sync();
  for (float** b : {&x_, &xn_, &q_, &k_, &v_, &att_, &g_, &u_, &act_, &tmp_, &ple_tok_, &ple_proj_, &ple_pack_}) {
    dev_free(*b);
    *b = nullptr;
  }
  dev_free(xs_);
  xs_ = nullptr;
  dev_free(xsum_);
  xsum_ = nullptr;
  const Config& c = m_->cfg;
  int qmax = 0, kvmax = 0, fmax = 0;
  for (auto& L : c.layers) {
    qmax = std::max(qmax, L.q_dim);
    kvmax = std::max(kvmax, L.kv_dim);
    fmax = std::max(fmax, L.ffn_dim);
  }
  size_t R = (size_t)rows;
  x_ = dev_alloc<float>(R * H_);
  xn_ = dev_alloc<float>(R * std::max(H_, qmax));
  q_ = dev_alloc<float>(R * qmax);
  k_ = dev_alloc<float>(R * kvmax);
  v_ = dev_alloc<float>(R * kvmax);
  att_ = dev_alloc<float>(R * qmax);
  g_ = dev_alloc<float>(R * fmax);
  u_ = dev_alloc<float>(R * fmax);
  act_ = dev_alloc<float>(R * fmax);
  tmp_ = dev_alloc<float>(R * std::max(qmax, fmax));
  kpart_ok_ = std::max(qmax, fmax) >= H_;  // tmp_ holds a split-K partial of a [rows, hidden] output
  // fp16 (hi, lo) pair of the widest GEMM input, for the matrix-core prefill projections
  xs_halves_ = 2 * R * std::max(std::max(H_, qmax), fmax);
  xs_ = dev_alloc<__half>(xs_halves_);
  xsum_ = dev_alloc<float>(R * std::max(std::max(H_, qmax), fmax) / 32 + 1);
  if (gemma_ && c.ple_dim > 0) {
    const size_t pack = (size_t)c.n_layers * c.ple_dim;
    ple_tok_ = dev_alloc<float>(R * pack);
    ple_proj_ = dev_alloc<float>(R * pack);
    ple_pack_ = dev_alloc<float>(R * pack);
  }
  rows_cap_ = rows;
}

// The weight copy the decode matvec streams: the regrouped layout when the model built one, else
// the native blocks.
static const void* mv_weight(const DevTensor& t, int K, int* dt) {
  if (t.dev_r && K <= 16384) {
    *dt = t.dtype_r;
    return t.dev_r;
  }
  *dt = t.dtype;
  return t.dev;
}

// One projection over `rows` activation rows: matvec for a single row, GEMM otherwise. `xs` is
// the fp16 (hi, lo) split of `a` when the caller has made it (rows*K halves each), else null.
// `f32`: the prefill's f32 mode (an input beyond the fp16 pair's range was seen): the SIMT GEMM
// on the f32 activation.
static void project(const DevTensor& w, const float* a, const __half* xs, int rows, int K, int N, float* out,
                    const float* resid, hipStream_t st, bool f32 = false) {
  if (w.dims.size() != 2 || (int)w.dims[0] != K || (int)w.dims[1] != N)
    fail(ST_MATMUL, "inner dim mismatch: weight dims do not match the activation width");
  if (rows == 1) {
    MvSegDesc s{w.dev, out, resid, N};
    launch_matvec(w.dtype, &s, 1, a, K, resid ? 1 : 0, st);
  } else if (f32) {
    launch_gemm_f32(w.dtype, w.dev, a, rows, K, N, out, resid, st);
  } else if (xs && gemm_mfma_ok(w.dtype, w.dev, K, N)) {
    launch_gemm_mfma(w.dtype, w.dev, xs, xs + (size_t)rows * K, rows, K, N, out, resid, st);
  } else {
    launch_gemm(w.dtype, w.dev, a, rows, K, N, out, resid, st);
  }
}

// Prefill projections through the scale-factored matrix-core GEMM when every weight qualifies:
// `a` (M x K) must already be split into xs_ (fp16 pair) and summed per 32 into xsum_.
// Returns false when the caller should fall back to per-matrix projections.
// Whether project_q takes these weights (the checks it makes before launching).
bool Session::quant_ready(const DevTensor* const* ws, int nseg, int M, int K) const {
  if (M < 2) return false;
  int dt = -1;
  for (int i = 0; i < nseg; ++i) {
    const DevTensor& w = *ws[i];
    if (w.dims.size() != 2 || (int)w.dims[0] != K) return false;
    int wdt = w.dtype;
    const void* p = w.dev;
    if (w.dev_r && w.dtype_r == DT_Q6K_R) {
      wdt = DT_Q6K_R;
      p = w.dev_r;
    }
    if ((dt >= 0 && wdt != dt) || !gemm_q_ok(wdt, p, K)) return false;
    dt = wdt;
  }
  return true;
}

// The weight pointer and layout the K-quant GEMMs read (the regrouped Q6_K copy when there is one).
static const void* kq_weight(const DevTensor& w, int* dt) {
  if (w.dev_r && w.dtype_r == DT_Q6K_R) {
    *dt = DT_Q6K_R;
    return w.dev_r;
  }
  *dt = w.dtype;
  return w.dev;
}

bool Session::project_q(const DevTensor* const* ws, float* const* outs, int nseg, int M, int K, const float* resid,
                        float* kpart, bool* pending, const __half* xin, const float* sin) {
  if (M < 2) return false;
  int dt = -1;
  GemmQSeg segs[3];
  for (int i = 0; i < nseg; ++i) {
    const DevTensor& w = *ws[i];
    if (w.dims.size() != 2 || (int)w.dims[0] != K) return false;
    int wdt = w.dtype;
    const void* p = w.dev;
    if (w.dev_r && w.dtype_r == DT_Q6K_R) {
      wdt = DT_Q6K_R;
      p = w.dev_r;
    }
    if (dt >= 0 && wdt != dt) return false;
    dt = wdt;
    if (!gemm_q_ok(dt, p, K)) return false;
    segs[i] = GemmQSeg{p, outs[i], (int)w.dims[1]};
  }
  const __half* xh = xin ? xin : xs_;
  const bool left = launch_gemm_q(dt, segs, nseg, xh, xh + (size_t)M * K, sin ? sin : xsum_, M, K, resid, st_, kpart,
                                  pending != nullptr);
  if (pending) *pending = left;
  return true;
}

// Gate/up with SwiGLU in the GEMM epilogue, input in xs_ / xsum_: the act planes go to g_ (as
// halves) and their per-32 sums to u_ (xs_ and xsum_ still hold the GEMM's own input while it
// runs); the f32 act goes to act_ only when the down projection cannot take the planes.
bool Session::gate_up_glu(int li, int M) {
  const LayerTensors& L = m_->layers[li];
  const int ffn = m_->cfg.layers[li].ffn_dim;
  const DevTensor* wgu[2] = {&L.gate, &L.up};
  if (M < 2 || ffn % 32 != 0 || H_ % 32 != 0 || !quant_ready(wgu, 2, M, H_) || (int)L.gate.dims[1] != ffn ||
      (int)L.up.dims[1] != ffn)
    return false;
  int dg = -1, du = -1;
  const void* pg = kq_weight(L.gate, &dg);
  const void* pu = kq_weight(L.up, &du);
  if (dg != du) return false;
  const DevTensor* wd[1] = {&L.down};
  __half* ah = reinterpret_cast<__half*>(g_);
  return launch_gemm_q_glu(dg, pg, pu, ffn, xs_, xs_ + (size_t)M * H_, xsum_, M, H_, ah, ah + (size_t)M * ffn, u_,
                           quant_ready(wd, 1, M, ffn) ? nullptr : act_, d_ovf_, st_);
}

bool Session::layer_prefill(int li, int M, bool pend_in) {
  const Config& c = m_->cfg;
  const LayerSpec& S = c.layers[li];
  const LayerTensors& L = m_->layers[li];
  const int hd = S.head_dim, qd = S.q_dim, kvd = S.kv_dim;
  const float eps = c.rms_eps;
  // attention sub-layer: pre-norm, projections, RoPE at prompt positions 0..M-1, KV append at the
  // cache's current length, causal attention within the prompt, O projection + residual.
  // fp16 pair (and per-32 sums) of a GEMM input, only when it has more than one row and a width
  // the split takes; the pre-norms and SwiGLU emit them as they write their output
  // In the f32 mode no input is split: every projection runs the SIMT GEMM on f32 activations.
  const bool wide = M >= 2 && !f32_prefill_;
  const bool f32 = f32_prefill_;
  auto split = [&](const float* a, int K) -> const __half* {
    if (!wide || K % 32 != 0) return nullptr;
    launch_split_sums(a, M, K, xs_, xs_ + (size_t)M * K, xsum_, d_ovf_, st_);
    return xs_;
  };
  // (the f32 output is written only when a consumer may fall back to it). A split-K partial left
  // in tmp_ by the preceding projection is added into x_ by the norm itself.
  auto norm_split = [&](const DevTensor& w, bool need_f32, bool pend) -> const __half* {
    if (!wide || H_ % 32 != 0) {
      if (pend) launch_add_f32(x_, tmp_, (size_t)M * H_, st_);
      launch_rmsnorm(x_, (const float*)w.dev, M, H_, eps, xn_, st_);
      return nullptr;
    }
    launch_rmsnorm_split(x_, (const float*)w.dev, M, H_, eps, need_f32 ? xn_ : nullptr, xs_, xs_ + (size_t)M * H_,
                         xsum_, d_ovf_, st_, pend ? tmp_ : nullptr);
    return xs_;
  };
  const DevTensor* wqkv[3] = {&L.wq, &L.wk, &L.wv};
  const bool qkv_q = quant_ready(wqkv, 3, M, H_) || (quant_ready(wqkv, 2, M, H_) && quant_ready(wqkv + 2, 1, M, H_));
  const __half* xs = norm_split(L.attn_norm, !qkv_q, pend_in);
  {
    const DevTensor* ws[3] = {&L.wq, &L.wk, &L.wv};
    float* outs[3] = {q_, k_, v_};
    if (!xs || !project_q(ws, outs, 3, M, H_, nullptr)) {
      // Q and K share a launch when only V differs (a Q6_K attn_v in a Q4_K_M file)
      if (!xs || !project_q(ws, outs, 2, M, H_, nullptr)) {
        project(L.wq, xn_, xs, M, H_, qd, q_, nullptr, st_, f32);
        project(L.wk, xn_, xs, M, H_, kvd, k_, nullptr, st_, f32);
      }
      if (!xs || !project_q(ws + 2, outs + 2, 1, M, H_, nullptr))
        project(L.wv, xn_, xs, M, H_, kvd, v_, nullptr, st_, f32);
    }
  }
  if (c.unpack_qk) {
    launch_unpack_qk(q_, tmp_, M, qd, c.n_heads, hd, st_);
    launch_copy_f32(tmp_, q_, (size_t)M * qd, st_);
    launch_unpack_qk(k_, tmp_, M, kvd, c.n_kv_heads, hd, st_);
    launch_copy_f32(tmp_, k_, (size_t)M * kvd, st_);
  }
  const RopeTable& rt = m_->rope_tables[L.rope_table];
  // xs_ (the GEMM input pair, consumed by the Q/K/V projection above) is free until the O
  // projection's split: the shared-K/V attention stages its fp16 K / V planes there. RoPE, the KV
  // append and those planes go in one launch when that path applies.
  const bool prepped = !f32 && qd == c.n_heads * hd && kvd == c.n_kv_heads * hd &&
                       launch_attn_prefill_prep(q_, k_, v_, M, c.n_heads, c.n_kv_heads, hd, rt.dev, S.rotary_dim / 2,
                                                kc_[li], vc_[li], kv_f32_, ctx_, pos_, xs_, xs_halves(), d_ovf_, st_);
  if (!prepped) {
    launch_rope_rows(q_, M, qd, c.n_heads, hd, 0, rt.dev, S.rotary_dim / 2, st_);
    launch_rope_rows(k_, M, kvd, c.n_kv_heads, hd, 0, rt.dev, S.rotary_dim / 2, st_);
    launch_kv_store(k_, v_, M, kvd, kc_[li], vc_[li], kv_f32_, c.n_kv_heads, hd, ctx_, nullptr, pos_, st_);
  }
  const float scale = 1.0f / sqrtf((float)hd);
  if (f32)
    launch_attn_prefill_f32(q_, k_, v_, att_, M, c.n_heads, c.n_kv_heads, hd, S.window, scale, st_);
  else
    launch_attn_prefill(q_, k_, v_, att_, M, c.n_heads, c.n_kv_heads, hd, S.window, scale, st_, xs_, xs_halves(),
                        prepped, d_ovf_);
  bool opend = false;
  {
    const __half* xa = split(att_, qd);
    const DevTensor* ws[1] = {&L.wo};
    float* outs[1] = {x_};
    if (!xa || !project_q(ws, outs, 1, M, qd, x_, kpart_ok_ ? tmp_ : nullptr, &opend))
      project(L.wo, att_, xa, M, qd, H_, x_, x_, st_, f32);
  }
  // FFN sub-layer: pre-norm, gate/up, SwiGLU, down + residual.
  const DevTensor* wgu[2] = {&L.gate, &L.up};
  xs = norm_split(L.ffn_norm, M == 1 || !quant_ready(wgu, 2, M, H_), opend);
  const __half* xa = nullptr;
  const float* xa_sums = nullptr;  // per-32 sums of the down projection's input (default xsum_)
  const bool glu = xs && gate_up_glu(li, M);
  if (glu) {
    xa = reinterpret_cast<const __half*>(g_);
    xa_sums = u_;
    // act is in xa / xa_sums
  } else if (M == 1 && L.gate.dtype == L.up.dtype) {
    MvSegDesc s[2] = {{L.gate.dev, act_, nullptr, S.ffn_dim}, {L.up.dev, nullptr, nullptr, S.ffn_dim}};
    launch_matvec(L.gate.dtype, s, 2, xn_, H_, 2, st_);
  } else {
    const DevTensor* ws[2] = {&L.gate, &L.up};
    float* outs[2] = {g_, u_};
    if (!xs || !project_q(ws, outs, 2, M, H_, nullptr)) {
      project(L.gate, xn_, xs, M, H_, S.ffn_dim, g_, nullptr, st_, f32);
      project(L.up, xn_, xs, M, H_, S.ffn_dim, u_, nullptr, st_, f32);
    }
    if (wide && S.ffn_dim % 32 == 0) {
      const DevTensor* wd[1] = {&L.down};
      launch_swiglu_split(g_, u_, quant_ready(wd, 1, M, S.ffn_dim) ? nullptr : act_, M, S.ffn_dim, xs_,
                          xs_ + (size_t)M * S.ffn_dim, xsum_, d_ovf_, st_);
      xa = xs_;
    } else {
      launch_swiglu(g_, u_, act_, (size_t)M * S.ffn_dim, st_);
    }
  }
  bool dpend = false;
  {
    const DevTensor* ws[1] = {&L.down};
    float* outs[1] = {x_};
    if (!xa || !project_q(ws, outs, 1, M, S.ffn_dim, x_, kpart_ok_ ? tmp_ : nullptr, &dpend, xa, xa_sums))
      project(L.down, act_, xa, M, S.ffn_dim, H_, x_, x_, st_, f32);
  }
  return dpend;
}

// Decode layer, fused path: 5 launches (QKV+norm+RoPE+KV append, attention, O+residual,
// gate/up+norm+SwiGLU, down+residual). Conditions: no Q/K un-permute, same K-quant dtype for
// Q/K/V and for gate/up, K a multiple of 256.
bool Session::fused_ok(int li) const {
  const Config& c = m_->cfg;
  const LayerTensors& L = m_->layers[li];
  auto kq = [](int dt) { return dt == DT_Q4K || dt == DT_Q6K; };
  return !c.unpack_qk && L.wq.dtype == L.wk.dtype && L.wq.dtype == L.wv.dtype && kq(L.wq.dtype) &&
         L.gate.dtype == L.up.dtype && kq(L.gate.dtype) && H_ % 256 == 0 && c.layers[li].head_dim % 2 == 0;
}

// Launch arguments of the fused decode path's four matvecs of layer li (QKV with RMSNorm, RoPE and
// the KV append; O + residual; gate/up with RMSNorm and SwiGLU; down + residual) and their
// weight layouts.
void Session::decode_args(int li, MvArgs& a, MvArgs& o, MvArgs& f, MvArgs& dn, int* dts) {
  const Config& c = m_->cfg;
  const LayerSpec& S = c.layers[li];
  const LayerTensors& L = m_->layers[li];
  const int hd = S.head_dim, qd = S.q_dim, kvd = S.kv_dim;
  const RopeTable& rt = m_->rope_tables[L.rope_table];
  a = MvArgs{};
  a.nseg = 3;
  a.w[0] = (const uint8_t*)L.wq.dev;
  a.w[1] = (const uint8_t*)L.wk.dev;
  a.w[2] = (const uint8_t*)L.wv.dev;
  a.out[0] = qd_;
  a.n[0] = qd;
  a.n[1] = kvd;
  a.n[2] = kvd;
  a.x = xdec_;
  a.norm_w = (const float*)L.attn_norm.dev;
  a.eps = c.rms_eps;
  a.K = H_;
  a.epi = EPI_QKV;
  a.rope_cs = rt.dev;
  a.npairs = S.rotary_dim / 2;
  a.head_dim = hd;
  a.ctx = ctx_;
  a.pos = d_pos_;
  a.kc = kc_[li];
  a.vc = vc_[li];
  a.kv_f32 = kv_f32_ ? 1 : 0;
  dts[0] = L.wq.dtype;
  o = MvArgs{};
  o.nseg = 1;
  o.w[0] = (const uint8_t*)L.wo.dev;
  o.out[0] = xdec_;
  o.n[0] = H_;
  o.x = attd_;
  o.K = qd;
  o.epi = EPI_RESID;
  o.resid = xdec_;
  dts[1] = L.wo.dtype;
  f = MvArgs{};
  f.nseg = 2;
  f.w[0] = (const uint8_t*)L.gate.dev;
  f.w[1] = (const uint8_t*)L.up.dev;
  f.out[0] = actd_;
  f.n[0] = S.ffn_dim;
  f.n[1] = S.ffn_dim;
  f.x = xdec_;
  f.norm_w = (const float*)L.ffn_norm.dev;
  f.eps = c.rms_eps;
  f.K = H_;
  f.epi = EPI_SWIGLU;
  dts[2] = L.gate.dtype;
  dn = MvArgs{};
  dn.nseg = 1;
  int down_dt = L.down.dtype;
  dn.w[0] = (const uint8_t*)mv_weight(L.down, S.ffn_dim, &down_dt);
  dn.out[0] = xdec_;
  dn.n[0] = H_;
  dn.x = actd_;
  dn.K = S.ffn_dim;
  dn.epi = EPI_RESID;
  dn.resid = xdec_;
  dts[3] = down_dt;
}

void Session::layer_decode(int li, bool last) {
  const Config& c = m_->cfg;
  const LayerSpec& S = c.layers[li];
  const int hd = S.head_dim;
  const float scale = 1.0f / sqrtf((float)hd);
  if (!fused_ok(li)) {
    layer_decode_unfused(li);
    if (last) launch_add_int(d_pos_, 1, st_);
    return;
  }
  MvArgs a, o, f, dn;
  int dts[4];
  decode_args(li, a, o, f, dn, dts);
  launch_mv(dts[0], a, st_);
  launch_attn_decode(qd_, kc_[li], vc_[li], kv_f32_, attd_, part_, d_cnt_, c.n_heads, c.n_kv_heads, hd, ctx_, d_pos_,
                     S.window, scale, ctx_, st_);
  launch_mv(dts[1], o, st_);
  launch_mv(dts[2], f, st_);
  dn.pos_inc = last ? d_pos_ : nullptr;
  launch_mv(dts[3], dn, st_);
}

static size_t embedding_hidden(const DevTensor& t, size_t* vocab) {
  // lookup_embedding_rows (embeddings.rs:108-116): hidden = the smaller dim.
  if (t.dims.size() != 2) fail(ST_TENSOR, "expected 2D embedding tensor");
  size_t h = std::min(t.dims[0], t.dims[1]);
  *vocab = std::max(t.dims[0], t.dims[1]);
  return h;
}

// Decode chain path (Mistral/Llama family): the decode step as 2 launches per layer, each chain
// launch running the O projection, gate/up, down and the next layer's Q/K/V as phases of one
// persistent kernel (kernels/chain.hip), the attention in between. Taken when every layer is on
// the fused path with Q4_K Q/K/V, O, gate/up, a Q4_K or regrouped Q6_K down projection and LM head,
// and widths the chain kernel supports; otherwise decode runs the per-launch kernels.
void Session::prepare_chain() {
  const Config& c = m_->cfg;
  // the Q/K/V epilogue appends f32 K and V rows (an fp16 cache would take another epilogue)
  if (gemma_ || c.n_layers <= 0 || c.unpack_qk || !kv_f32_) return;
  const int G = num_cus();
  auto wdt = [](const DevTensor& t, int* dt) -> const uint8_t* {
    if (t.dev_r && t.dtype_r == DT_Q6K_R) {
      *dt = DT_Q6K_R;
      return (const uint8_t*)t.dev_r;
    }
    *dt = t.dtype;
    return (const uint8_t*)t.dev;
  };
  auto dims_ok = [](const DevTensor& t, int K, int N) {
    return t.dims.size() == 2 && (int)t.dims[0] == K && (int)t.dims[1] == N && N % 2 == 0;
  };
  auto phase_ok = [&](int dt, int K, bool norm, int units) {
    if (!chain_phase_ok(dt, K, norm)) return false;
    const int npass = (K + 4095) / 4096;
    return (long long)units * G < (1ll << 31) && ((units + G - 1) / G) * 2 * npass <= 512;
  };
  for (int li = 0; li < c.n_layers; ++li) {
    const LayerSpec& S = c.layers[li];
    const LayerTensors& L = m_->layers[li];
    int dq, dk, dv, dd;
    wdt(L.wq, &dq);
    wdt(L.wk, &dk);
    wdt(L.wv, &dv);
    wdt(L.down, &dd);
    // Q4_K_M files give some layers a Q6_K attn_v: that layer's V rows run as a phase of their own
    if (c.unpack_qk || H_ % 256 != 0 || dq != DT_Q4K || dk != DT_Q4K || (dv != DT_Q4K && dv != DT_Q6K_R) ||
        L.wo.dtype != DT_Q4K || L.gate.dtype != DT_Q4K || L.up.dtype != DT_Q4K || (dd != DT_Q4K && dd != DT_Q6K_R))
      return;
    if (!dims_ok(L.wq, H_, S.q_dim) || !dims_ok(L.wk, H_, S.kv_dim) || !dims_ok(L.wv, H_, S.kv_dim) ||
        !dims_ok(L.wo, S.q_dim, H_) || !dims_ok(L.gate, H_, S.ffn_dim) || !dims_ok(L.up, H_, S.ffn_dim) ||
        !dims_ok(L.down, S.ffn_dim, H_) || S.head_dim % 2 != 0 || S.rotary_dim > S.head_dim)
      return;
    const bool split_v = dv != DT_Q4K;
    if (!phase_ok(DT_Q4K, H_, true, (S.q_dim + (split_v ? 1 : 2) * S.kv_dim) / 2) ||
        (split_v && !phase_ok(dv, H_, true, S.kv_dim / 2)) || !phase_ok(DT_Q4K, S.q_dim, false, H_ / 2) ||
        !phase_ok(DT_Q4K, H_, true, S.ffn_dim) || !phase_ok(dd, S.ffn_dim, false, H_ / 2))
      return;
  }
  int dh;
  const uint8_t* head_w = wdt(m_->lm_head, &dh);
  if ((dh != DT_Q4K && dh != DT_Q6K_R) || !dims_ok(m_->lm_head, H_, c.vocab) || !phase_ok(dh, H_, true, c.vocab / 2))
    return;
  size_t vocab;
  embedding_hidden(m_->token_embd, &vocab);
  chain_embed_ = m_->token_embd.dtype == DT_Q4K && H_ % 256 == 0 && c.embed_scale == 1.0f;
  auto base = [&](int dt, int K, int epi, int units, const float* x, const float* norm, int wait_prev) {
    ChainPhase P{};
    P.dt = dt;
    P.K = K;
    P.npass = (K + 4095) / 4096;
    P.epi = epi;
    P.units = units;
    P.x = x;
    P.norm_w = norm;
    P.eps = c.rms_eps;
    P.wait_prev = wait_prev;
    P.x_mode = CX_F32;
    return P;
  };
  // Q/K/V of layer li with RMSNorm, RoPE and the KV append: one phase, or a Q/K phase and a V phase
  // when V's rows are another dtype (the V phase needs no barrier: its input is the Q/K phase's)
  auto qkv = [&](int li, int wait_prev, bool embed, std::vector<ChainPhase>& v) {
    const LayerSpec& S = c.layers[li];
    const LayerTensors& L = m_->layers[li];
    int dv;
    const uint8_t* wv = wdt(L.wv, &dv);
    const bool split_v = dv != DT_Q4K;
    ChainPhase P = base(DT_Q4K, H_, CE_QKV, (S.q_dim + (split_v ? 1 : 2) * S.kv_dim) / 2, xdec_,
                        (const float*)L.attn_norm.dev, wait_prev);
    P.nseg = split_v ? 2 : 3;
    P.seg[0] = ChainSeg{(const uint8_t*)L.wq.dev, qd_, S.q_dim, 0};
    P.seg[1] = ChainSeg{(const uint8_t*)L.wk.dev, nullptr, S.kv_dim, 0};
    if (!split_v) P.seg[2] = ChainSeg{wv, nullptr, S.kv_dim, 0};
    P.rope_cs = m_->rope_tables[L.rope_table].dev;
    P.npairs = S.rotary_dim / 2;
    P.head_dim = S.head_dim;
    P.ctx = ctx_;
    P.kc = (float*)kc_[li];
    P.vc = (float*)vc_[li];
    if (embed) {
      P.x_mode = CX_EMBED_Q4K;
      P.emb = (const uint8_t*)m_->token_embd.dev;
      P.emb_out = xdec_;
      P.emb_rows = (int)vocab;
    }
    v.push_back(P);
    if (split_v) {
      ChainPhase V = P;
      V.dt = dv;
      V.units = S.kv_dim / 2;
      V.nseg = 1;
      V.seg[0] = ChainSeg{wv, nullptr, S.kv_dim, 0};
      V.seg[1] = V.seg[2] = ChainSeg{};
      V.role0 = 2;
      V.wait_prev = 0;
      v.push_back(V);
    }
  };
  auto ffn = [&](int li, std::vector<ChainPhase>& v) {
    const LayerSpec& S = c.layers[li];
    const LayerTensors& L = m_->layers[li];
    ChainPhase o = base(DT_Q4K, S.q_dim, CE_RESID, H_ / 2, attd_, nullptr, 0);
    o.nseg = 1;
    o.seg[0] = ChainSeg{(const uint8_t*)L.wo.dev, xdec_, H_, 0};
    o.resid = xdec_;
    v.push_back(o);
    ChainPhase g = base(DT_Q4K, H_, CE_SWIGLU, S.ffn_dim, xdec_, (const float*)L.ffn_norm.dev, 1);
    g.nseg = 2;
    g.seg[0] = ChainSeg{(const uint8_t*)L.gate.dev, actd_, S.ffn_dim, 0};
    g.seg[1] = ChainSeg{(const uint8_t*)L.up.dev, nullptr, S.ffn_dim, 0};
    v.push_back(g);
    int dd;
    const uint8_t* dw = wdt(L.down, &dd);
    ChainPhase d = base(dd, S.ffn_dim, CE_RESID, H_ / 2, actd_, nullptr, 1);
    d.nseg = 1;
    d.seg[0] = ChainSeg{dw, xdec_, H_, 0};
    d.resid = xdec_;
    v.push_back(d);
  };
  std::vector<std::vector<ChainPhase>> launches(1);
  qkv(0, 0, chain_embed_, launches[0]);
  for (int li = 0; li < c.n_layers; ++li) {
    std::vector<ChainPhase> v;
    ffn(li, v);
    if (li + 1 < c.n_layers) qkv(li + 1, 1, false, v);
    launches.push_back(v);
  }
  {
    std::vector<ChainPhase> v = launches.back();
    ChainPhase h = base(dh, H_, CE_ARGMAX, c.vocab / 2, xdec_, (const float*)m_->output_norm.dev, 1);
    h.nseg = 1;
    h.seg[0] = ChainSeg{head_w, logits_, c.vocab, 0};
    h.softcap = c.has_softcap ? c.softcap : 0.f;
    v.push_back(h);
    launches.push_back(v);
  }
  // The tiled chain (launch_chain2): per phase, the phase whose output is its x, whether a later
  // phase reads its output, and per superblock of x how many workgroups write part of it. It is
  // taken only when IEK_CHAIN=2 asks for it and every phase fits it; the row-item chain
  // (launch_chain) is the default, measured faster at C2 (57.6 against 67-71 us per launch).
  const char* ev = getenv("IEK_CHAIN");
  chain2_ = ev && ev[0] == '2';
  auto out_range = [&](const ChainPhase& P, int b, int* lo, int* hi) {
    const long long u0 = (long long)P.units * b / G, u1 = (long long)P.units * (b + 1) / G;
    *lo = (int)(P.epi == CE_SWIGLU ? u0 : 2 * u0);
    *hi = (int)(P.epi == CE_SWIGLU ? u1 : 2 * u1);
  };
  for (auto& v : launches) {
    for (size_t i = 0; i < v.size(); ++i) {
      ChainPhase& P = v[i];
      P.x_src = -1;
      P.arrive = 0;
      if (P.wait_prev) P.x_src = (int)i - 1;
      else if (i > 0 && P.epi == CE_QKV && P.role0 == 2) P.x_src = v[i - 1].x_src;  // the V-only phase
      const int rows = 2 * ((P.units + G - 1) / G);
      if (!chain2_phase_ok(P.dt, P.K, P.norm_w != nullptr, rows)) chain2_ = false;
    }
    for (size_t i = 0; i < v.size(); ++i) {
      ChainPhase& P = v[i];
      if (P.x_src < 0) continue;
      v[P.x_src].arrive = 1;
      const int nsb = P.K / 256;
      for (int sb = 0; sb < nsb; ++sb) P.expect[sb] = 0;
      for (int b = 0; b < G; ++b) {
        int lo, hi;
        out_range(v[P.x_src], b, &lo, &hi);
        if (hi <= lo) continue;
        if (hi > P.K) chain2_ = false;  // the producer's output is wider than this phase's x
        for (int sb = lo / 256; sb <= (hi - 1) / 256 && sb < nsb; ++sb) ++P.expect[sb];
      }
    }
  }
  size_t total = 0;
  for (auto& v : launches) total += v.size();
  std::vector<ChainPhase> host;
  host.reserve(total);
  for (auto& v : launches) host.insert(host.end(), v.begin(), v.end());
  IEK_HIP(hipMalloc(&chain_blob_, total * sizeof(ChainPhase)));
  IEK_HIP(hipMemcpy(chain_blob_, host.data(), total * sizeof(ChainPhase), hipMemcpyHostToDevice));
  size_t off = 0;
  for (auto& v : launches) {
    chain_ph_.push_back(static_cast<const char*>(chain_blob_) + off * sizeof(ChainPhase));
    chain_np_.push_back((int)v.size());
    off += v.size();
  }
  d_chain_cnt_ = dev_alloc<unsigned>(chain_counter_words());
  d_chain_err_ = dev_alloc<int>(2);  // [error code, bounded-wait limit (0: default)]
  launch_fill_i32((int*)d_chain_cnt_, 0, chain_counter_words(), st_);
  launch_fill_i32(d_chain_err_, 0, 2, st_);
  chain_ = true;
}

// A bounded wait that ran out in a chain launch leaves its flag set; the counters are cleared and
// the step reports a device error (the session state is then undefined, as after any failed step).
void Session::check_chain_error() {
  if (!chain_) return;
  int err = 0;
  IEK_HIP(hipMemcpyAsync(&err, d_chain_err_, 4, hipMemcpyDeviceToHost, st_));
  sync();
  if (err) {
    launch_fill_i32((int*)d_chain_cnt_, 0, chain_counter_words(), st_);
    launch_fill_i32(d_chain_err_, 0, 1, st_);
    sync();
    fail(ST_DEVICE, "decode chain: a bounded wait ran out (code " + std::to_string(err) + ")");
  }
}

void Session::set_chain_spin(unsigned spin) {
  if (!chain_) fail(ST_OP, "set_chain_spin: the session does not decode through the chain");
  launch_set_int(d_chain_err_ + 1, (int)spin, st_);
  sync();
}

void Session::layer_decode_unfused(int li) {
  const Config& c = m_->cfg;
  const LayerSpec& S = c.layers[li];
  const LayerTensors& L = m_->layers[li];
  const int hd = S.head_dim, qd = S.q_dim, kvd = S.kv_dim;
  launch_rmsnorm(xdec_, (const float*)L.attn_norm.dev, 1, H_, c.rms_eps, xndec_, st_);
  if (L.wq.dtype == L.wk.dtype && L.wq.dtype == L.wv.dtype) {
    MvSegDesc s[3] = {{L.wq.dev, qd_, nullptr, qd}, {L.wk.dev, kd_, nullptr, kvd}, {L.wv.dev, vd_, nullptr, kvd}};
    launch_matvec(L.wq.dtype, s, 3, xndec_, H_, 0, st_);
  } else {
    project(L.wq, xndec_, nullptr, 1, H_, qd, qd_, nullptr, st_);
    project(L.wk, xndec_, nullptr, 1, H_, kvd, kd_, nullptr, st_);
    project(L.wv, xndec_, nullptr, 1, H_, kvd, vd_, nullptr, st_);
  }
  if (c.unpack_qk) {
    launch_unpack_qk(qd_, tmpd_, 1, qd, c.n_heads, hd, st_);
    launch_copy_f32(tmpd_, qd_, qd, st_);
    launch_unpack_qk(kd_, tmpd_, 1, kvd, c.n_kv_heads, hd, st_);
    launch_copy_f32(tmpd_, kd_, kvd, st_);
  }
  const RopeTable& rt = m_->rope_tables[L.rope_table];
  launch_rope_table(qd_, c.n_heads, hd, S.rotary_dim / 2, rt.dev, d_pos_, st_);
  launch_rope_table(kd_, c.n_kv_heads, hd, S.rotary_dim / 2, rt.dev, d_pos_, st_);
  launch_kv_store(kd_, vd_, 1, kvd, kc_[li], vc_[li], kv_f32_, c.n_kv_heads, hd, ctx_, d_pos_, 0, st_);
  const float scale = 1.0f / sqrtf((float)hd);
  launch_attn_decode(qd_, kc_[li], vc_[li], kv_f32_, attd_, part_, d_cnt_, c.n_heads, c.n_kv_heads, hd, ctx_, d_pos_, S.window,
                     scale, ctx_, st_);
  project(L.wo, attd_, nullptr, 1, qd, H_, xdec_, xdec_, st_);
  launch_rmsnorm(xdec_, (const float*)L.ffn_norm.dev, 1, H_, c.rms_eps, xndec_, st_);
  if (L.gate.dtype == L.up.dtype) {
    MvSegDesc s[2] = {{L.gate.dev, actd_, nullptr, S.ffn_dim}, {L.up.dev, nullptr, nullptr, S.ffn_dim}};
    launch_matvec(L.gate.dtype, s, 2, xndec_, H_, 2, st_);
  } else {
    project(L.gate, xndec_, nullptr, 1, H_, S.ffn_dim, tmpd_, nullptr, st_);
    project(L.up, xndec_, nullptr, 1, H_, S.ffn_dim, actd_, nullptr, st_);
    launch_swiglu(tmpd_, actd_, actd_, S.ffn_dim, st_);
  }
  project(L.down, actd_, nullptr, 1, S.ffn_dim, H_, xdec_, xdec_, st_);
}

// ---- Gemma-4 family ---------------------------------------------------------------------------

// fp16 (hi, lo) pair and per-32 sums of a GEMM input, when it has more than one row and a width
// the split takes; null otherwise.
const __half* Session::split_rows(const float* a, int M, int K) {
  if (M < 2 || K % 32 != 0 || f32_prefill_) return nullptr;
  launch_split_sums(a, M, K, xs_, xs_ + (size_t)M * K, xsum_, d_ovf_, st_);
  return xs_;
}

// Per-layer embedding inputs for n token rows (compute_packed_per_layer_inputs,
// gemma4_ple.rs:27-109): model projection of the scaled embeddings `x`, per-layer RMSNorm, plus
// the per-layer token rows scaled by sqrt(pd), times 1/sqrt(2).
void Session::embed_ple(const uint32_t* d_ids, int n, const float* x, const __half* xs, float* tok, float* proj,
                        float* pack) {
  const Config& c = m_->cfg;
  if (c.ple_dim <= 0) return;
  const int packn = c.n_layers * c.ple_dim;
  size_t vocab;
  const DevTensor& te = m_->ple_token_embd;
  if (te.dims.size() != 2) fail(ST_TENSOR, "expected 2D embedding tensor");
  const size_t row = std::min(te.dims[0], te.dims[1]);
  vocab = std::max(te.dims[0], te.dims[1]);
  if ((int)row != packn) fail(ST_MODEL, "per_layer_token_embd row width != n_layers*ple_dim");
  if (m_->ple_proj_norm.host_f32.size() != (size_t)c.ple_dim)
    fail(ST_MODEL, "per_layer_proj_norm len != ple_dim");
  launch_embed(te.dtype, te.dev, row, vocab, d_ids, n, 1.0f, tok, st_);
  project(m_->ple_model_proj, x, xs, n, H_, packn, proj, nullptr, st_, f32_prefill_);
  launch_ple_pack(proj, tok, (const float*)m_->ple_proj_norm.dev, n, c.n_layers, c.ple_dim, c.rms_eps,
                  c.ple_proj_scale, sqrtf((float)c.ple_dim), c.ple_combine_scale, pack, st_);
}

// prefill_layer_block for Gemma-4 (block.rs:12-47): attention with q/k head norms, v norm,
// optional KV borrowing and sliding window, scale 1 (attention.rs:175-422), post-attention norm +
// residual; GeGLU FFN with post-FFN norm + residual (ffn.rs:120-167); PLE tail (ffn.rs:170-240)
// and the layer output scale (ffn.rs:242-278), folded into the last residual update.
void Session::layer_prefill_gemma(int li, int M) {
  const Config& c = m_->cfg;
  const LayerSpec& S = c.layers[li];
  const LayerTensors& L = m_->layers[li];
  const int hd = S.head_dim, qd = S.q_dim, kvd = S.kv_dim;
  const float eps = c.rms_eps;
  const bool borrow = S.kv_borrow >= 0;
  if (borrow && pos_ != 0) fail(ST_MODEL, "prefill attention: borrow source cache len mismatch");
  if (!L.attn_post_norm.present()) fail(ST_MODEL, "Gemma 4: missing post_attention_norm");
  if (!L.ffn_post_norm.present()) fail(ST_MODEL, "Gemma 4: missing post_ffw_norm");
  launch_rmsnorm(x_, (const float*)L.attn_norm.dev, M, H_, eps, xn_, st_);
  const __half* xs = split_rows(xn_, M, H_);
  {
    const DevTensor* ws[3] = {&L.wq, &L.wk, &L.wv};
    float* outs[3] = {q_, k_, v_};
    if (!xs || !project_q(ws, outs, borrow ? 1 : 3, M, H_, nullptr)) {
      project(L.wq, xn_, xs, M, H_, qd, q_, nullptr, st_, f32_prefill_);
      if (!borrow) {
        project(L.wk, xn_, xs, M, H_, kvd, k_, nullptr, st_, f32_prefill_);
        project(L.wv, xn_, xs, M, H_, kvd, v_, nullptr, st_, f32_prefill_);
      }
    }
  }
  const RopeTable& rt = m_->rope_tables[L.rope_table];
  launch_head_prep(q_, k_, v_, M, qd, kvd, c.n_heads, borrow ? 0 : c.n_kv_heads, hd,
                   L.q_norm.present() ? (const float*)L.q_norm.dev : nullptr,
                   L.k_norm.present() ? (const float*)L.k_norm.dev : nullptr, eps, true, rt.dev, S.rotary_dim / 2,
                   nullptr, 0, pos_, borrow ? nullptr : kc_[li], borrow ? nullptr : vc_[li], kv_f32_, ctx_, st_);
  if (borrow) launch_kv_load(kc_[li], vc_[li], kv_f32_, M, c.n_kv_heads, hd, ctx_, k_, v_, st_);
  if (f32_prefill_)
    launch_attn_prefill_f32(q_, k_, v_, att_, M, c.n_heads, c.n_kv_heads, hd, S.window, 1.0f, st_);
  else
    launch_attn_prefill(q_, k_, v_, att_, M, c.n_heads, c.n_kv_heads, hd, S.window, 1.0f, st_, xs_, xs_halves(), false,
                        d_ovf_);  // xs_ (the Q/K/V input pair, consumed) holds the K / V^T planes
  {
    const __half* xa = split_rows(att_, M, qd);
    const DevTensor* ws[1] = {&L.wo};
    float* outs[1] = {tmp_};
    if (!xa || !project_q(ws, outs, 1, M, qd, nullptr))
      project(L.wo, att_, xa, M, qd, H_, tmp_, nullptr, st_, f32_prefill_);
  }
  launch_rmsnorm_add(x_, tmp_, (const float*)L.attn_post_norm.dev, M, H_, eps, false, 1.f, st_);
  launch_rmsnorm(x_, (const float*)L.ffn_norm.dev, M, H_, eps, xn_, st_);
  xs = split_rows(xn_, M, H_);
  {
    const DevTensor* ws[2] = {&L.gate, &L.up};
    float* outs[2] = {g_, u_};
    if (!xs || !project_q(ws, outs, 2, M, H_, nullptr)) {
      project(L.gate, xn_, xs, M, H_, S.ffn_dim, g_, nullptr, st_, f32_prefill_);
      project(L.up, xn_, xs, M, H_, S.ffn_dim, u_, nullptr, st_, f32_prefill_);
    }
  }
  launch_gelu_mul(g_, u_, act_, (size_t)M * S.ffn_dim, st_);
  {
    const __half* xa = split_rows(act_, M, S.ffn_dim);
    const DevTensor* ws[1] = {&L.down};
    float* outs[1] = {tmp_};
    if (!xa || !project_q(ws, outs, 1, M, S.ffn_dim, nullptr))
      project(L.down, act_, xa, M, S.ffn_dim, H_, tmp_, nullptr, st_, f32_prefill_);
  }
  const bool ple = c.ple_dim > 0;
  launch_rmsnorm_add(x_, tmp_, (const float*)L.ffn_post_norm.dev, M, H_, eps, !ple && L.has_out_scale,
                     L.out_scale_value, st_);
  if (ple) {
    const int pd = c.ple_dim;
    if (!L.ple_gate.present() || !L.ple_proj.present() || !L.ple_post_norm.present())
      fail(ST_MODEL, "PLE: missing inp_gate / proj / post_norm");
    xs = split_rows(x_, M, H_);
    project(L.ple_gate, x_, xs, M, H_, pd, g_, nullptr, st_, f32_prefill_);
    launch_ple_gate(g_, ple_pack_, M, pd, c.n_layers, li, st_);
    const __half* xg = split_rows(g_, M, pd);
    project(L.ple_proj, g_, xg, M, pd, H_, tmp_, nullptr, st_, f32_prefill_);
    launch_rmsnorm_add(x_, tmp_, (const float*)L.ple_post_norm.dev, M, H_, eps, L.has_out_scale, L.out_scale_value,
                       st_);
  }
}

// One decode-step matvec over up to three weights sharing x (optionally RMS-normalised on the
// way in). Uses the regrouped copies when every weight has one of the same layout.
static void mv_multi(const DevTensor* const* ws, float* const* outs, int nseg, const float* x, int K,
                     const float* norm_w, float eps, int epi, hipStream_t st, const ResidUpdate* pre = nullptr,
                     float* pre_out = nullptr, const float* mulv = nullptr) {
  int dt0 = -1;
  const void* wp[3];
  bool same = true;
  for (int i = 0; i < nseg; ++i) {
    const DevTensor& w = *ws[i];
    if (w.dims.size() != 2 || (int)w.dims[0] != K)
      fail(ST_MATMUL, "inner dim mismatch: weight dims do not match the activation width");
    int dt;
    wp[i] = mv_weight(w, K, &dt);
    if (dt0 >= 0 && dt != dt0) same = false;
    dt0 = dt;
  }
  if (!same) {  // mixed layouts: native blocks, one launch per weight
    for (int i = 0; i < nseg; ++i) {
      const DevTensor* one[1] = {ws[i]};
      DevTensor native = *ws[i];
      native.dev_r = nullptr;
      one[0] = &native;
      float* o[1] = {outs[i]};
      mv_multi(one, o, 1, x, K, norm_w, eps, epi, st, pre, pre_out, mulv);
    }
    return;
  }
  MvArgs a{};
  a.nseg = nseg;
  for (int i = 0; i < nseg; ++i) {
    a.w[i] = (const uint8_t*)wp[i];
    a.out[i] = outs[i];
    a.n[i] = (int)ws[i]->dims[1];
  }
  a.x = x;
  a.norm_w = norm_w;
  a.eps = eps;
  a.K = K;
  a.epi = epi;
  a.mulv = mulv;
  if (pre && pre->t) {
    a.pre_t = pre->t;
    a.pre_w = pre->w;
    a.pre_out = pre_out;
    a.pre_scale = pre->scale;
    a.pre_has_scale = pre->has_scale ? 1 : 0;
  }
  launch_mv(dt0, a, st);
}

// decode_layer_block for Gemma-4 (block.rs:50-89), same sub-steps as layer_prefill_gemma for one
// token at the device position (*d_pos_). Each post-norm residual update
//   x <- (x + rmsnorm(t, w)) [* layer scale]
// is carried into the staging of the next matvec that reads x (`pend` -> the launch's pre-op),
// which writes the updated x to the other of the two residual buffers; `xr` tracks which one holds
// the current residual.
void Session::layer_decode_gemma(int li, float*& xr, ResidUpdate& pend) {
  const Config& c = m_->cfg;
  const LayerSpec& S = c.layers[li];
  const LayerTensors& L = m_->layers[li];
  const int hd = S.head_dim, qd = S.q_dim, kvd = S.kv_dim;
  const float eps = c.rms_eps;
  const bool borrow = S.kv_borrow >= 0;
  if (!L.attn_post_norm.present()) fail(ST_MODEL, "Gemma 4: missing post_attention_norm");
  if (!L.ffn_post_norm.present()) fail(ST_MODEL, "Gemma 4: missing post_ffw_norm");
  auto other = [&]() { return xr == xdec_ ? xdec2_ : xdec_; };
  // matvec over the current residual, applying the pending update first (then it is current)
  auto mv_x = [&](const DevTensor* const* ws, float* const* outs, int nseg, const float* norm_w, int epi,
                  const float* mulv) {
    if (pend.t) {
      float* nx = other();
      mv_multi(ws, outs, nseg, xr, H_, norm_w, eps, epi, st_, &pend, nx, mulv);
      xr = nx;
      pend = ResidUpdate{};
    } else {
      mv_multi(ws, outs, nseg, xr, H_, norm_w, eps, epi, st_, nullptr, nullptr, mulv);
    }
  };
  {
    const DevTensor* ws[3] = {&L.wq, &L.wk, &L.wv};
    float* outs[3] = {qd_, kd_, vd_};
    mv_x(ws, outs, borrow ? 1 : 3, (const float*)L.attn_norm.dev, EPI_STORE, nullptr);
  }
  const RopeTable& rt = m_->rope_tables[L.rope_table];
  launch_head_prep(qd_, kd_, vd_, 1, qd, kvd, c.n_heads, borrow ? 0 : c.n_kv_heads, hd,
                   L.q_norm.present() ? (const float*)L.q_norm.dev : nullptr,
                   L.k_norm.present() ? (const float*)L.k_norm.dev : nullptr, eps, true, rt.dev, S.rotary_dim / 2,
                   d_pos_, 0, 0, borrow ? nullptr : kc_[li], borrow ? nullptr : vc_[li], kv_f32_, ctx_, st_);
  launch_attn_decode(qd_, kc_[li], vc_[li], kv_f32_, attd_, part_, d_cnt_, c.n_heads, c.n_kv_heads, hd, ctx_, d_pos_,
                     S.window, 1.0f, ctx_, st_);
  {
    const DevTensor* ws[1] = {&L.wo};
    float* outs[1] = {tmpd_};
    mv_multi(ws, outs, 1, attd_, qd, nullptr, eps, EPI_STORE, st_);
  }
  pend = ResidUpdate{tmpd_, (const float*)L.attn_post_norm.dev, false, 1.f};
  {
    const DevTensor* ws[2] = {&L.gate, &L.up};
    float* outs[2] = {actd_, nullptr};
    mv_x(ws, outs, 2, (const float*)L.ffn_norm.dev, EPI_GEGLU, nullptr);
  }
  {
    const DevTensor* ws[1] = {&L.down};
    float* outs[1] = {tmpd_};
    mv_multi(ws, outs, 1, actd_, S.ffn_dim, nullptr, eps, EPI_STORE, st_);
  }
  const bool ple = c.ple_dim > 0;
  pend = ResidUpdate{tmpd_, (const float*)L.ffn_post_norm.dev, !ple && L.has_out_scale, L.out_scale_value};
  if (ple) {
    const int pd = c.ple_dim;
    if (!L.ple_gate.present() || !L.ple_proj.present() || !L.ple_post_norm.present())
      fail(ST_MODEL, "PLE: missing inp_gate / proj / post_norm");
    {
      // gelu_tanh(x . inp_gate) * this layer's per-layer input (ffn.rs:196-205) in the epilogue
      const DevTensor* ws[1] = {&L.ple_gate};
      float* outs[1] = {actd_};
      mv_x(ws, outs, 1, nullptr, EPI_GELU_MUL, ple_packd_ + (size_t)li * pd);
    }
    {
      const DevTensor* ws[1] = {&L.ple_proj};
      float* outs[1] = {tmpd_};
      mv_multi(ws, outs, 1, actd_, pd, nullptr, eps, EPI_STORE, st_);
    }
    pend = ResidUpdate{tmpd_, (const float*)L.ple_post_norm.dev, L.has_out_scale, L.out_scale_value};
  }
}


void Session::prefill(const uint32_t* ids, int n) {
  const Config& c = m_->cfg;
  // prefill_from_tokens_loaded (embed.rs:104-138) checks, then the vocabulary range check of
  // lookup_embedding_rows (embeddings.rs:118-125).
  if (n <= 0) fail(ST_MODEL, "prefill: empty token list");
  if (n > c.context_length)
    fail(ST_MODEL, "prefill: token length " + std::to_string(n) + " exceeds context length " +
                       std::to_string(c.context_length));
  size_t vocab;
  size_t hid = embedding_hidden(m_->token_embd, &vocab);
  for (int i = 0; i < n; ++i)
    if ((size_t)ids[i] >= vocab)
      fail(ST_MODEL, "token ID " + std::to_string(ids[i]) + " out of vocabulary range [0, " + std::to_string(vocab) + ")");
  if ((int)hid != H_) fail(ST_MODEL, "ForwardState: embedding dim mismatch");
  if (pos_ + n > ctx_) fail(ST_KVCACHE, "KVCache is Full: max len is " + std::to_string(ctx_) + ".");
  ensure_rows(n);
  IEK_HIP(hipMemcpyAsync(d_ids_, ids, (size_t)n * 4, hipMemcpyHostToDevice, st_));
  auto body = [&] {
    launch_embed(m_->token_embd.dtype, m_->token_embd.dev, hid, vocab, d_ids_, n, c.embed_scale, x_, st_);
    if (gemma_) {
      embed_ple(d_ids_, n, x_, split_rows(x_, n, H_), ple_tok_, ple_proj_, ple_pack_);
      for (int li = 0; li < c.n_layers; ++li) layer_prefill_gemma(li, n);
    } else {
      bool pend = false;  // the down projection's split-K partial goes into the next layer's norm
      for (int li = 0; li < c.n_layers; ++li) pend = layer_prefill(li, n, pend);
      if (pend) launch_add_f32(x_, tmp_, (size_t)n * H_, st_);
    }
  };
  // The matrix-core GEMMs and attention take each activation as an fp16 (hi, lo) pair. A value or
  // per-32 sum beyond the pair's range, which the reference's f32 arithmetic takes, sets d_ovf_ in
  // the kernel that splits it; the prefill then runs again in the f32 mode (SIMT GEMMs and
  // attention on f32 activations). The KV rows it appends are rewritten at the same positions.
  launch_fill_i32(d_ovf_, 0, 1, st_);
  body();
  if (overflowed()) {
    f32_prefill_ = true;
    try {
      body();
    } catch (...) {
      f32_prefill_ = false;
      throw;
    }
    f32_prefill_ = false;
    ++f32_prefills_;
  }
  launch_copy_f32(x_ + (size_t)(n - 1) * H_, xdec_, H_, st_);
  pos_ += n;
  launch_set_int(d_pos_, pos_, st_);
  state_rows_ = n;
  state_prefill_ = true;
  state_ple_ = gemma_ && c.ple_dim > 0;
  layer_cursor_ = 0;
  sync();
}

double Session::bench_kernel(int which, int reps, double* work) {
  const Config& c = m_->cfg;
  if (reps <= 0) fail(ST_OP, "bench_kernel: reps must be positive");
  check_state();
  const int L = c.n_layers;
  auto wbytes = [](const DevTensor& t) { return (double)t.bytes; };
  // Launch i works on layer i % (number of layers) so that consecutive launches stream different
  // weights from HBM (one layer's weights would stay in the 256 MB last-level cache).
  std::function<void(int)> launch;
  double total = 0.0;
  int period = 0;
  if (which == 0) {
    if (!chain_ || L < 2) fail(ST_OP, "bench_kernel: the session does not decode through the chain");
    if (pos_ >= ctx_) fail(ST_KVCACHE, "KVCache is Full: max len is " + std::to_string(ctx_) + ".");
    // launch k (1 <= k < L): layer k-1's O, gate/up and down, layer k's Q/K/V
    period = L - 1;
    for (int k = 1; k < L; ++k) {
      const LayerTensors& P = m_->layers[k - 1];
      const LayerTensors& N = m_->layers[k];
      const LayerSpec& S = c.layers[k - 1];
      const LayerSpec& T = c.layers[k];
      total += wbytes(P.wo) + wbytes(P.gate) + wbytes(P.up) + wbytes(P.down) + wbytes(N.wq) + wbytes(N.wk) +
               wbytes(N.wv) + 4.0 * ((double)S.q_dim + 4.0 * H_ + 2.0 * S.ffn_dim + T.q_dim + 2.0 * T.kv_dim);
    }
    launch = [&](int i) {
      const int k = 1 + i % (L - 1);
      ChainArgs a{};
      a.phases = static_cast<const ChainPhase*>(chain_ph_[k]);
      a.nphase = chain_np_[k];
      a.pos = d_pos_;
      a.tok = d_tok_;
      a.counters = d_chain_cnt_;
      a.err = d_chain_err_;
      chain2_ ? launch_chain2(a, st_) : launch_chain(a, st_);
    };
  } else if (which == 1) {
    if (gemma_ || !state_prefill_ || state_rows_ < 2) fail(ST_OP, "bench_kernel: needs a Mistral/Llama prefill state");
    const int M = state_rows_;
    period = L;
    for (int li = 0; li < L; ++li) {
      const DevTensor* ws[2] = {&m_->layers[li].gate, &m_->layers[li].up};
      if (!quant_ready(ws, 2, M, H_)) fail(ST_OP, "bench_kernel: gate/up do not run on the K-quant GEMM");
      total += 2.0 * M * H_ * 2.0 * c.layers[li].ffn_dim;
    }
    // the gate/up projection as the prefill runs it (SwiGLU in the epilogue where it applies)
    launch = [&, M](int i) {
      const int li = i % L;
      if (gate_up_glu(li, M)) return;
      const DevTensor* w2[2] = {&m_->layers[li].gate, &m_->layers[li].up};
      float* outs[2] = {g_, u_};
      project_q(w2, outs, 2, M, H_, nullptr);
    };
  } else if (which == 2 || which == 3) {
    // 2: the down projection + residual (split K where the prefill splits it); 3: Q/K/V. The
    // input pair is whatever the GEMM input buffer holds (the timing does not depend on values).
    if (gemma_ || !state_prefill_ || state_rows_ < 2) fail(ST_OP, "bench_kernel: needs a Mistral/Llama prefill state");
    const int M = state_rows_;
    period = L;
    for (int li = 0; li < L; ++li) {
      const LayerTensors& T = m_->layers[li];
      const LayerSpec& S = c.layers[li];
      if (which == 2) {
        const DevTensor* ws[1] = {&T.down};
        if (!quant_ready(ws, 1, M, S.ffn_dim)) fail(ST_OP, "bench_kernel: down does not run on the K-quant GEMM");
        total += 2.0 * M * S.ffn_dim * H_;
      } else {
        const DevTensor* ws[3] = {&T.wq, &T.wk, &T.wv};
        if (!quant_ready(ws, 3, M, H_)) fail(ST_OP, "bench_kernel: Q/K/V do not share one K-quant GEMM");
        total += 2.0 * M * H_ * ((double)S.q_dim + 2.0 * S.kv_dim);
      }
    }
    launch = [&, M, which](int i) {
      const LayerTensors& T = m_->layers[i % L];
      if (which == 2) {
        const DevTensor* ws[1] = {&T.down};
        float* outs[1] = {x_};
        project_q(ws, outs, 1, M, c.layers[i % L].ffn_dim, x_, kpart_ok_ ? tmp_ : nullptr);
      } else {
        const DevTensor* ws[3] = {&T.wq, &T.wk, &T.wv};
        float* outs[3] = {q_, k_, v_};
        project_q(ws, outs, 3, M, H_, nullptr);
      }
    };
  } else {
    fail(ST_OP, "bench_kernel: which must be 0, 1, 2 or 3");
  }
  *work = total / period;
  hipEvent_t e0, e1;
  IEK_HIP(hipEventCreate(&e0));
  IEK_HIP(hipEventCreate(&e1));
  {
    ChainTurn turn(m_->device, st_, which == 0);
    for (int i = 0; i < 3; ++i) launch(i);
    IEK_HIP(hipEventRecord(e0, st_));
    for (int i = 0; i < reps; ++i) launch(i);
    IEK_HIP(hipEventRecord(e1, st_));
  }
  IEK_HIP(hipEventSynchronize(e1));
  float ms = 0.f;
  IEK_HIP(hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  check_chain_error();
  reset();
  sync();
  return 1e3 * (double)ms / reps;
}

// ---- forward-level steps -------------------------------------------------------------------------

void Session::embed(const uint32_t* ids, int n) {
  const Config& c = m_->cfg;
  if (n <= 0) fail(ST_MODEL, "prefill: empty token list");
  if (n > c.context_length)
    fail(ST_MODEL, "prefill: token length " + std::to_string(n) + " exceeds context length " +
                       std::to_string(c.context_length));
  size_t vocab;
  size_t hid = embedding_hidden(m_->token_embd, &vocab);
  for (int i = 0; i < n; ++i)
    if ((size_t)ids[i] >= vocab)
      fail(ST_MODEL, "token ID " + std::to_string(ids[i]) + " out of vocabulary range [0, " + std::to_string(vocab) + ")");
  if ((int)hid != H_) fail(ST_MODEL, "ForwardState: embedding dim mismatch");
  ensure_rows(n);
  IEK_HIP(hipMemcpyAsync(d_ids_, ids, (size_t)n * 4, hipMemcpyHostToDevice, st_));
  launch_embed(m_->token_embd.dtype, m_->token_embd.dev, hid, vocab, d_ids_, n, c.embed_scale, x_, st_);
  if (gemma_) {
    launch_fill_i32(d_ovf_, 0, 1, st_);
    embed_ple(d_ids_, n, x_, split_rows(x_, n, H_), ple_tok_, ple_proj_, ple_pack_);
    if (overflowed()) {  // the per-layer inputs again, on f32 activations
      f32_prefill_ = true;
      try {
        embed_ple(d_ids_, n, x_, split_rows(x_, n, H_), ple_tok_, ple_proj_, ple_pack_);
      } catch (...) {
        f32_prefill_ = false;
        throw;
      }
      f32_prefill_ = false;
      ++f32_prefills_;
    }
  }
  launch_copy_f32(x_ + (size_t)(n - 1) * H_, xdec_, H_, st_);  // the last row, read by the LM head
  state_rows_ = n;
  state_prefill_ = true;
  state_ple_ = gemma_ && c.ple_dim > 0;
  layer_cursor_ = 0;
  sync();
}

void Session::set_hidden(const float* rows, int n) {
  if (n <= 0) fail(ST_MODEL, "ForwardState: empty input");
  ensure_rows(n);
  IEK_HIP(hipMemcpyAsync(x_, rows, (size_t)n * H_ * 4, hipMemcpyHostToDevice, st_));
  launch_copy_f32(x_ + (size_t)(n - 1) * H_, xdec_, H_, st_);
  state_rows_ = n;
  state_prefill_ = true;
  state_ple_ = false;
  layer_cursor_ = 0;
  sync();
}

void Session::prefill_layer(int li) {
  const Config& c = m_->cfg;
  if (li < 0 || li >= c.n_layers) fail(ST_MODEL, "layer index out of range");
  if (li != layer_cursor_)
    fail(ST_MODEL, "layer-level forward: expected layer " + std::to_string(layer_cursor_) + ", got " +
                       std::to_string(li));
  if (!state_prefill_ || state_rows_ <= 0) fail(ST_MODEL, "prefill_layer_block: no prompt state");
  if (gemma_ && c.ple_dim > 0 && !state_ple_) fail(ST_MODEL, "PLE: per-layer inputs missing from the state");
  const int M = state_rows_;
  if (pos_ + M > ctx_) fail(ST_KVCACHE, "KVCache is Full: max len is " + std::to_string(ctx_) + ".");
  // the layer's input is kept so that the layer can run again in the f32 mode (as Session::prefill)
  if (x_save_cap_ < (size_t)M * H_) {
    sync();
    dev_free(x_save_);
    x_save_ = dev_alloc<float>((size_t)M * H_);
    x_save_cap_ = (size_t)M * H_;
  }
  launch_copy_f32(x_, x_save_, (size_t)M * H_, st_);
  launch_fill_i32(d_ovf_, 0, 1, st_);
  auto run = [&] {
    if (gemma_) layer_prefill_gemma(li, M);
    else if (layer_prefill(li, M)) launch_add_f32(x_, tmp_, (size_t)M * H_, st_);
  };
  run();
  if (overflowed()) {
    launch_copy_f32(x_save_, x_, (size_t)M * H_, st_);
    f32_prefill_ = true;
    try {
      run();
    } catch (...) {
      f32_prefill_ = false;
      throw;
    }
    f32_prefill_ = false;
    ++f32_prefills_;
  }
  launch_copy_f32(x_ + (size_t)(M - 1) * H_, xdec_, H_, st_);
  if (++layer_cursor_ == c.n_layers) {
    pos_ += M;
    launch_set_int(d_pos_, pos_, st_);
    layer_cursor_ = 0;
  }
  sync();
}

void Session::decode_layer(int li) {
  const Config& c = m_->cfg;
  if (li < 0 || li >= c.n_layers) fail(ST_MODEL, "layer index out of range");
  if (li != layer_cursor_)
    fail(ST_MODEL, "layer-level forward: expected layer " + std::to_string(layer_cursor_) + ", got " +
                       std::to_string(li));
  if (state_rows_ != 1) fail(ST_MODEL, "decode_layer_block: seq_len must be 1");
  if (pos_ >= ctx_) fail(ST_KVCACHE, "KVCache is Full: max len is " + std::to_string(ctx_) + ".");
  if (gemma_ && c.ple_dim > 0 && !state_ple_) fail(ST_MODEL, "PLE: per-layer inputs missing from the state");
  if (li == 0 && state_prefill_) {
    // a one-row prompt state becomes the decode state (and its per-layer inputs the decode ones)
    launch_copy_f32(x_, xdec_, H_, st_);
    if (state_ple_) launch_copy_f32(ple_pack_, ple_packd_, (size_t)c.n_layers * c.ple_dim, st_);
    state_prefill_ = false;
  }
  const bool last = li == c.n_layers - 1;
  if (gemma_) {
    float* xr = xdec_;
    ResidUpdate pend{};
    layer_decode_gemma(li, xr, pend);
    if (pend.t) launch_rmsnorm_add(xr, pend.t, pend.w, 1, H_, c.rms_eps, pend.has_scale, pend.scale, st_, xdec_);
    else if (xr != xdec_) launch_copy_f32(xr, xdec_, H_, st_);
    if (last) launch_add_int(d_pos_, 1, st_);
  } else {
    layer_decode(li, last);
  }
  if (++layer_cursor_ == c.n_layers) {
    pos_ += 1;
    layer_cursor_ = 0;
  }
  sync();
}

void Session::decode_body(bool head) {
  const Config& c = m_->cfg;
  size_t vocab;
  size_t hid = embedding_hidden(m_->token_embd, &vocab);
  if (chain_) {
    if (!chain_embed_) launch_embed(m_->token_embd.dtype, m_->token_embd.dev, hid, vocab, d_tok_, 1, c.embed_scale, xdec_, st_);
    const int L = c.n_layers;
    for (int li = 0; li <= L; ++li) {
      if (li > 0) {
        const LayerSpec& S = c.layers[li - 1];
        launch_attn_decode(qd_, kc_[li - 1], vc_[li - 1], kv_f32_, attd_, part_, d_cnt_, c.n_heads, c.n_kv_heads,
                           S.head_dim, ctx_, d_pos_, S.window, 1.0f / sqrtf((float)S.head_dim), ctx_, st_);
      }
      const int k = (li == L && head) ? L + 1 : li;
      ChainArgs a{};
      a.phases = static_cast<const ChainPhase*>(chain_ph_[k]);
      a.nphase = chain_np_[k];
      a.pos = d_pos_;
      a.tok = d_tok_;
      a.counters = d_chain_cnt_;
      a.err = d_chain_err_;
      if (li == L) {
        a.pos_inc = d_pos_;
        if (head) {
          a.finish_argmax = 1;
          a.amax_key = d_key_;
          a.amax_flag = d_flag_;
          a.out_tok = d_tok_;
          a.gen = d_gen_;
          a.flags = d_flags_;
          a.step = d_step_;
        }
      }
      chain2_ ? launch_chain2(a, st_) : launch_chain(a, st_);
    }
    return;
  }
  launch_embed(m_->token_embd.dtype, m_->token_embd.dev, hid, vocab, d_tok_, 1, c.embed_scale, xdec_, st_);
  if (gemma_) {
    embed_ple(d_tok_, 1, xdec_, nullptr, ple_tokd_, ple_projd_, ple_packd_);
    float* xr = xdec_;
    ResidUpdate pend{};
    for (int li = 0; li < c.n_layers; ++li) layer_decode_gemma(li, xr, pend);
    // the last layer's update lands in xdec_, where the LM head and the next step read the state
    if (pend.t) launch_rmsnorm_add(xr, pend.t, pend.w, 1, H_, c.rms_eps, pend.has_scale, pend.scale, st_, xdec_);
    else if (xr != xdec_) launch_copy_f32(xr, xdec_, H_, st_);
    launch_add_int(d_pos_, 1, st_);
  } else {
    for (int li = 0; li < c.n_layers; ++li) layer_decode(li, li == c.n_layers - 1);
  }
}

// One greedy step of the loop in generate_greedy: decode the token in d_tok_, then the LM head and
// argmax of the new state (the argmax of the first state runs before the loop).
void Session::step_body() {
  if (chain_) {
    decode_body(true);
  } else {
    decode_body(false);
    argmax_body(true);
  }
}

void Session::decode_token(uint32_t id) {
  size_t vocab;
  embedding_hidden(m_->token_embd, &vocab);
  if ((size_t)id >= vocab)
    fail(ST_MODEL, "token ID " + std::to_string(id) + " out of vocabulary range [0, " + std::to_string(vocab) + ")");
  if (pos_ >= ctx_) fail(ST_KVCACHE, "KVCache is Full: max len is " + std::to_string(ctx_) + ".");
  check_no_layer_forward();
  IEK_HIP(hipMemcpyAsync(d_tok_, &id, 4, hipMemcpyHostToDevice, st_));
  {
    ChainTurn turn(m_->device, st_, chain_);
    decode_body();
  }
  pos_ += 1;
  state_rows_ = 1;
  state_prefill_ = false;
  state_ple_ = gemma_ && m_->cfg.ple_dim > 0;
  layer_cursor_ = 0;
  sync();
  check_chain_error();
}

void Session::check_state() const {
  if (state_rows_ == 0) fail(ST_MODEL, "final_logits_last_token: empty input");
  check_no_layer_forward();
}

// Session-level calls need every layer of the state done: a layer-level forward stopped part way
// has appended its rows to the KV caches of some layers only.
void Session::check_no_layer_forward() const {
  if (layer_cursor_ != 0)
    fail(ST_MODEL, "a layer-level forward is in progress (next layer " + std::to_string(layer_cursor_) + ")");
}

// Final RMSNorm (last row) + LM head (+ soft cap). With `argmax`, the LM-head epilogue also folds
// every logit into the packed greedy key (d_key_) and the non-finite flag (d_flag_).
void Session::logits_body(bool argmax) {
  const Config& c = m_->cfg;
  MvArgs a{};
  a.nseg = 1;
  int head_dt = m_->lm_head.dtype;
  a.w[0] = (const uint8_t*)mv_weight(m_->lm_head, H_, &head_dt);
  a.out[0] = logits_;
  a.n[0] = c.vocab;
  a.x = xdec_;
  a.norm_w = (const float*)m_->output_norm.dev;
  a.eps = c.rms_eps;
  a.K = H_;
  const DevTensor& w = m_->lm_head;
  if (w.dims.size() != 2 || (int)w.dims[0] != H_ || (int)w.dims[1] != c.vocab)
    fail(ST_MATMUL, "LM head dims do not match hidden_dim x vocab_size");
  if (argmax) {
    a.epi = EPI_ARGMAX;
    a.amax_key = d_key_;
    a.amax_flag = d_flag_;
    a.softcap = c.has_softcap ? c.softcap : 0.f;
    launch_mv(head_dt, a, st_);
  } else {
    a.epi = EPI_STORE;
    launch_mv(head_dt, a, st_);
    if (c.has_softcap) launch_softcap(logits_, c.vocab, c.softcap, st_);
  }
}

void Session::logits_last_token(float* out, int n) {
  check_state();
  if (n < m_->cfg.vocab) fail(ST_OP, "logits buffer smaller than vocab_size");
  logits_body(false);
  IEK_HIP(hipMemcpyAsync(out, logits_, (size_t)m_->cfg.vocab * 4, hipMemcpyDeviceToHost, st_));
  sync();
}

// LM head with the fused argmax, then one thread publishes the token (and resets the key/flag).
void Session::argmax_body(bool record) {
  logits_body(true);
  launch_argmax_finish(d_key_, d_flag_, d_tok_, d_gen_, d_flags_, record ? d_step_ : nullptr, st_);
}

uint32_t Session::greedy_next_token() {
  check_state();
  if (m_->cfg.vocab == 0) fail(ST_SAMPLING, "logits slice is empty");
  launch_fill_i32(d_flags_, 0, 1, st_);
  argmax_body(false);
  uint32_t tok = 0;
  int flag = 0;
  IEK_HIP(hipMemcpyAsync(&tok, d_tok_, 4, hipMemcpyDeviceToHost, st_));
  IEK_HIP(hipMemcpyAsync(&flag, d_flags_, 4, hipMemcpyDeviceToHost, st_));
  sync();
  if (flag) fail(ST_SAMPLING, "invalid logits for argmax (empty or non-finite)");
  return tok;
}

uint32_t Session::sample_temperature(float temperature, float r) {
  check_state();
  if (m_->cfg.vocab == 0) fail(ST_SAMPLING, "logits slice is empty");
  logits_body(false);
  launch_sample_temperature(logits_, m_->cfg.vocab, temperature, r, d_tok_, st_);
  uint32_t tok = 0;
  IEK_HIP(hipMemcpyAsync(&tok, d_tok_, 4, hipMemcpyDeviceToHost, st_));
  sync();
  return tok;
}

void Session::generate_greedy(int n, uint32_t* out_ids, bool use_graph) {
  if (n <= 0) return;
  check_state();
  if (pos_ + n > ctx_) fail(ST_KVCACHE, "KVCache is Full: max len is " + std::to_string(ctx_) + ".");
  launch_fill_i32(d_flags_, 0, n + 1, st_);
  launch_set_int(d_step_, 0, st_);
  launch_copy_f32(xdec_, xdec_save_, H_, st_);  // the state to restore if the first step fails
  // greedy token of the current state (step 0), then n x { decode it; greedy token of the new
  // state (step i + 1) }: the last step's token is computed and not returned
  {
    ChainTurn turn(m_->device, st_, chain_);  // waits before, records after (outside the capture)
    argmax_body(true);
    if (use_graph) {
      if (!step_exec_) {
        sync();
        IEK_HIP(hipStreamBeginCapture(st_, hipStreamCaptureModeThreadLocal));
        try {
          step_body();
        } catch (...) {
          hipGraph_t g;
          (void)hipStreamEndCapture(st_, &g);
          if (g) (void)hipGraphDestroy(g);
          throw;
        }
        IEK_HIP(hipStreamEndCapture(st_, &step_graph_));
        IEK_HIP(hipGraphInstantiate(&step_exec_, step_graph_, nullptr, nullptr, 0));
      }
      for (int i = 0; i < n; ++i) IEK_HIP(hipGraphLaunch(step_exec_, st_));
    } else {
      for (int i = 0; i < n; ++i) step_body();
    }
  }
  std::vector<int> flags(n);
  IEK_HIP(hipMemcpyAsync(out_ids, d_gen_, (size_t)n * 4, hipMemcpyDeviceToHost, st_));
  IEK_HIP(hipMemcpyAsync(flags.data(), d_flags_, (size_t)n * 4, hipMemcpyDeviceToHost, st_));
  sync();
  check_chain_error();
  const int pos0 = pos_;
  pos_ += n;
  state_rows_ = 1;
  state_prefill_ = false;
  for (int i = 0; i < n; ++i) {
    if (!flags[i]) continue;
    // The reference loop (src/main.rs:100-116) stops at the first failing greedy_next_token: the KV
    // cache then holds pos0 + i positions and the state is the output of step i - 1's decode. The
    // replayed steps from i on decoded an arbitrary token, so the state is rebuilt: step i - 1's
    // decode runs again at its own position (it rewrites the same KV row with the same values), or,
    // for i == 0, the state from before the loop is restored.
    if (i == 0) {
      launch_copy_f32(xdec_save_, xdec_, H_, st_);
      pos_ = pos0;
      launch_set_int(d_pos_, pos_, st_);
    } else {
      pos_ = pos0 + i - 1;
      launch_set_int(d_pos_, pos_, st_);
      IEK_HIP(hipMemcpyAsync(d_tok_, &out_ids[i - 1], 4, hipMemcpyHostToDevice, st_));
      ChainTurn again(m_->device, st_, chain_);
      decode_body();
      pos_ += 1;
    }
    sync();
    fail(ST_SAMPLING, "invalid logits for argmax (empty or non-finite) at step " + std::to_string(i));
  }
}

void Session::copy_hidden(float* out, size_t cap, int* rows) {
  *rows = state_rows_;
  size_t n = (size_t)state_rows_ * H_;
  if (cap < n) fail(ST_OP, "hidden buffer too small");
  const float* src = state_prefill_ ? x_ : xdec_;
  if (n) IEK_HIP(hipMemcpyAsync(out, src, n * 4, hipMemcpyDeviceToHost, st_));
  sync();
}

void Session::copy_kv(int layer, bool v, float* out, size_t cap) {
  const Config& c = m_->cfg;
  if (layer < 0 || layer >= c.n_layers) fail(ST_MODEL, "layer index out of range");
  const int hd = c.layers[layer].head_dim;
  size_t n = (size_t)c.n_kv_heads * pos_ * hd;
  if (cap < n) fail(ST_OP, "kv buffer too small");
  const size_t cells = (size_t)c.n_kv_heads * ctx_ * hd;
  std::vector<uint8_t> host(cells * (kv_f32_ ? 4 : 2));
  IEK_HIP(hipMemcpyAsync(host.data(), v ? vc_[layer] : kc_[layer], host.size(), hipMemcpyDeviceToHost, st_));
  sync();
  const __half* h16 = reinterpret_cast<const __half*>(host.data());
  const float* h32 = reinterpret_cast<const float*>(host.data());
  for (int h = 0; h < c.n_kv_heads; ++h)
    for (int p = 0; p < pos_; ++p)
      for (int d = 0; d < hd; ++d) {
        const size_t src = ((size_t)h * ctx_ + p) * hd + d;
        out[((size_t)h * pos_ + p) * hd + d] = kv_f32_ ? h32[src] : __half2float(h16[src]);
      }
}

}  // namespace iek
