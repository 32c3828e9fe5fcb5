// Device-resident inference session: owns the f32 KV cache, activation buffers, the HIP stream
// and the captured decode-step graph. Mirrors InferenceSession (src/engine/session.rs:12-75).
#pragma once
#include <vector>

#include "model.h"
#include "kernels/chain.h"
#include "kernels/mv_args.h"

namespace iek {

// A pending residual update x <- (x + rmsnorm(t, w)) [* scale] (Gemma-4 post-norms and layer
// output scale), applied by the staging of the next matvec that reads x.
struct ResidUpdate {
  const float* t = nullptr;
  const float* w = nullptr;
  bool has_scale = false;
  float scale = 1.f;
};

class Session {
 public:
  explicit Session(Model* m);
  ~Session();

  void reset();                                   // session.rs:40-42 (fresh KV caches)
  void prefill(const uint32_t* ids, int n);        // session.rs:44-56 (prefill_forward)
  void decode_token(uint32_t id);                  // session.rs:58-69 (decode_forward)
  void logits_last_token(float* out, int n);       // session.rs:71-74 (final_logits_last_token)
  uint32_t greedy_next_token();                    // generation.rs:10-16
  uint32_t sample_temperature(float temperature, float r);  // sampling.rs:54-79 on the device
  // n x (greedy_next_token; decode_token), the loop of main.rs:100-116 / bench_metrics.rs:178-182,
  // replayed as one captured decode-step graph. Returns the n chosen ids.
  void generate_greedy(int n, uint32_t* out_ids, bool use_graph = true);

  // Forward-level steps over the session's ForwardState (src/engine/runtime.rs:14-61,
  // src/layers/block.rs:12-89, src/engine/embed.rs:53-149). Layers run in order: the next call
  // must be for layer `next_layer()`; after the last layer the KV length grows by the state rows.
  void embed(const uint32_t* ids, int n);           // prefill_from_tokens_loaded: state = embeddings
  void set_hidden(const float* rows, int n);        // ForwardState::from_flat (no PLE payload)
  void prefill_layer(int li);                       // prefill_layer_block
  void decode_layer(int li);                        // decode_layer_block (one-row state)
  int next_layer() const { return layer_cursor_; }
  int n_layers() const { return m_->cfg.n_layers; }
  void check_no_layer_forward() const;  // IEK_ERR_MODEL while a layer-level forward is part way

  // Average duration (us) of `reps` back-to-back launches of one hot kernel on the session stream,
  // between two HIP events, and its algorithmic work per launch (*work: bytes or flops).
  // which 0: the decode chain launch of a middle layer (O, gate/up, down, next layer's Q/K/V);
  // which 1: the prefill gate/up GEMM over the last prefill's rows. Leaves the session reset.
  double bench_kernel(int which, int reps, double* work);

  int kv_len() const { return pos_; }
  int decode_path() const { return chain_ ? (chain2_ ? 2 : 1) : 0; }
  // Iteration limit of the decode chain's bounded waits (0: the default). A test aid: a small
  // limit makes the next chain step give up its waits and fail with ST_DEVICE.
  void set_chain_spin(unsigned spin);
  // Prefills (session or layer level) that ran again in the f32 mode because an activation was
  // beyond the fp16 pair's range.
  int f32_prefills() const { return f32_prefills_; }
  int state_rows() const { return state_rows_; }
  void copy_hidden(float* out, size_t cap, int* rows);
  void copy_kv(int layer, bool v, float* out, size_t cap);  // [n_kv][pos][head_dim] -> f32
  hipStream_t stream() const { return st_; }
  Model* model() const { return m_; }

 private:
  void ensure_rows(int rows);
  // pend_in: tmp_ holds split-K partial sums still to be added into x_ (the previous layer's down
  // projection); returns true when this layer's down projection leaves such partial sums.
  bool layer_prefill(int li, int M, bool pend_in = false);
  // *pending (when given): a split-K partial was left in kpart for the caller to add into outs[0].
  // xin / sin: the input's fp16 pair planes and per-32 sums (default xs_ and xsum_).
  bool project_q(const DevTensor* const* ws, float* const* outs, int nseg, int M, int K, const float* resid,
                 float* kpart = nullptr, bool* pending = nullptr, const __half* xin = nullptr,
                 const float* sin = nullptr);
  bool quant_ready(const DevTensor* const* ws, int nseg, int M, int K) const;
  bool gate_up_glu(int li, int M);
  bool fused_ok(int li) const;
  void decode_args(int li, MvArgs& qkv, MvArgs& o, MvArgs& gate_up, MvArgs& down, int* dts);
  void layer_decode(int li, bool last);
  void layer_decode_unfused(int li);
  // Gemma-4 family (attention.rs / ffn.rs Gemma branches, gemma4_ple.rs)
  const __half* split_rows(const float* a, int M, int K);
  void embed_ple(const uint32_t* d_ids, int n, const float* x, const __half* xs, float* tok, float* proj, float* pack);
  void layer_prefill_gemma(int li, int M);
  void layer_decode_gemma(int li, float*& xr, ResidUpdate& pend);
  // embed(d_tok) + every layer + pos++ (and, with `head` on the chain path, the LM head and
  // greedy argmax of the new state, recorded like argmax_body(true)); no host sync
  void decode_body(bool head = false);
  void step_body();  // one greedy step: decode d_tok + argmax of the new state (recorded)
  void prepare_chain();
  void check_chain_error();
  void logits_body(bool argmax);  // final norm + LM head (+ softcap) into logits_
  void argmax_body(bool record);
  void sync();
  bool overflowed();
  void check_state() const;

  Model* m_;
  hipStream_t st_ = nullptr;
  int ctx_ = 0, H_ = 0;
  void* kv_blob_ = nullptr;
  // per-layer K/V caches [n_kv][ctx][head_dim]: fp16, or f32 when kv_f32_ (Gemma-4)
  std::vector<void*> kc_, vc_;
  bool kv_f32_ = false;
  // activations; prefill buffers hold rows_cap_ rows
  int rows_cap_ = 0;
  float *x_ = nullptr, *xn_ = nullptr, *q_ = nullptr, *k_ = nullptr, *v_ = nullptr, *att_ = nullptr;
  float *g_ = nullptr, *u_ = nullptr, *act_ = nullptr, *tmp_ = nullptr;
  bool kpart_ok_ = false;  // tmp_ can hold a [rows, hidden] split-K partial
  __half* xs_ = nullptr;  // fp16 (hi, lo) split of the current prefill GEMM input
  size_t xs_halves_ = 0;
  size_t xs_halves() const { return xs_halves_; }
  float* xsum_ = nullptr;  // its per-32 row sums (Q4_K min term)
  float *xdec_ = nullptr, *xdec2_ = nullptr, *xdec_save_ = nullptr, *xndec_ = nullptr, *qd_ = nullptr, *kd_ = nullptr, *vd_ = nullptr, *attd_ = nullptr;
  float *actd_ = nullptr, *logits_ = nullptr, *part_ = nullptr, *tmpd_ = nullptr;
  // per-layer embeddings (Gemma-4): token rows, model projection and packed inputs, [rows][L*pd]
  float *ple_tok_ = nullptr, *ple_proj_ = nullptr, *ple_pack_ = nullptr;
  float *ple_tokd_ = nullptr, *ple_projd_ = nullptr, *ple_packd_ = nullptr;
  bool gemma_ = false;
  // device-side loop state
  int* d_pos_ = nullptr;
  int* d_step_ = nullptr;
  int* d_flags_ = nullptr;
  uint32_t* d_tok_ = nullptr;
  uint32_t* d_ids_ = nullptr;  // prompt ids / generated ids
  uint32_t* d_gen_ = nullptr;
  unsigned long long* d_key_ = nullptr;
  int* d_flag_ = nullptr;  // non-finite logit seen by the fused argmax
  int* d_cnt_ = nullptr;   // per-KV-head slice counters of the decode attention
  // Prefill inputs beyond the fp16 pair's range: the flag the splitting kernels set, its pinned
  // host copy, whether the prefill is running in the f32 mode, how often it has, and the layer
  // input a layer-level prefill keeps for a rerun.
  int* d_ovf_ = nullptr;
  int* h_ovf_ = nullptr;
  bool f32_prefill_ = false;
  int f32_prefills_ = 0;
  float* x_save_ = nullptr;
  size_t x_save_cap_ = 0;
  int pos_ = 0;
  int state_rows_ = 0;  // rows of the last ForwardState (0 = none)
  bool state_prefill_ = false;
  bool state_ple_ = false;   // the state carries its per-layer-embedding payload (Gemma-4)
  int layer_cursor_ = 0;     // next layer of a layer-level forward
  // decode chain path (kernels/chain.hip): device ChainPhase arrays per launch; launch 0 holds
  // layer 0's Q/K/V, launch l + 1 layer l's O, gate/up, down and layer l + 1's Q/K/V; the last
  // layer's launch comes in two forms, without and with the LM head + argmax
  bool chain_ = false;
  bool chain_embed_ = false;  // launch 0 dequantises the token's embedding row itself
  bool chain2_ = false;       // the tiled chain kernel (launch_chain2) rather than chain_kernel
  static int chain_counter_words() { return std::max(CHAIN_COUNTER_WORDS, CHAIN2_COUNTER_WORDS); }
  void* chain_blob_ = nullptr;
  std::vector<const void*> chain_ph_;
  std::vector<int> chain_np_;
  unsigned* d_chain_cnt_ = nullptr;
  int* d_chain_err_ = nullptr;
  hipGraphExec_t step_exec_ = nullptr;
  hipGraph_t step_graph_ = nullptr;
};

}  // namespace iek
