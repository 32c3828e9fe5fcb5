// Internal declarations shared by the host runtime (C++) and the HIP kernel launchers.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <string>

namespace iek {

// Status codes: the reference's EngineError variants (src/error.rs:5-38) plus a device class.
enum Status : int {
  ST_OK = 0, ST_IO = 1, ST_UTF8 = 2, ST_GGUF = 3, ST_TENSOR = 4, ST_MATMUL = 5, ST_MODEL = 6,
  ST_TOKENIZER = 7, ST_KVCACHE = 8, ST_SAMPLING = 9, ST_OP = 10, ST_DEVICE = 11,
};

// dtype ids follow the reference's TensorType (src/core/tensor.rs:13-23).
enum DType : int { DT_F32 = 0, DT_Q4K = 1, DT_Q6K = 2, DT_Q8_0 = 3,
                   // internal only: Q6_K bytes regrouped per row for 16-byte lane loads (see
                   // kernels/matvec.hip, Q6RTr); never crosses the C ABI
                   DT_Q6K_R = 4,
                   // internal only: Q8_0 quants and scales split into per-row runs (Q8RTr)
                   DT_Q8_0_R = 5 };
// Row bytes of the regrouped Q6_K layout: nsb superblocks of [4 x 48 B lane chunks] followed by
// nsb x 16 scale bytes and nsb x 2 d bytes, padded to 16.
__host__ __device__ inline size_t q6r_row_bytes(size_t nsb) { return nsb * 208 + ((2 * nsb + 15) / 16) * 16; }
void launch_repack_q6k(const void* src, int K, int N, void* dst, hipStream_t st);
// Row bytes of the regrouped Q8_0 layout: nb x 32 quant bytes, then nb x 2 scale bytes padded to 16.
__host__ __device__ inline size_t q8r_row_bytes(size_t nb) { return nb * 32 + ((2 * nb + 15) / 16) * 16; }
void launch_repack_q80(const void* src, int K, int N, void* dst, hipStream_t st);

struct Error {
  int code;
  std::string msg;
};

[[noreturn]] void fail(int code, const std::string& msg);
void check_hip(hipError_t e, const char* what);
#define IEK_HIP(call) ::iek::check_hip((call), #call)

struct MvSegDesc {
  const void* w;
  float* out;
  const float* resid;
  int n;
};

// ---- kernel launchers (all asynchronous on `st`) ----
// epi: 0 store, 1 residual add (out = resid + dot), 2 SwiGLU over a (gate, up) segment pair.
void launch_matvec(int dt, const MvSegDesc* segs, int nseg, const float* x, int K, int epi, hipStream_t st);
void launch_gemm(int dt, const void* w, const float* a, int M, int K, int N, float* out, const float* resid,
                 hipStream_t st);
// Matrix-core GEMM on activations pre-split into fp16 pairs (kernels/gemm_mfma.hip).
void launch_split_f16(const float* x, size_t n, __half* hi, __half* lo, hipStream_t st);
bool gemm_mfma_ok(int dt, const void* w, int K, int N);
// Matrix-core GEMM for K-quant / Q8_0 weights with block scales applied outside the fp16 operands
// (kernels/gemm_q.hip); up to three weight matrices sharing the activation in one launch.
struct GemmQSeg {
  const void* w;
  float* out;
  int n;
};
bool gemm_q_ok(int dt, const void* w, int K);
int num_cus();  // compute units of the current device
void launch_block_sums(const float* a, int M, int K, float* xs, hipStream_t st);
// kpart: optional M x N f32 scratch; with it a one-segment K-quant GEMM whose tiles would fill at
// most half the CUs splits K in two and adds the second half's partial sums in a second pass; with
// defer_add that pass is left to the caller (true is returned while kpart holds the partial sums:
// out + kpart is the result, e.g. through launch_rmsnorm_split's `part`).
bool launch_gemm_q(int dt, const GemmQSeg* segs, int nseg, const __half* xh, const __half* xl, const float* xs, int M,
                   int K, const float* resid, hipStream_t st, float* kpart = nullptr, bool defer_add = false);
// Gate/up projection with SwiGLU in its epilogue (K-quant Q4_K or regrouped Q6_K weights of equal
// shape, N % 32 == 0): writes act = silu(x W_gate^T) * (x W_up^T) as the down projection's input,
// the fp16 (hi, lo) planes [M][N], optionally their per-32 sums (as launch_swiglu_split's `sums`)
// and the f32 act; the same bits as launch_gemm_q into gate and up followed by launch_swiglu_split.
// Returns false, launching nothing, for other weight types or shapes.
bool launch_gemm_q_glu(int dt, const void* w_gate, const void* w_up, int N, const __half* xh, const __half* xl,
                       const float* xs, int M, int K, __half* act_hi, __half* act_lo, float* act_sums, float* act_f32,
                       int* ovf, hipStream_t st);
// out[i] += part[i] for i < n (n % 4 == 0, 16-byte aligned)
void launch_add_f32(float* out, const float* part, size_t n, hipStream_t st);
void launch_gemm_mfma(int dt, const void* w, const __half* xh, const __half* xl, int M, int K, int N, float* out,
                      const float* resid, hipStream_t st);
void launch_dequant(int dt, const void* blocks, size_t nblocks, float* out, hipStream_t st);
// rows: the table's row count (vocabulary); device-produced ids are clamped below it
void launch_embed(int dt, const void* table, size_t hidden, size_t rows, const uint32_t* ids, int n, float scale,
                  float* out, hipStream_t st);
void launch_rmsnorm(const float* in, const float* w, int rows, int dim, float eps, float* out, hipStream_t st);
// Producers that also emit a prefill GEMM input: fp16 (hi, lo) planes of their [rows, dim] output
// and its per-32 sums as an fp16 pair (two planes of rows * dim / 32 halves at `sums`), as
// launch_split_f16 + launch_block_sums would (dim % 32 == 0, 16-byte aligned rows). A null `out`
// skips the f32 output. With `part`, in[i] + part[i] (one f32 add, as launch_add_f32) is
// normalised and written back to `in`. A value or per-32 sum beyond the pair's range (F16_PAIR_MAX)
// sets *ovf (when given).
void launch_rmsnorm_split(float* in, const float* w, int rows, int dim, float eps, float* out, __half* hi,
                          __half* lo, float* sums, int* ovf, hipStream_t st, const float* part = nullptr);
void launch_split_sums(const float* a, int rows, int K, __half* hi, __half* lo, float* sums, int* ovf,
                       hipStream_t st);
void launch_swiglu_split(const float* g, const float* u, float* out, int rows, int K, __half* hi, __half* lo,
                         float* sums, int* ovf, hipStream_t st);
// *ovf = 1 when some |a[i]| (i < n) exceeds F16_PAIR_MAX (a prefill attention input the matrix-core
// kernels split into fp16 pairs themselves).
void launch_range_flag(const float* a, size_t n, int* ovf, hipStream_t st);
// Op-level GEMM inputs with any f32 range: per row, the power-of-two factor s (1 unless the row's
// largest |value| or per-32 sum exceeds 2^15, then the factor that brings it into [2^14, 2^15)),
// the fp16 (hi, lo) planes of s * a and the per-32 sums of s * a (fp16 pair planes), and
// inv[m] = 1 / s. Then launch_row_scale multiplies each output row by inv[m]; power-of-two factors
// make both steps exact.
void launch_split_scaled(const float* a, int rows, int K, __half* hi, __half* lo, float* sums, float* inv,
                         hipStream_t st);
void launch_row_scale(float* out, int rows, int N, const float* inv, hipStream_t st);
// Prefill attention on f32 inputs (the path taken when an input is beyond the fp16 pair's range):
// q [M][n_heads*hd], k and v [M][n_kv*hd] (RoPE applied), causal over the M prompt rows with the
// sliding-window bound; one wave per (query row, head), online softmax in f32.
void launch_attn_prefill_f32(const float* q, const float* k, const float* v, float* out, int M, int n_heads, int n_kv,
                             int head_dim, int window, float scale, hipStream_t st);
// The tiled SIMT GEMM on f32 activations (no fp16 operand), for every weight type.
void launch_gemm_f32(int dt, const void* w, const float* a, int M, int K, int N, float* out, const float* resid,
                     hipStream_t st);
void launch_rope_rows(float* v, int rows, int row_stride, int n_heads, int head_dim, int pos0, const float* cs,
                      int half_pairs, hipStream_t st);
void launch_rope_table(float* v, int n_heads, int head_dim, int npairs, const float* cs, const int* pos_dev,
                       hipStream_t st);
// K/V rows into a [n_kv][ctx][head_dim] cache of f32 (kv_f32) or fp16
void launch_kv_store(const float* k, const float* v, int rows, int kv_dim, void* kc, void* vc, bool kv_f32, int n_kv,
                     int head_dim, int ctx, const int* pos_dev, int pos0, hipStream_t st);
void launch_swiglu(const float* g, const float* u, float* out, size_t n, hipStream_t st);
void launch_gelu_mul(const float* g, const float* u, float* out, size_t n, hipStream_t st);
void launch_residual_add(const float* a, const float* b, float* out, size_t n, hipStream_t st);
void launch_softmax(const float* in, float* out, int n, hipStream_t st);
// Greedy argmax: atomicMax of packed (value, first-index) keys; non-finite logits set flags[*step].
void launch_argmax(const float* logits, int n, unsigned long long* key_out, int* flags, const int* step, hipStream_t st);
// tok[0] = argmax index, flags[step] = *flag; with a step counter also list[*step] = index and
// ++*step; then *key = 0 and *flag = 0.
// sample_temperature (src/engine/sampling.rs:54-79) into *out_dev; validates n, T and r.
void launch_sample_temperature(const float* logits, int n, float temperature, float r, uint32_t* out_dev,
                               hipStream_t st);
void launch_argmax_finish(unsigned long long* key, int* flag, uint32_t* tok, uint32_t* list, int* flags, int* step,
                          hipStream_t st);
void launch_softcap(float* z, int n, float cap, hipStream_t st);
void launch_unpack_qk(const float* src, float* dst, int rows, int row_stride, int n_groups, int head_dim,
                      hipStream_t st);
void launch_copy_f32(const float* src, float* dst, size_t n, hipStream_t st);
void launch_fill_i32(int* p, int v, int n, hipStream_t st);
// `counters` holds 2 * n_kv zero-initialised ints (one per KV head and query-head group); the
// kernel leaves them zero again.
// The cache is fp16, or f32 when kv_f32 (Gemma-4 sessions).
void launch_attn_decode(const float* q, const void* kc, const void* vc, bool kv_f32, float* out, float* part,
                        int* counters, int n_heads, int n_kv, int head_dim, int ctx, const int* pos_dev, int window,
                        float scale, int max_len, hipStream_t st);
// Floats of `part` that launch_attn_decode needs at most for a cache of max_len keys.
size_t attn_decode_part_floats(int n_heads, int head_dim, int max_len);
// The no-allocation scratch (kernels/noalloc.hip): a file-scope device array of this many bytes
// per device, [counters + position: NOALLOC_COUNTER_BYTES][attention partials: the rest].
constexpr size_t NOALLOC_SCRATCH_BYTES = 16u << 20;
constexpr size_t NOALLOC_COUNTER_BYTES = 4096;
// Device address of the scratch array of the stream's device (the current device for the null
// stream), resolved once per device.
void* noalloc_scratch(hipStream_t st);
// With a scratch buffer of attn_prefill_scratch_halves() halves (head_dim 64, 128 or 256), each K/V
// block is staged once for all the query heads of its KV head; otherwise one workgroup per query
// head.
size_t attn_prefill_scratch_halves(int M, int n_kv, int head_dim);
// planes_ready: launch_attn_prefill_prep already wrote the K/V planes into the scratch (and
// flagged out-of-range inputs); otherwise q, k and v are range-checked here into *ovf (when given).
void launch_attn_prefill(const float* q, const float* k, const float* v, float* out, int M, int n_heads, int n_kv,
                         int head_dim, int window, float scale, hipStream_t st, void* scratch = nullptr,
                         size_t scratch_halves = 0, bool planes_ready = false, int* ovf = nullptr);
// RoPE (table `cs`, npairs pairs, prompt positions 0..M-1) on q in place and on k, the KV append of
// k and v at cache position pos0 and the K/V planes of the shared-K/V path, in one launch (k and v
// are left as they were). Returns false, launching nothing, when the shared-K/V path does not
// apply (then the caller runs RoPE, the append and launch_attn_prefill with planes_ready false).
// A q, k or v value beyond F16_PAIR_MAX sets *ovf.
bool launch_attn_prefill_prep(float* q, const float* k, const float* v, int M, int n_heads, int n_kv, int head_dim,
                              const float* cs, int npairs, void* kc, void* vc, bool kv_f32, int ctx, int pos0,
                              void* scratch, size_t scratch_halves, int* ovf, hipStream_t st);
// Gemma-4 pieces (kernels/gemma.hip).
void launch_head_prep(float* q, float* k, float* v, int rows, int q_stride, int kv_stride, int nq, int nkv, int hd,
                      const float* qn, const float* kn, float eps, bool vnorm, const float* cs, int npairs,
                      const int* pos_dev, int rope0, int kv0, void* kc, void* vc, bool kv_f32, int ctx,
                      hipStream_t st);
void launch_rmsnorm_add(float* x, const float* t, const float* w, int rows, int dim, float eps, bool has_scale,
                        float scale, hipStream_t st, float* y = nullptr);
void launch_ple_pack(const float* proj, const float* tok, const float* norm_w, int rows, int n_layers, int pd,
                     float eps, float proj_scale, float sqrt_pd, float combine, float* out, hipStream_t st);
void launch_ple_gate(float* go, const float* packed, int rows, int pd, int n_layers, int layer, hipStream_t st);
void launch_kv_load(const void* kc, const void* vc, bool kv_f32, int rows, int n_kv, int hd, int ctx, float* k,
                    float* v, hipStream_t st);
void launch_fill_u64(unsigned long long* p, unsigned long long v, int n, hipStream_t st);
void launch_set_int(int* p, int v, hipStream_t st);
void launch_add_int(int* p, int v, hipStream_t st);

}  // namespace iek
