// Launch arguments of the decode matvec family (kernels/matvec.hip), shared with the host engine.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace iek {

enum MvEpilogue : int {
  EPI_STORE = 0,   // out[s][n] = dot
  EPI_RESID = 1,   // out[0][n] = resid[n] + dot
  EPI_SWIGLU = 2,  // w[0] = gate, w[1] = up: out[0][n] = silu(gate.x) * (up.x)
  EPI_QKV = 3,     // segments q, k, v: RoPE on q and k pairs, q -> out[0], k/v -> the KV cache (f32 or fp16) at *pos
  EPI_ARGMAX = 4,  // logits -> out[0] (optional soft cap), atomicMax of packed (value, first index)
  EPI_GEGLU = 5,   // w[0] = gate, w[1] = up: out[0][n] = gelu_tanh(gate.x) * (up.x)
  EPI_GELU_MUL = 6,  // out[0][n] = gelu_tanh(dot) * mulv[n]
};

struct MvArgs {
  const uint8_t* w[3];
  float* out[3];
  int n[3];
  int seg_start[4];
  int nseg;
  const float* x;       // input vector (raw residual stream when norm_w is set)
  const float* norm_w;  // fused RMSNorm weight, or null
  float eps;
  int K;
  int epi;
  const float* resid;
  // EPI_QKV
  const float* rope_cs;  // [ctx][npairs][2] (cos, sin)
  int npairs, head_dim, ctx;
  const int* pos;
  void* kc;  // [n_kv][ctx][head_dim] of f32 (kv_f32) or fp16
  void* vc;
  int kv_f32;
  // EPI_ARGMAX
  unsigned long long* amax_key;
  int* amax_flag;
  float softcap;  // <= 0: none
  int* pos_inc;   // when set, one thread adds 1 after the launch's work is issued (end of a decode step)
  // EPI_GELU_MUL
  const float* mulv;
  // Optional residual update ahead of the staging (f32-staged traits and the generic path):
  //   y = (x + (pre_t * pre_w) / rms(pre_t)) [* pre_scale]
  // the launch then uses y as its input x (RMS-normalised again when norm_w is set), and workgroup
  // 0 writes y to pre_out (a buffer other than x and pre_t).
  const float* pre_t;
  const float* pre_w;
  float* pre_out;
  float pre_scale;
  int pre_has_scale;
};

__host__ __device__ inline int seg_of(const MvArgs& a, int row) {
  int s = 0;
  if (a.nseg > 1 && row >= a.seg_start[1]) s = 1;
  if (a.nseg > 2 && row >= a.seg_start[2]) s = 2;
  return s;
}

void launch_mv(int dt, MvArgs a, hipStream_t st);
// Segment starts of a launch's row space (launch_mv calls it; exposed for launch builders).
void mv_finalize(MvArgs& a);

}  // namespace iek
