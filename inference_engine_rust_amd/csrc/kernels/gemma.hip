// Gemma-4 pieces of the token loop that the Mistral path does not have:
//   per-head RMSNorm of q and k, scale-free RMSNorm of v, then RoPE and the KV append
//     (src/layers/attention.rs:277-308, 424-455; src/ops/rmsnorm.rs:8-23)
//   post-norm + residual, with the layer output scale folded into the last one of a layer
//     (attention.rs:696-940 Gemma branch; src/layers/ffn.rs:120-167, 170-240, 242-278)
//   per-layer-embedding (PLE) packing and its gated input (src/layers/gemma4_ple.rs:27-109,
//     ffn.rs:196-205)
//   f32 rows from a KV cache, for prefill attention of a layer that borrows another layer's
//     cache (attention.rs:219-241, 362)
// Every f32 step the reference rounds separately is kept separate (contract off).
#include "common.cuh"
#include "../iek_internal.h"

namespace iek {

// rms = sqrt(sum / dim + eps) with the reference's roundings.
IEK_DEV float rms_value(float ss, int dim, float eps) {
#pragma clang fp contract(off)
  return sqrtf(ss / (float)dim + eps);
}

// One wave per (row, head). Heads [0, nq) are q heads, [nq, nq + nkv) k heads and
// [nq + nkv, nq + 2 nkv) v heads (absent when the layer borrows its cache). q/k: RMSNorm with the
// head weight when one is given, then RoPE on pairs (2p, 2p+1), p < npairs, at the row's position;
// v: x / rms when vnorm. k and v are written back as f32 (prefill attention reads them) and, when
// kc is set, appended to the cache (f32, or fp16 when kv_f32 is 0). Positions: a decode step
// reads both from pos_dev; a prompt rotates row r at rope0 + r (the reference's prompt positions
// start at 0) and appends it at kv0 + r (the cache's current length).
template <int EPL>
__global__ __launch_bounds__(64) void head_prep_kernel(float* __restrict__ q, float* __restrict__ k,
                                                       float* __restrict__ v, int q_stride, int kv_stride, int nq,
                                                       int nkv, int hd, const float* __restrict__ qn,
                                                       const float* __restrict__ kn, float eps, int vnorm,
                                                       const float* __restrict__ cs, int npairs,
                                                       const int* __restrict__ pos_dev, int rope0, int kv0,
                                                       void* __restrict__ kc, void* __restrict__ vc, int kv_f32,
                                                       int ctx) {
#pragma clang fp contract(off)
  __shared__ float sh[EPL * 64];
  const int row = blockIdx.x, head = blockIdx.y, lane = threadIdx.x;
  int kind, hh;
  if (head < nq) {
    kind = 0;
    hh = head;
  } else if (head < nq + nkv) {
    kind = 1;
    hh = head - nq;
  } else {
    kind = 2;
    hh = head - nq - nkv;
  }
  float* base = kind == 0 ? q + (size_t)row * q_stride : (kind == 1 ? k : v) + (size_t)row * kv_stride;
  base += (size_t)hh * hd;
  const float* nw = kind == 0 ? qn : (kind == 1 ? kn : nullptr);
  float x[EPL];
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < EPL; ++t) {
    const int e = lane + 64 * t;
    x[t] = e < hd ? base[e] : 0.f;
    ss += x[t] * x[t];
  }
  if (nw || (kind == 2 && vnorm)) {
    ss = wave_sum(ss);
    const float rms = rms_value(ss, hd, eps);
#pragma unroll
    for (int t = 0; t < EPL; ++t) {
      const int e = lane + 64 * t;
      if (e < hd) {
        if (nw) x[t] = (x[t] * nw[e]) / rms;
        else if (rms > 0.f) x[t] = x[t] / rms;
      }
    }
  }
  const int dpos = pos_dev ? *pos_dev : 0;
  const int pos = (pos_dev ? dpos : rope0) + row, kpos = (pos_dev ? dpos : kv0) + row;
  if (kind < 2 && npairs > 0) {
#pragma unroll
    for (int t = 0; t < EPL; ++t) sh[lane + 64 * t] = x[t];
    __syncthreads();
#pragma unroll
    for (int t = 0; t < EPL; ++t) {
      const int e = lane + 64 * t, p = e >> 1;
      if (e < hd && p < npairs) {
        const float c = cs[((size_t)pos * npairs + p) * 2], s = cs[((size_t)pos * npairs + p) * 2 + 1];
        const float t0 = sh[2 * p], t1 = sh[2 * p + 1];
        x[t] = (e & 1) == 0 ? t0 * c - t1 * s : t0 * s + t1 * c;
      }
    }
  }
#pragma unroll
  for (int t = 0; t < EPL; ++t) {
    const int e = lane + 64 * t;
    if (e < hd) {
      base[e] = x[t];
      if (kind > 0 && kc) {
        const size_t dst = ((size_t)hh * ctx + kpos) * hd + e;
        void* cache = kind == 1 ? kc : vc;
        if (kv_f32) static_cast<float*>(cache)[dst] = x[t];
        else static_cast<__half*>(cache)[dst] = __float2half_rn(x[t]);
      }
    }
  }
}

void launch_head_prep(float* q, float* k, float* v, int rows, int q_stride, int kv_stride, int nq, int nkv, int hd,
                      const float* qn, const float* kn, float eps, bool vnorm, const float* cs, int npairs,
                      const int* pos_dev, int rope0, int kv0, void* kc, void* vc, bool kv_f32, int ctx,
                      hipStream_t st) {
  if (rows <= 0) return;
  if (hd <= 0 || hd > 512 || hd % 2 != 0) fail(ST_OP, "head prep: head_dim must be even and at most 512");
  dim3 grid(rows, nq + 2 * nkv);
#define IEK_HP(E)                                                                                                   \
  hipLaunchKernelGGL(head_prep_kernel<E>, grid, dim3(64), 0, st, q, k, v, q_stride, kv_stride, nq, nkv, hd, qn, kn, \
                     eps, vnorm ? 1 : 0, cs, npairs, pos_dev, rope0, kv0, kc, vc, kv_f32 ? 1 : 0, ctx)
  if (hd <= 64) IEK_HP(1);
  else if (hd <= 128) IEK_HP(2);
  else if (hd <= 256) IEK_HP(4);
  else IEK_HP(8);
#undef IEK_HP
}

// y[r] = (x[r] + (t[r] * w) / rms(t[r])) * scale (y = x when no output is given), one 256-thread
// workgroup per row; has_scale false skips the multiply (the reference applies no scale when the
// layer has none).
__global__ __launch_bounds__(256) void rmsnorm_add_kernel(const float* x, const float* __restrict__ t,
                                                          const float* __restrict__ w, int dim, float eps,
                                                          float scale, int has_scale, float* y) {
#pragma clang fp contract(off)
  __shared__ float sh[4];
  const float* tr = t + (size_t)blockIdx.x * dim;
  const float* xr = x + (size_t)blockIdx.x * dim;
  float* yr = y + (size_t)blockIdx.x * dim;
  float ss = 0.f;
  for (int i = threadIdx.x; i < dim; i += 256) ss += tr[i] * tr[i];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = ss;
  __syncthreads();
  ss = (sh[0] + sh[1]) + (sh[2] + sh[3]);
  const float rms = rms_value(ss, dim, eps);
  for (int i = threadIdx.x; i < dim; i += 256) {
    float v = xr[i] + (tr[i] * w[i]) / rms;
    if (has_scale) v = v * scale;
    yr[i] = v;
  }
}

void launch_rmsnorm_add(float* x, const float* t, const float* w, int rows, int dim, float eps, bool has_scale,
                        float scale, hipStream_t st, float* y) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(rmsnorm_add_kernel, dim3(rows), dim3(256), 0, st, x, t, w, dim, eps, scale, has_scale ? 1 : 0,
                     y ? y : x);
}

// PLE packing (gemma4_ple.rs:27-109) for one (row, layer) per workgroup:
//   v = proj * proj_scale; out = (rmsnorm(v, norm_w) + tok * sqrt(pd)) * combine
// where proj is the row's per_layer_model_proj output and tok its per_layer_token_embd row.
__global__ __launch_bounds__(256) void ple_pack_kernel(const float* __restrict__ proj, const float* __restrict__ tok,
                                                       const float* __restrict__ nw, int pd, int pack, float eps,
                                                       float proj_scale, float sqrt_pd, float combine,
                                                       float* __restrict__ out) {
#pragma clang fp contract(off)
  __shared__ float sh[4];
  const size_t off = (size_t)blockIdx.x * pack + (size_t)blockIdx.y * pd;
  float ss = 0.f;
  for (int i = threadIdx.x; i < pd; i += 256) {
    const float v = proj[off + i] * proj_scale;
    ss += v * v;
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = ss;
  __syncthreads();
  ss = (sh[0] + sh[1]) + (sh[2] + sh[3]);
  const float rms = rms_value(ss, pd, eps);
  for (int i = threadIdx.x; i < pd; i += 256) {
    const float v = proj[off + i] * proj_scale;
    const float nv = (v * nw[i]) / rms;
    out[off + i] = (nv + tok[off + i] * sqrt_pd) * combine;
  }
}

void launch_ple_pack(const float* proj, const float* tok, const float* norm_w, int rows, int n_layers, int pd,
                     float eps, float proj_scale, float sqrt_pd, float combine, float* out, hipStream_t st) {
  if (rows <= 0 || n_layers <= 0) return;
  hipLaunchKernelGGL(ple_pack_kernel, dim3(rows, n_layers), dim3(256), 0, st, proj, tok, norm_w, pd, n_layers * pd,
                     eps, proj_scale, sqrt_pd, combine, out);
}

// go[r][i] = gelu_tanh(go[r][i]) * packed[r][layer * pd + i] (ffn.rs:196-205).
__global__ void ple_gate_kernel(float* __restrict__ go, const float* __restrict__ packed, int rows, int pd, int pack,
                                int layer) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * pd) return;
  const int r = i / pd, c = i % pd;
  go[i] = gelu_tanh_dev(go[i]) * packed[(size_t)r * pack + (size_t)layer * pd + c];
}

void launch_ple_gate(float* go, const float* packed, int rows, int pd, int n_layers, int layer, hipStream_t st) {
  const int n = rows * pd;
  if (n <= 0) return;
  hipLaunchKernelGGL(ple_gate_kernel, dim3((n + 255) / 256), dim3(256), 0, st, go, packed, rows, pd, n_layers * pd,
                     layer);
}

// Rows [0, rows) of a layer's cache ([n_kv][ctx][hd], fp16 or f32) as f32 rows [rows][n_kv * hd].
template <class T>
__global__ void kv_load_kernel(const T* __restrict__ kc, const T* __restrict__ vc, int rows, int n_kv, int hd,
                               int ctx, float* __restrict__ k, float* __restrict__ v) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t kvd = (size_t)n_kv * hd;
  if (i >= (size_t)rows * kvd) return;
  const int r = (int)(i / kvd), c = (int)(i % kvd), h = c / hd, d = c % hd;
  const size_t src = ((size_t)h * ctx + r) * hd + d;
  k[i] = (float)kc[src];
  v[i] = (float)vc[src];
}

void launch_kv_load(const void* kc, const void* vc, bool kv_f32, int rows, int n_kv, int hd, int ctx, float* k,
                    float* v, hipStream_t st) {
  const size_t n = (size_t)rows * n_kv * hd;
  if (n == 0) return;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (kv_f32)
    hipLaunchKernelGGL(kv_load_kernel<float>, grid, dim3(256), 0, st, (const float*)kc, (const float*)vc, rows, n_kv,
                       hd, ctx, k, v);
  else
    hipLaunchKernelGGL(kv_load_kernel<__half>, grid, dim3(256), 0, st, (const __half*)kc, (const __half*)vc, rows,
                       n_kv, hd, ctx, k, v);
}

}  // namespace iek
