// Attention over an fp16 KV cache laid out per layer as [n_kv][ctx][head_dim].
//
// Decode (src/layers/attention.rs:462-655): split-K flash-decode. One wave owns one KV head and
// one 64-key slice; each lane scores one key for all G = n_heads/n_kv query heads of the GQA
// group (K streamed once per group), then lanes switch to head dimensions to accumulate
// p*V. Slices write (max, sum, o[]) partials; a combine pass merges them with the usual
// rescaling. The number of slices is fixed by the cache capacity so the launch shape never
// changes between captured decode steps; the live length is read from device memory.
//
// Prefill (attention.rs:175-422): causal attention over the f32 K/V of the prompt (the
// reference attends to the layer's own k_data/v_data, not the cache).
#include "common.cuh"
#include "../iek_internal.h"

namespace iek {

constexpr int SPLIT = 64;

template <int HD>
__global__ __launch_bounds__(64) void attn_decode_partial_kernel(const float* __restrict__ q,
                                                                 const __half* __restrict__ kc,
                                                                 const __half* __restrict__ vc, float* __restrict__ part,
                                                                 int n_heads, int n_kv, int ctx, const int* pos_dev,
                                                                 int window, float scale, int nsplit) {
  constexpr int DPL = HD / 64;  // head dims per lane in the PV phase
  const int kvh = blockIdx.x, sp = blockIdx.y, lane = threadIdx.x;
  const int G = n_heads / n_kv;
  const int total = *pos_dev + 1;
  const int jmin = (window > 0 && total > window) ? total - window : 0;
  const int j0 = max(sp * SPLIT, jmin), j1 = min(total, (sp + 1) * SPLIT);
  __shared__ float qs[8][HD];
  __shared__ float ps[8][SPLIT];
  for (int i = lane; i < G * HD; i += 64) qs[i / HD][i % HD] = q[(size_t)(kvh * G + i / HD) * HD + i % HD];
  __syncthreads();
  float* prow = part + ((size_t)(kvh * G) * nsplit + sp) * (HD + 2);
  if (j0 >= j1) {
    for (int g = 0; g < G; ++g) {
      float* pr = prow + (size_t)g * nsplit * (HD + 2);
      if (lane == 0) {
        pr[0] = -INFINITY;
        pr[1] = 0.f;
      }
      for (int d = lane; d < HD; d += 64) pr[2 + d] = 0.f;
    }
    return;
  }
  const int j = j0 + lane;
  const bool valid = j < j1;
  float sc[8];
#pragma unroll
  for (int g = 0; g < 8; ++g) sc[g] = 0.f;
  if (valid) {
    const uint4* kp = reinterpret_cast<const uint4*>(kc + ((size_t)kvh * ctx + j) * HD);
#pragma unroll 4
    for (int c = 0; c < HD / 8; ++c) {
      uint4 raw = kp[c];
      const __half2* h2 = reinterpret_cast<const __half2*>(&raw);
      float kf[8];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        float2 f = __half22float2(h2[t]);
        kf[2 * t] = f.x;
        kf[2 * t + 1] = f.y;
      }
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        if (g < G) {
#pragma unroll
          for (int t = 0; t < 8; ++t) sc[g] += qs[g][8 * c + t] * kf[t];
        }
      }
    }
  }
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    if (g >= G) break;
    float s = valid ? sc[g] * scale : -INFINITY;
    float m = wave_max(s);
    float p = valid ? expf(s - m) : 0.f;
    float l = wave_sum(p);
    ps[g][lane] = p;
    if (lane == 0) {
      float* pr = prow + (size_t)g * nsplit * (HD + 2);
      pr[0] = m;
      pr[1] = l;
    }
  }
  __syncthreads();
  float o[8][DPL];
#pragma unroll
  for (int g = 0; g < 8; ++g)
#pragma unroll
    for (int t = 0; t < DPL; ++t) o[g][t] = 0.f;
  const int nk = j1 - j0;
  const __half* vbase = vc + ((size_t)kvh * ctx + j0) * HD;
  for (int jj = 0; jj < nk; ++jj) {
    float vf[DPL];
#pragma unroll
    for (int t = 0; t < DPL; ++t) vf[t] = __half2float(vbase[(size_t)jj * HD + lane + 64 * t]);
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      if (g < G) {
        float p = ps[g][jj];
#pragma unroll
        for (int t = 0; t < DPL; ++t) o[g][t] += p * vf[t];
      }
    }
  }
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    if (g < G) {
      float* pr = prow + (size_t)g * nsplit * (HD + 2);
#pragma unroll
      for (int t = 0; t < DPL; ++t) pr[2 + lane + 64 * t] = o[g][t];
    }
  }
}

__global__ void attn_decode_combine_kernel(const float* part, float* out, int nsplit, int hd) {
  const int h = blockIdx.x;
  const float* pr = part + (size_t)h * nsplit * (hd + 2);
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, pr[(size_t)s * (hd + 2)]);
  float L = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    float m = pr[(size_t)s * (hd + 2)];
    if (m != -INFINITY) L += pr[(size_t)s * (hd + 2) + 1] * expf(m - M);
  }
  for (int d = threadIdx.x; d < hd; d += blockDim.x) {
    float acc = 0.f;
    for (int s = 0; s < nsplit; ++s) {
      float m = pr[(size_t)s * (hd + 2)];
      if (m != -INFINITY) acc += pr[(size_t)s * (hd + 2) + 2 + d] * expf(m - M);
    }
    out[(size_t)h * hd + d] = acc / L;
  }
}

void launch_attn_decode(const float* q, const __half* kc, const __half* vc, float* out, float* part, int n_heads,
                        int n_kv, int head_dim, int ctx, const int* pos_dev, int window, float scale, int max_len,
                        hipStream_t st) {
  const int nsplit = (max_len + SPLIT - 1) / SPLIT;
  dim3 grid(n_kv, nsplit);
  if (n_heads / n_kv > 8) fail(ST_OP, "attention: GQA group larger than 8 is not supported");
  switch (head_dim) {
    case 64:
      hipLaunchKernelGGL(attn_decode_partial_kernel<64>, grid, dim3(64), 0, st, q, kc, vc, part, n_heads, n_kv, ctx,
                         pos_dev, window, scale, nsplit);
      break;
    case 128:
      hipLaunchKernelGGL(attn_decode_partial_kernel<128>, grid, dim3(64), 0, st, q, kc, vc, part, n_heads, n_kv, ctx,
                         pos_dev, window, scale, nsplit);
      break;
    case 256:
      hipLaunchKernelGGL(attn_decode_partial_kernel<256>, grid, dim3(64), 0, st, q, kc, vc, part, n_heads, n_kv, ctx,
                         pos_dev, window, scale, nsplit);
      break;
    default:
      fail(ST_OP, "attention: head_dim must be 64, 128 or 256");
  }
  hipLaunchKernelGGL(attn_decode_combine_kernel, dim3(n_heads), dim3(128), 0, st, part, out, nsplit, head_dim);
}

// Prefill: one wave per (head, 64-query tile); lane i owns query i. Keys/values are staged in
// LDS 32 at a time; online softmax per query.
template <int HD>
__global__ __launch_bounds__(64) void attn_prefill_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                          const float* __restrict__ v, float* __restrict__ out, int M,
                                                          int n_heads, int n_kv, int window, float scale) {
  constexpr int KT = 32;
  const int h = blockIdx.x, qt = blockIdx.y, lane = threadIdx.x;
  const int G = n_heads / n_kv, kvh = h / G;
  const int qd = n_heads * HD, kvd = n_kv * HD;
  const int i = qt * 64 + lane;
  const bool valid = i < M;
  __shared__ float ks[KT][HD];
  __shared__ float vs[KT][HD];
  float qr[HD], o[HD];
#pragma unroll
  for (int d = 0; d < HD; ++d) {
    qr[d] = valid ? q[(size_t)i * qd + h * HD + d] : 0.f;
    o[d] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const int last_q = min(M - 1, qt * 64 + 63);
  const int jmin_tile = window > 0 ? max(0, qt * 64 - (window - 1)) : 0;
  for (int jt = (jmin_tile / KT) * KT; jt <= last_q; jt += KT) {
    __syncthreads();
    for (int e = lane; e < KT * HD; e += 64) {
      int jj = jt + e / HD, d = e % HD;
      ks[e / HD][d] = jj < M ? k[(size_t)jj * kvd + kvh * HD + d] : 0.f;
      vs[e / HD][d] = jj < M ? v[(size_t)jj * kvd + kvh * HD + d] : 0.f;
    }
    __syncthreads();
    if (!valid) continue;
    const int jmin = window > 0 ? max(0, i - (window - 1)) : 0;
    for (int t = 0; t < KT; ++t) {
      const int j = jt + t;
      if (j > i || j < jmin) continue;
      float s = 0.f;
#pragma unroll
      for (int d = 0; d < HD; ++d) s += qr[d] * ks[t][d];
      s *= scale;
      const float mn = fmaxf(m, s);
      const float corr = expf(m - mn);
      const float p = expf(s - mn);
      l = l * corr + p;
#pragma unroll
      for (int d = 0; d < HD; ++d) o[d] = o[d] * corr + p * vs[t][d];
      m = mn;
    }
  }
  if (valid) {
#pragma unroll
    for (int d = 0; d < HD; ++d) out[(size_t)i * qd + h * HD + d] = o[d] / l;
  }
}

void launch_attn_prefill(const float* q, const float* k, const float* v, float* out, int M, int n_heads, int n_kv,
                         int head_dim, int window, float scale, hipStream_t st) {
  dim3 grid(n_heads, (M + 63) / 64);
  switch (head_dim) {
    case 64:
      hipLaunchKernelGGL(attn_prefill_kernel<64>, grid, dim3(64), 0, st, q, k, v, out, M, n_heads, n_kv, window, scale);
      break;
    case 128:
      hipLaunchKernelGGL(attn_prefill_kernel<128>, grid, dim3(64), 0, st, q, k, v, out, M, n_heads, n_kv, window,
                         scale);
      break;
    default:
      fail(ST_OP, "prefill attention: head_dim must be 64 or 128");
  }
}

}  // namespace iek
