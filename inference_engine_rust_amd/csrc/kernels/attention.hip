// Attention over an fp16 KV cache laid out per layer as [n_kv][ctx][head_dim].
//
// Decode (src/layers/attention.rs:462-655): split-K flash-decode over 64-key slices, GQA groups
// sharing one K/V stream; the slice count is fixed by the cache capacity so the launch shape
// never changes between captured decode steps, and the live length is read from device memory.
//
// Prefill (attention.rs:175-422): causal attention over the f32 K/V of the prompt (the
// reference attends to the layer's own k_data/v_data, not the cache).
#include <type_traits>

#include "common.cuh"
#include "../iek_internal.h"

namespace iek {

constexpr int SPLIT = 64;

// One wave per (KV head, 64-key slice). Lane j scores key j0+j against the G query heads of the
// group; the V rows of the slice are fetched in the same burst (lanes over head dims) so each
// wave makes a single trip to HBM. Slices publish (max, sum, o[]) partials; the last wave of a
// KV head (device-scope counter, reset by that wave) merges them into the attention output.
template <int HD>
__global__ __launch_bounds__(64) void attn_decode_kernel(const float* __restrict__ q, const __half* __restrict__ kc,
                                                         const __half* __restrict__ vc, float* __restrict__ part,
                                                         float* __restrict__ out, int* __restrict__ counters,
                                                         int n_heads, int n_kv, int ctx, const int* pos_dev,
                                                         int window, float scale, int nsplit) {
  constexpr int DPL = HD / 64;  // head dims per lane in the PV phase
  constexpr int KV4 = HD / 8;   // uint4 (8 halves) per key row
  const int kvh = blockIdx.x, sp = blockIdx.y, lane = threadIdx.x;
  const int G = n_heads / n_kv;
  const int total = *pos_dev + 1;
  const int jmin = (window > 0 && total > window) ? total - window : 0;
  const int j0 = max(sp * SPLIT, jmin), j1 = min(total, (sp + 1) * SPLIT);
  __shared__ float qs[8][HD];
  __shared__ float ps[8][SPLIT];
  __shared__ int last;
  const int nk = j1 - j0;
  if (nk > 0) {
    const int j = j0 + lane;
    const bool valid = lane < nk;
    uint4 kr[KV4];
    if (valid) {
      const uint4* kp = reinterpret_cast<const uint4*>(kc + ((size_t)kvh * ctx + j) * HD);
#pragma unroll
      for (int c = 0; c < KV4; ++c) kr[c] = kp[c];
    }
    // lane owns head dims [DPL*lane, DPL*lane + DPL) of every V row of the slice
    static_assert(DPL == 2 || DPL == 1 || DPL == 4, "head_dim");
    using VT = typename std::conditional<DPL == 1, uint16_t, typename std::conditional<DPL == 2, uint32_t, uint2>::type>::type;
    VT vraw[SPLIT];
    {
      const __half* vb = vc + ((size_t)kvh * ctx + j0) * HD + DPL * lane;
#pragma unroll
      for (int jj = 0; jj < SPLIT; ++jj)
        if (jj < nk) vraw[jj] = *reinterpret_cast<const VT*>(vb + (size_t)jj * HD);
    }
    for (int i = lane; i < G * HD; i += 64) qs[i / HD][i % HD] = q[(size_t)(kvh * G) * HD + i];
    __syncthreads();
    float sc[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) sc[g] = 0.f;
    if (valid) {
#pragma unroll
      for (int c = 0; c < KV4; ++c) {
        const __half2* h2 = reinterpret_cast<const __half2*>(&kr[c]);
        float kf[8];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float2 f = __half22float2(h2[t]);
          kf[2 * t] = f.x;
          kf[2 * t + 1] = f.y;
        }
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          if (g < G) {
            const float4 qa = *reinterpret_cast<const float4*>(&qs[g][8 * c]);
            const float4 qb = *reinterpret_cast<const float4*>(&qs[g][8 * c + 4]);
            sc[g] += qa.x * kf[0] + qa.y * kf[1] + qa.z * kf[2] + qa.w * kf[3] + qb.x * kf[4] + qb.y * kf[5] +
                     qb.z * kf[6] + qb.w * kf[7];
          }
        }
      }
    }
    float mg[8], lg[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      if (g < G) {
        const float s = valid ? sc[g] * scale : -INFINITY;
        mg[g] = wave_max(s);
        const float p = valid ? expf(s - mg[g]) : 0.f;
        lg[g] = wave_sum(p);
        ps[g][lane] = p;
      }
    }
    __syncthreads();
    float o[8][DPL];
#pragma unroll
    for (int g = 0; g < 8; ++g)
#pragma unroll
      for (int t = 0; t < DPL; ++t) o[g][t] = 0.f;
#pragma unroll
    for (int jj = 0; jj < SPLIT; ++jj) {
      if (jj < nk) {
        float vf[DPL];
        const __half* hv = reinterpret_cast<const __half*>(&vraw[jj]);
#pragma unroll
        for (int t = 0; t < DPL; ++t) vf[t] = __half2float(hv[t]);
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          if (g < G) {
            const float p = ps[g][jj];
#pragma unroll
            for (int t = 0; t < DPL; ++t) o[g][t] += p * vf[t];
          }
        }
      }
    }
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      if (g < G) {
        float* pr = part + ((size_t)(kvh * G + g) * nsplit + sp) * (HD + 2);
        if (lane == 0) {
          pr[0] = mg[g];
          pr[1] = lg[g];
        }
#pragma unroll
        for (int t = 0; t < DPL; ++t) pr[2 + DPL * lane + t] = o[g][t];
      }
    }
  }
  // publish, then let the last slice of this KV head merge
  __threadfence();
  if (lane == 0) {
    const int prev = atomicAdd(&counters[kvh], 1);
    last = prev == nsplit - 1;
    if (last) counters[kvh] = 0;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  const int nlive = (total + SPLIT - 1) / SPLIT;
  const int s0 = jmin / SPLIT;
  for (int g = 0; g < G; ++g) {
    const float* pr = part + (size_t)(kvh * G + g) * nsplit * (HD + 2);
    float M = -INFINITY;
    for (int s = s0; s < nlive; ++s) M = fmaxf(M, __builtin_nontemporal_load(pr + (size_t)s * (HD + 2)));
    float L = 0.f;
    float acc[DPL];
#pragma unroll
    for (int t = 0; t < DPL; ++t) acc[t] = 0.f;
    for (int s = s0; s < nlive; ++s) {
      const float* e = pr + (size_t)s * (HD + 2);
      const float w = expf(__builtin_nontemporal_load(e) - M);
      L += __builtin_nontemporal_load(e + 1) * w;
#pragma unroll
      for (int t = 0; t < DPL; ++t) acc[t] += __builtin_nontemporal_load(e + 2 + DPL * lane + t) * w;
    }
#pragma unroll
    for (int t = 0; t < DPL; ++t) out[(size_t)(kvh * G + g) * HD + DPL * lane + t] = acc[t] / L;
  }
}

void launch_attn_decode(const float* q, const __half* kc, const __half* vc, float* out, float* part, int* counters,
                        int n_heads, int n_kv, int head_dim, int ctx, const int* pos_dev, int window, float scale,
                        int max_len, hipStream_t st) {
  const int nsplit = (max_len + SPLIT - 1) / SPLIT;
  dim3 grid(n_kv, nsplit);
  if (n_heads % n_kv != 0 || n_heads / n_kv > 8) fail(ST_OP, "attention: GQA group larger than 8 is not supported");
  switch (head_dim) {
    case 64:
      hipLaunchKernelGGL(attn_decode_kernel<64>, grid, dim3(64), 0, st, q, kc, vc, part, out, counters, n_heads, n_kv,
                         ctx, pos_dev, window, scale, nsplit);
      break;
    case 128:
      hipLaunchKernelGGL(attn_decode_kernel<128>, grid, dim3(64), 0, st, q, kc, vc, part, out, counters, n_heads,
                         n_kv, ctx, pos_dev, window, scale, nsplit);
      break;
    case 256:
      hipLaunchKernelGGL(attn_decode_kernel<256>, grid, dim3(64), 0, st, q, kc, vc, part, out, counters, n_heads,
                         n_kv, ctx, pos_dev, window, scale, nsplit);
      break;
    default:
      fail(ST_OP, "attention: head_dim must be 64, 128 or 256");
  }
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
