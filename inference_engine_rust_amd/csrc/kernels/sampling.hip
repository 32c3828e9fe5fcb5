// Temperature sampling on the device (src/engine/sampling.rs:54-79): softmax(logits / T) with the
// reference's f32 arithmetic (src/ops/softmax.rs:3-28), then the first index i whose cumulative
// probability exceeds the uniform draw r (the reference's `rng.gen_range(0.0..1.0)`, drawn by the
// caller), the last index when none does.
//
// The reference sums exp(s - max) and then the probabilities one after the other in f32; those
// roundings decide the index when r is near a boundary (over 262144 logits they move the
// cumulative sum by ~1e-5), so they are kept: one 1024-thread workgroup computes each chunk of
// up to CH terms in parallel into LDS, and wave 0 adds the chunk's terms in index order (uniform
// broadcast reads, one dependent f32 add per term). Terms: s_i = x_i / T (f32 division);
// e_i = exp(s_i - max) rounded to f32 from the f64 exponential (the correctly rounded value,
// which glibc's expf returns to within its 0.5-ulp design); p_i = e_i / sum (f32 division).
// A NaN or +inf s_i, or a maximum of -inf, makes every reference probability NaN, so its loop
// never meets `r < cum` and returns the last index: so does this kernel.
// Cost: two passes of dependent adds over the vocabulary (~4 clocks per logit in wave 0; the
// search pass stops at the pick): ~0.1 ms for 32000 logits. It is not on the greedy path.
#include "common.cuh"
#include "../iek_internal.h"

namespace iek {

namespace {

constexpr int ST = 1024;   // threads
constexpr int CH = 16384;  // terms per LDS chunk (64 KiB)
constexpr int GRP = 32;    // terms per group of the search pass (one compare per group)

IEK_DEV float exp_rn(float v) { return (float)exp((double)v); }

__global__ __launch_bounds__(ST) void sample_temperature_kernel(const float* __restrict__ logits, int n, float temp,
                                                                float r, uint32_t* __restrict__ out) {
  __shared__ __align__(16) float buf[CH];
  __shared__ float smax[ST / 64];
  __shared__ int sbad[ST / 64];
  __shared__ float ssum;
  __shared__ int spick;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  // max of s and the NaN / +inf flag
  float m = -INFINITY;
  int bad = 0;
  for (int i = t; i < n; i += ST) {
    const float s = logits[i] / temp;
    bad |= (s != s) | (s == INFINITY);
    m = fmaxf(m, s);
  }
  m = wave_max(m);
  bad = __any(bad) ? 1 : 0;
  if (lane == 0) {
    smax[w] = m;
    sbad[w] = bad;
  }
  __syncthreads();
  float mx = -INFINITY;
  int anybad = 0;
  for (int k = 0; k < ST / 64; ++k) {
    mx = fmaxf(mx, smax[k]);
    anybad |= sbad[k];
  }
  if (anybad || mx == -INFINITY) {
    if (t == 0) *out = (uint32_t)(n - 1);
    return;  // uniform across the workgroup
  }
  // sum_exp in index order (softmax.rs:20-22)
  float sum = 0.f;
  for (int c0 = 0; c0 < n; c0 += CH) {
    const int len = min(CH, n - c0);
    for (int j = t; j < len; j += ST) buf[j] = exp_rn(logits[c0 + j] / temp - mx);
    __syncthreads();
    if (w == 0) {
      int j = 0;
      for (; j + 4 <= len; j += 4) {
        const float4 v = *reinterpret_cast<const float4*>(&buf[j]);
        sum = sum + v.x;
        sum = sum + v.y;
        sum = sum + v.z;
        sum = sum + v.w;
      }
      for (; j < len; ++j) sum = sum + buf[j];
    }
    __syncthreads();
  }
  if (t == 0) ssum = sum;
  if (t == 0) spick = -1;
  __syncthreads();
  sum = ssum;
  // cum += exp(s - max) / sum in index order; first i with r < cum (sampling.rs:70-77)
  float cum = 0.f;
  for (int c0 = 0; c0 < n; c0 += CH) {
    const int len = min(CH, n - c0);
    for (int j = t; j < len; j += ST) buf[j] = exp_rn(logits[c0 + j] / temp - mx) / sum;
    __syncthreads();
    if (w == 0) {
      for (int g0 = 0; g0 < len; g0 += GRP) {
        const int ge = min(g0 + GRP, len);
        float c = cum;
        for (int j = g0; j < ge; ++j) c = c + buf[j];
        if (r < c) {
          // the group holds the pick: walk it again with the same adds
          c = cum;
          int j = g0;
          for (; j < ge; ++j) {
            c = c + buf[j];
            if (r < c) break;
          }
          if (lane == 0) spick = c0 + j;
          break;
        }
        cum = c;
      }
    }
    __syncthreads();        // wave 0 is done with buf before it is refilled
    if (spick >= 0) break;  // uniform: read after the barrier
  }
  if (t == 0) *out = (uint32_t)(spick >= 0 ? spick : n - 1);
}

}  // namespace

void launch_sample_temperature(const float* logits, int n, float temperature, float r, uint32_t* out_dev,
                               hipStream_t st) {
  if (n <= 0) fail(ST_SAMPLING, "logits slice is empty");
  if (!std::isfinite(temperature) || temperature <= 0.0f)
    fail(ST_SAMPLING, "temperature must be positive, got " + std::to_string(temperature));
  if (!(r >= 0.0f && r < 1.0f)) fail(ST_OP, "sample_temperature: the uniform draw must be in [0, 1)");
  hipLaunchKernelGGL(sample_temperature_kernel, dim3(1), dim3(ST), 0, st, logits, n, temperature, r, out_dev);
}

}  // namespace iek
