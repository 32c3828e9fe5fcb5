// Small ops: block dequant, embedding gather, RMSNorm, RoPE (+KV append), gated
// activations, residual add, softmax and the on-device greedy argmax.
// Each follows the reference op it replaces (src/ops/*.rs). HIP's __fmul_rn/__fadd_rn are plain
// operators that clang may still fuse into FMAs, so functions whose f32 steps the reference rounds
// separately also turn contraction off (#pragma clang fp contract(off)).
#include "common.cuh"
#include "../iek_internal.h"

namespace iek {

__global__ void dequant_kernel(int dt, const uint8_t* blocks, size_t n, float* out) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = flat_elem(dt, blocks, i);
}

void launch_dequant(int dt, const void* blocks, size_t nblocks, float* out, hipStream_t st) {
  size_t be = dt == DT_Q8_0 ? Q8_0_ELEMS : QK_K;
  size_t n = nblocks * be;
  if (n == 0) return;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, dt,
                     (const uint8_t*)blocks, n, out);
}

// Token-row gather (src/layers/embeddings.rs:95-210): element h of token t sits at flat index
// t*hidden + h. `ids` lives in device memory so a captured decode step can read the token that
// the previous step's argmax produced.
// One thread per element: row r = blockIdx.x, elements blockIdx.y*256 + threadIdx.x (a single
// decode row spreads over hidden/256 workgroups instead of looping in one).
// The host range-checks the ids it is given; an id the device produced is clamped to the table
// (a flagged step, whose id is never used, cannot send the read past it).
__global__ void embed_kernel(int dt, const uint8_t* table, size_t hidden, size_t rows, const uint32_t* ids, float scale,
                             float* out) {
  const int r = blockIdx.x;
  const size_t h = (size_t)blockIdx.y * 256 + threadIdx.x;
  if (h >= hidden) return;
  const size_t base = std::min((size_t)ids[r], rows - 1) * hidden;
  float v = flat_elem(dt, table, base + h);
  if (scale != 1.0f) v = v * scale;
  out[(size_t)r * hidden + h] = v;
}

void launch_embed(int dt, const void* table, size_t hidden, size_t rows, const uint32_t* ids, int n, float scale,
                  float* out, hipStream_t st) {
  if (rows == 0) fail(ST_TENSOR, "embedding table has no rows");
  hipLaunchKernelGGL(embed_kernel, dim3(n, (unsigned)((hidden + 255) / 256)), dim3(256), 0, st, dt,
                     (const uint8_t*)table, hidden, rows, ids, scale, out);
}

// Block-wide sum for 256-thread blocks.
IEK_DEV float block_sum256(float v, float* sh) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  if (l == 0) sh[w] = v;
  __syncthreads();
  float t = 0.f;
  if (threadIdx.x < 64) {
    t = threadIdx.x < (blockDim.x >> 6) ? sh[threadIdx.x] : 0.f;
    t = wave_sum(t);
    if (threadIdx.x == 0) sh[0] = t;
  }
  __syncthreads();
  t = sh[0];
  __syncthreads();
  return t;
}

// rmsnorm (src/ops/rmsnorm.rs:25-50): rms = sqrt(sum(x^2)/dim + eps); y = (x*w)/rms.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* in, const float* w, int dim, float eps, float* out) {
#pragma clang fp contract(off)
  __shared__ float sh[8];
  const float* x = in + (size_t)blockIdx.x * dim;
  float* y = out + (size_t)blockIdx.x * dim;
  float ss = 0.f;
  for (int i = threadIdx.x; i < dim; i += blockDim.x) ss += x[i] * x[i];
  ss = block_sum256(ss, sh);
  const float rms = sqrtf(ss / (float)dim + eps);
  for (int i = threadIdx.x; i < dim; i += blockDim.x) y[i] = (x[i] * w[i]) / rms;
}

void launch_rmsnorm(const float* in, const float* w, int rows, int dim, float eps, float* out, hipStream_t st) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, st, in, w, dim, eps, out);
}

// ---- GEMM inputs: fp16 pair planes and per-32 sums emitted by the producing kernel -----------
// Eight consecutive values v = a[8i .. 8i+7] of a [rows, K] input (K % 32 == 0): hi = fp16(v),
// lo = fp16(v - hi), and the per-32 sum of the block they belong to, summed in the order the
// stand-alone per-32 sum pass uses (eight float4 partials (x + y) + (z + w), left to right) and
// stored as an fp16 pair. The four consecutive lanes of one block exchange their partials by
// shuffles, so every lane of the wave calls this (`live` masks the stores).
// A value or per-32 sum beyond fp16's range (|x| > 65504: its pair would not hold it) sets *ovf;
// the prefill then runs again on f32 activations (Session::prefill).
IEK_DEV void emit_split8(const float (&v)[8], size_t i, bool live, uint4* __restrict__ hi, uint4* __restrict__ lo,
                         _Float16* __restrict__ sh, _Float16* __restrict__ sl, int* __restrict__ ovf) {
#pragma clang fp contract(off)
  _Float16 h[8], l[8];
  bool big = false;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    h[k] = (_Float16)v[k];
    l[k] = (_Float16)(v[k] - (float)h[k]);
    big |= fabsf(v[k]) > F16_PAIR_MAX;
  }
  auto pk = [](_Float16 a, _Float16 b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
  };
  if (live) {
    hi[i] = make_uint4(pk(h[0], h[1]), pk(h[2], h[3]), pk(h[4], h[5]), pk(h[6], h[7]));
    lo[i] = make_uint4(pk(l[0], l[1]), pk(l[2], l[3]), pk(l[4], l[5]), pk(l[6], l[7]));
  }
  const float pa = (v[0] + v[1]) + (v[2] + v[3]), pb = (v[4] + v[5]) + (v[6] + v[7]);
  const int lane = threadIdx.x & 63, base = lane & ~3;
  float p[8];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    p[2 * q] = __shfl(pa, base + q, 64);
    p[2 * q + 1] = __shfl(pb, base + q, 64);
  }
  if (live && (lane & 3) == 0) {
    float sum = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) sum += p[t];
    const _Float16 s16 = (_Float16)sum;
    sh[i / 4] = s16;
    sl[i / 4] = (_Float16)(sum - (float)s16);
    big |= fabsf(sum) > F16_PAIR_MAX;
  }
  if (live && big && ovf) *ovf = 1;
}

// rmsnorm (as rmsnorm_kernel) that also emits the GEMM input planes of its output (the f32 output
// itself only when `out` is set).
// With `part` the row is in + part (one f32 add per element, as the split-K add pass would do),
// written back to `in`. Each thread keeps its chunks of eight (chunk t, t + 256, ...; CPT of them)
// in registers between the sum of squares and the scaling, so the row is read once.
template <int CPT>
__global__ __launch_bounds__(256) void rmsnorm_split_kernel(float* in, const float* w, int dim, float eps,
                                                            float* out, uint4* hi, uint4* lo, _Float16* sh,
                                                            _Float16* sl, const float* part, int* ovf) {
#pragma clang fp contract(off)
  __shared__ float red[8];
  float* x = in + (size_t)blockIdx.x * dim;
  const float* pr = part ? part + (size_t)blockIdx.x * dim : nullptr;
  float* y = out + (size_t)blockIdx.x * dim;
  const int n8 = dim / 8;
  float4 xv[CPT][2];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int e = 256 * k + threadIdx.x;
    const int c = e < n8 ? e : 0;
    float4 xa = reinterpret_cast<const float4*>(x)[2 * c], xb = reinterpret_cast<const float4*>(x)[2 * c + 1];
    if (pr) {
      const float4 pa = reinterpret_cast<const float4*>(pr)[2 * c], pb = reinterpret_cast<const float4*>(pr)[2 * c + 1];
      xa.x += pa.x;
      xa.y += pa.y;
      xa.z += pa.z;
      xa.w += pa.w;
      xb.x += pb.x;
      xb.y += pb.y;
      xb.z += pb.z;
      xb.w += pb.w;
    }
    xv[k][0] = xa;
    xv[k][1] = xb;
    if (e < n8)
      ss += (((xa.x * xa.x + xa.y * xa.y) + (xa.z * xa.z + xa.w * xa.w)) +
             ((xb.x * xb.x + xb.y * xb.y) + (xb.z * xb.z + xb.w * xb.w)));
  }
  ss = block_sum256(ss, red);  // every read of the row is done
  const float rms = sqrtf(ss / (float)dim + eps);
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int e = 256 * k + threadIdx.x;
    const bool live = e < n8;
    const int c = live ? e : 0;
    const float4 xa = xv[k][0], xb = xv[k][1];
    if (pr && live) {
      reinterpret_cast<float4*>(x)[2 * c] = xa;
      reinterpret_cast<float4*>(x)[2 * c + 1] = xb;
    }
    const float4 wa = reinterpret_cast<const float4*>(w)[2 * c], wb = reinterpret_cast<const float4*>(w)[2 * c + 1];
    float v[8];
    v[0] = (xa.x * wa.x) / rms;
    v[1] = (xa.y * wa.y) / rms;
    v[2] = (xa.z * wa.z) / rms;
    v[3] = (xa.w * wa.w) / rms;
    v[4] = (xb.x * wb.x) / rms;
    v[5] = (xb.y * wb.y) / rms;
    v[6] = (xb.z * wb.z) / rms;
    v[7] = (xb.w * wb.w) / rms;
    if (live && out) {
      reinterpret_cast<float4*>(y)[2 * c] = make_float4(v[0], v[1], v[2], v[3]);
      reinterpret_cast<float4*>(y)[2 * c + 1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    // emit_split8 exchanges across the group of four lanes: every lane joins
    emit_split8(v, (size_t)blockIdx.x * n8 + c, live, hi, lo, sh, sl, ovf);
  }
}

void launch_rmsnorm_split(float* in, const float* w, int rows, int dim, float eps, float* out, __half* hi,
                          __half* lo, float* sums, int* ovf, hipStream_t st, const float* part) {
  if (rows <= 0) return;
  if (dim % 32 != 0 || (reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(out) |
                        reinterpret_cast<uintptr_t>(part)) % 16)
    fail(ST_OP, "rmsnorm_split: dim % 32 and 16-byte aligned rows");
  _Float16* s = reinterpret_cast<_Float16*>(sums);
  const size_t nb = (size_t)rows * (dim / 32);
  const int cpt = (dim / 8 + 255) / 256;  // chunks of eight per thread
#define IEK_RS(C)                                                                                                   \
  hipLaunchKernelGGL(rmsnorm_split_kernel<C>, dim3(rows), dim3(256), 0, st, in, w, dim, eps, out, (uint4*)hi,      \
                     (uint4*)lo, s, s + nb, part, ovf)
  if (cpt <= 1) IEK_RS(1);
  else if (cpt <= 2) IEK_RS(2);
  else if (cpt <= 4) IEK_RS(4);
  else if (cpt <= 8) IEK_RS(8);
  else fail(ST_OP, "rmsnorm_split: rows wider than 16384");
#undef IEK_RS
}

// fp16 pair planes and per-32 sums of an existing [rows, K] input in one pass.
__global__ __launch_bounds__(256) void split_sums_kernel(const float* __restrict__ a, size_t n8, uint4* hi, uint4* lo,
                                                         _Float16* sh, _Float16* sl, int* ovf) {
  for (size_t i0 = (size_t)blockIdx.x * 256; i0 < n8; i0 += (size_t)gridDim.x * 256) {
    const size_t i = i0 + threadIdx.x;
    const bool live = i < n8;
    const size_t c = live ? i : 0;
    const float4 xa = reinterpret_cast<const float4*>(a)[2 * c], xb = reinterpret_cast<const float4*>(a)[2 * c + 1];
    const float v[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    emit_split8(v, c, live, hi, lo, sh, sl, ovf);
  }
}

void launch_split_sums(const float* a, int rows, int K, __half* hi, __half* lo, float* sums, int* ovf,
                       hipStream_t st) {
  if (rows <= 0) return;
  if (K % 32 != 0 || reinterpret_cast<uintptr_t>(a) % 16) fail(ST_OP, "split_sums: K % 32 and 16-byte aligned input");
  const size_t n8 = (size_t)rows * (K / 8), nb = n8 / 4;
  _Float16* s = reinterpret_cast<_Float16*>(sums);
  const int blocks = (int)std::min<size_t>((n8 + 255) / 256, 4096);
  hipLaunchKernelGGL(split_sums_kernel, dim3(blocks), dim3(256), 0, st, a, n8, (uint4*)hi, (uint4*)lo, s, s + nb, ovf);
}

// *ovf = 1 when some |a[i]| exceeds the fp16 pair's range (NaN does not count: it stays NaN on
// either path).
__global__ __launch_bounds__(256) void range_flag_kernel(const float* __restrict__ a, size_t n, int* ovf) {
  bool big = false;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    big |= fabsf(a[i]) > F16_PAIR_MAX;
  if (big) *ovf = 1;
}

void launch_range_flag(const float* a, size_t n, int* ovf, hipStream_t st) {
  if (n == 0 || !ovf) return;
  const int blocks = (int)std::min<size_t>((n + 255) / 256, 2048);
  hipLaunchKernelGGL(range_flag_kernel, dim3(blocks), dim3(256), 0, st, a, n, ovf);
}

// Per-row scaled GEMM input (op level): one workgroup per row. Pass 1 finds the row's largest
// |value| and |per-32 sum| (sums in the order of block_sums_kernel: (x + y) + (z + w) per float4,
// left to right); the factor s = 2^e (e <= 0) brings that maximum below 2^15 when it is not
// already; pass 2 writes the fp16 (hi, lo) planes of s * a and s * sum (exact: a power of two).
__global__ __launch_bounds__(256) void split_scaled_kernel(const float* __restrict__ a, int K, _Float16* __restrict__ hi,
                                                           _Float16* __restrict__ lo, _Float16* __restrict__ sh,
                                                           _Float16* __restrict__ sl, size_t nb_total,
                                                           float* __restrict__ inv) {
#pragma clang fp contract(off)
  __shared__ float red[8];
  const int r = blockIdx.x, nb = K / 32;
  const float* x = a + (size_t)r * K;
  auto bsum = [&](int b) {
    const float4* p = reinterpret_cast<const float4*>(x + 32 * b);
    float s = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float4 v = p[t];
      s += (v.x + v.y) + (v.z + v.w);
    }
    return s;
  };
  float m = 0.f;
  for (int b = threadIdx.x; b < nb; b += 256) {
    const float4* p = reinterpret_cast<const float4*>(x + 32 * b);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float4 v = p[t];
      m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    m = fmaxf(m, fabsf(bsum(b)));
  }
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  // s = 2^(14 - floor(log2 m)) when m >= 2^15 (finite), else 1
  float scale = 1.f;
  if (m >= 32768.f && m <= 3.4028235e38f) {
    const int e = (int)((__float_as_uint(m) >> 23) & 0xFF) - 127;  // floor(log2 m) for a normal m
    scale = __uint_as_float((uint32_t)(127 + 14 - e) << 23);
  }
  if (threadIdx.x == 0) inv[r] = 1.f / scale;
  for (int i = threadIdx.x; i < K; i += 256) {
    const float v = x[i] * scale;
    const _Float16 h = (_Float16)v;
    hi[(size_t)r * K + i] = h;
    lo[(size_t)r * K + i] = (_Float16)(v - (float)h);
  }
  for (int b = threadIdx.x; b < nb; b += 256) {
    const float v = bsum(b) * scale;
    const _Float16 h = (_Float16)v;
    sh[(size_t)r * nb + b] = h;
    sl[(size_t)r * nb + b] = (_Float16)(v - (float)h);
  }
  (void)nb_total;
}

void launch_split_scaled(const float* a, int rows, int K, __half* hi, __half* lo, float* sums, float* inv,
                         hipStream_t st) {
  if (rows <= 0) return;
  if (K % 32 != 0 || reinterpret_cast<uintptr_t>(a) % 16) fail(ST_OP, "split_scaled: K % 32 and 16-byte aligned rows");
  const size_t nb = (size_t)rows * (K / 32);
  _Float16* s = reinterpret_cast<_Float16*>(sums);
  hipLaunchKernelGGL(split_scaled_kernel, dim3(rows), dim3(256), 0, st, a, K, reinterpret_cast<_Float16*>(hi),
                     reinterpret_cast<_Float16*>(lo), s, s + nb, nb, inv);
}

__global__ void row_scale_kernel(float* __restrict__ out, int N, const float* __restrict__ inv) {
  const float f = inv[blockIdx.y];
  if (f == 1.f) return;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < N; i += gridDim.x * 256) out[(size_t)blockIdx.y * N + i] *= f;
}

void launch_row_scale(float* out, int rows, int N, const float* inv, hipStream_t st) {
  if (rows <= 0 || N <= 0) return;
  hipLaunchKernelGGL(row_scale_kernel, dim3((unsigned)std::min((N + 255) / 256, 64), rows), dim3(256), 0, st, out, N,
                     inv);
}

// RoPE on adjacent pairs (src/ops/rope.rs:11-59). `cs` holds (cos, sin) per (position, pair),
// built on the host with the reference's f32 running-product angles and libm cosf/sinf.
IEK_DEV void rotate(float* v, int p, float c, float s) {
#pragma clang fp contract(off)
  float t0 = v[p], t1 = v[p + 1];
  v[p] = t0 * c - t1 * s;
  v[p + 1] = t0 * s + t1 * c;
}

__global__ void rope_rows_kernel(float* v, int rows, int row_stride, int n_heads, int head_dim, int pos0,
                                 const float* cs, int npairs) {
  const size_t total = (size_t)rows * n_heads * npairs;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int k = (int)(i % npairs);
  const int h = (int)((i / npairs) % n_heads);
  const int r = (int)(i / ((size_t)npairs * n_heads));
  const float* e = cs + ((size_t)(pos0 + r) * npairs + k) * 2;
  rotate(v + (size_t)r * row_stride + (size_t)h * head_dim, 2 * k, e[0], e[1]);
}

void launch_rope_rows(float* v, int rows, int row_stride, int n_heads, int head_dim, int pos0, const float* cs,
                      int npairs, hipStream_t st) {
  size_t total = (size_t)rows * n_heads * npairs;
  if (total == 0) return;
  hipLaunchKernelGGL(rope_rows_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, v, rows, row_stride,
                     n_heads, head_dim, pos0, cs, npairs);
}

// Decode-step RoPE: position read from device memory.
__global__ void rope_dev_kernel(float* v, int n_heads, int head_dim, int npairs, const float* cs, const int* pos_dev) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_heads * npairs) return;
  const int k = i % npairs, h = i / npairs;
  const float* e = cs + ((size_t)(*pos_dev) * npairs + k) * 2;
  rotate(v + (size_t)h * head_dim, 2 * k, e[0], e[1]);
}

void launch_rope_table(float* v, int n_heads, int head_dim, int npairs, const float* cs, const int* pos_dev,
                       hipStream_t st) {
  int total = n_heads * npairs;
  if (total == 0) return;
  hipLaunchKernelGGL(rope_dev_kernel, dim3((total + 255) / 256), dim3(256), 0, st, v, n_heads, head_dim, npairs, cs,
                     pos_dev);
}

// KV append: rows [r] of k/v ([rows][kv_dim], f32) go to cache position (pos + r) as fp16.
// Cache layout per layer: [n_kv][ctx][head_dim], so one head's keys are one contiguous stream.
template <typename T>
__global__ void kv_store_kernel(const float* k, const float* v, int rows, int kv_dim, T* kc, T* vc, int head_dim,
                                int ctx, const int* pos_dev, int pos0) {
  const size_t total = (size_t)rows * kv_dim;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int r = (int)(i / kv_dim), c = (int)(i % kv_dim);
  const int h = c / head_dim, d = c % head_dim;
  const int pos = (pos_dev ? *pos_dev : pos0) + r;
  const size_t dst = ((size_t)h * ctx + pos) * head_dim + d;
  if constexpr (std::is_same<T, float>::value) {
    kc[dst] = k[i];
    vc[dst] = v[i];
  } else {
    kc[dst] = __float2half_rn(k[i]);
    vc[dst] = __float2half_rn(v[i]);
  }
}

void launch_kv_store(const float* k, const float* v, int rows, int kv_dim, void* kc, void* vc, bool kv_f32, int n_kv,
                     int head_dim, int ctx, const int* pos_dev, int pos0, hipStream_t st) {
  (void)n_kv;
  size_t total = (size_t)rows * kv_dim;
  if (total == 0) return;
  const dim3 grid((unsigned)((total + 255) / 256));
  if (kv_f32)
    hipLaunchKernelGGL(kv_store_kernel<float>, grid, dim3(256), 0, st, k, v, rows, kv_dim, (float*)kc, (float*)vc,
                       head_dim, ctx, pos_dev, pos0);
  else
    hipLaunchKernelGGL(kv_store_kernel<__half>, grid, dim3(256), 0, st, k, v, rows, kv_dim, (__half*)kc, (__half*)vc,
                       head_dim, ctx, pos_dev, pos0);
}

// swiglu (src/ops/swiglu.rs:24-36): out = (g * sigmoid(g)) * u, two-branch stable sigmoid.
__global__ void swiglu_kernel(const float* g, const float* u, float* out, size_t n) {
#pragma clang fp contract(off)
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float x = g[i], s;
  if (x >= 0.0f) {
    float z = expf(-x);
    s = 1.0f / (1.0f + z);
  } else {
    float z = expf(x);
    s = z / (1.0f + z);
  }
  out[i] = x * s * u[i];
}

void launch_swiglu(const float* g, const float* u, float* out, size_t n, hipStream_t st) {
  if (n == 0) return;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, u, out, n);
}

// swiglu (as swiglu_kernel) over a [rows, K] input that also emits the GEMM input planes (the f32
// output itself only when `out` is set).
__global__ __launch_bounds__(256) void swiglu_split_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                           float* __restrict__ out, size_t n8, uint4* hi, uint4* lo,
                                                           _Float16* sh, _Float16* sl, int* ovf) {
#pragma clang fp contract(off)
  for (size_t i0 = (size_t)blockIdx.x * 256; i0 < n8; i0 += (size_t)gridDim.x * 256) {
    const size_t i = i0 + threadIdx.x;
    const bool live = i < n8;
    const size_t c = live ? i : 0;
    const float4 ga = reinterpret_cast<const float4*>(g)[2 * c], gb = reinterpret_cast<const float4*>(g)[2 * c + 1];
    const float4 ua = reinterpret_cast<const float4*>(u)[2 * c], ub = reinterpret_cast<const float4*>(u)[2 * c + 1];
    const float gx[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
    const float ux[8] = {ua.x, ua.y, ua.z, ua.w, ub.x, ub.y, ub.z, ub.w};
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float x = gx[k];
      float sg;
      if (x >= 0.0f) {
        const float z = expf(-x);
        sg = 1.0f / (1.0f + z);
      } else {
        const float z = expf(x);
        sg = z / (1.0f + z);
      }
      v[k] = x * sg * ux[k];
    }
    if (live && out) {
      reinterpret_cast<float4*>(out)[2 * c] = make_float4(v[0], v[1], v[2], v[3]);
      reinterpret_cast<float4*>(out)[2 * c + 1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    emit_split8(v, c, live, hi, lo, sh, sl, ovf);
  }
}

void launch_swiglu_split(const float* g, const float* u, float* out, int rows, int K, __half* hi, __half* lo,
                         float* sums, int* ovf, hipStream_t st) {
  if (rows <= 0) return;
  if (K % 32 != 0 || (reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(u) | reinterpret_cast<uintptr_t>(out)) % 16)
    fail(ST_OP, "swiglu_split: K % 32 and 16-byte aligned inputs");
  const size_t n8 = (size_t)rows * (K / 8), nb = n8 / 4;
  _Float16* s = reinterpret_cast<_Float16*>(sums);
  const int blocks = (int)std::min<size_t>((n8 + 255) / 256, 4096);
  hipLaunchKernelGGL(swiglu_split_kernel, dim3(blocks), dim3(256), 0, st, g, u, out, n8, (uint4*)hi, (uint4*)lo, s,
                     s + nb, ovf);
}

// gelu_tanh(g) * u (src/layers/ffn.rs:49-53); gelu_tanh_dev is in common.cuh.

__global__ void gelu_mul_kernel(const float* g, const float* u, float* out, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = u ? gelu_tanh_dev(g[i]) * u[i] : gelu_tanh_dev(g[i]);
}

void launch_gelu_mul(const float* g, const float* u, float* out, size_t n, hipStream_t st) {
  if (n == 0) return;
  hipLaunchKernelGGL(gelu_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, u, out, n);
}

__global__ void residual_add_kernel(const float* a, const float* b, float* out, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = a[i] + b[i];
}

void launch_residual_add(const float* a, const float* b, float* out, size_t n, hipStream_t st) {
  if (n == 0) return;
  hipLaunchKernelGGL(residual_add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a, b, out, n);
}

// softmax (src/ops/softmax.rs:3-28), one 256-thread block.
__global__ __launch_bounds__(256) void softmax_kernel(const float* in, float* out, int n) {
#pragma clang fp contract(off)
  __shared__ float sh[8];
  float m = -INFINITY;
  for (int i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, in[i]);
  m = wave_max(m);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  if (l == 0) sh[w] = m;
  __syncthreads();
  float mm = sh[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) mm = fmaxf(mm, sh[i]);
  __syncthreads();
  float s = 0.f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) s += expf(in[i] - mm);
  s = block_sum256(s, sh);
  for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = expf(in[i] - mm) / s;
}

void launch_softmax(const float* in, float* out, int n, hipStream_t st) {
  hipLaunchKernelGGL(softmax_kernel, dim3(1), dim3(256), 0, st, in, out, n);
}

// Greedy argmax (src/engine/sampling.rs:25-49): first index of the maximum; any non-finite logit
// raises a flag (the reference returns InvalidLogits). The (value, index) pair is packed into one
// u64 whose unsigned order is (value ascending, index descending), so a single atomicMax picks the
// first maximal index.
IEK_DEV unsigned long long argmax_key(float v, uint32_t idx) {
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}

__global__ __launch_bounds__(256) void argmax_kernel(const float* logits, int n, unsigned long long* key, int* flags,
                                                     const int* step) {
  unsigned long long best = 0;
  bool bad = false;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    float v = logits[i];
    if (!isfinite(v)) bad = true;
    unsigned long long k = argmax_key(v, (uint32_t)i);
    best = k > best ? k : best;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    unsigned long long o = __shfl_xor(best, off, WAVE);
    best = o > best ? o : best;
  }
  if ((threadIdx.x & 63) == 0) atomicMax(key, best);
  if (bad) atomicOr(&flags[step ? *step : 0], 1);
}

void launch_argmax(const float* logits, int n, unsigned long long* key_out, int* flags, const int* step, hipStream_t st) {
  int blocks = std::min(256, (n + 255) / 256);
  hipLaunchKernelGGL(argmax_kernel, dim3(blocks), dim3(256), 0, st, logits, n, key_out, flags, step);
}

// Publishes the chosen token: tok[0] feeds the next embedding gather; with a step counter the id
// and the non-finite flag are also appended to the per-step lists and the counter advances. The
// packed key and the flag are reset for the next LM-head launch.
__global__ void argmax_finish_kernel(unsigned long long* key, int* flag, uint32_t* tok, uint32_t* list, int* flags,
                                     int* step) {
  const unsigned long long k = *key;
  // every folded logit leaves a nonzero key; none (no logit reached the argmax) is an error, and
  // the published id stays a valid one
  uint32_t idx = k ? 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull) : 0u;
  tok[0] = idx;
  const int i = step ? *step : 0;
  flags[i] = k ? *flag : 1;
  if (step) {
    list[i] = idx;
    *step = i + 1;
  }
  *key = 0ull;
  *flag = 0;
}

void launch_argmax_finish(unsigned long long* key, int* flag, uint32_t* tok, uint32_t* list, int* flags, int* step,
                          hipStream_t st) {
  hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(1), 0, st, key, flag, tok, list, flags, step);
}

// Final-logit soft cap z -> cap * tanh(z / cap) (src/engine/runtime.rs:110-114).
__global__ void softcap_kernel(float* z, int n, float cap) {
#pragma clang fp contract(off)
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) z[i] = cap * tanhf(z[i] / cap);
}
void launch_softcap(float* z, int n, float cap, hipStream_t st) {
  hipLaunchKernelGGL(softcap_kernel, dim3((n + 255) / 256), dim3(256), 0, st, z, n, cap);
}

// Inverse HF->GGUF Q/K permutation on activation rows (src/layers/attention.rs:149-172):
// logical b*(d/2)+h <- stored h*2+b inside every head.
__global__ void unpack_qk_kernel(const float* src, float* dst, int rows, int row_stride, int n_groups, int head_dim) {
  const int half = head_dim / 2;
  size_t total = (size_t)rows * n_groups * head_dim;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  int e = (int)(i % head_dim);
  int g = (int)((i / head_dim) % n_groups);
  int r = (int)(i / ((size_t)head_dim * n_groups));
  int b = e / half, h = e % half;
  size_t base = (size_t)r * row_stride + (size_t)g * head_dim;
  dst[base + e] = src[base + h * 2 + b];
}
void launch_unpack_qk(const float* src, float* dst, int rows, int row_stride, int n_groups, int head_dim,
                      hipStream_t st) {
  size_t total = (size_t)rows * n_groups * head_dim;
  if (total == 0) return;
  hipLaunchKernelGGL(unpack_qk_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, src, dst, rows,
                     row_stride, n_groups, head_dim);
}

__global__ void copy_f32_kernel(const float* src, float* dst, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src[i];
}
void launch_copy_f32(const float* src, float* dst, size_t n, hipStream_t st) {
  if (n == 0) return;
  hipLaunchKernelGGL(copy_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, src, dst, n);
}

__global__ void fill_i32_kernel(int* p, int v, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}
void launch_fill_i32(int* p, int v, int n, hipStream_t st) {
  if (n <= 0) return;
  hipLaunchKernelGGL(fill_i32_kernel, dim3((n + 255) / 256), dim3(256), 0, st, p, v, n);
}

__global__ void fill_u64_kernel(unsigned long long* p, unsigned long long v, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}
void launch_fill_u64(unsigned long long* p, unsigned long long v, int n, hipStream_t st) {
  hipLaunchKernelGGL(fill_u64_kernel, dim3((n + 255) / 256), dim3(256), 0, st, p, v, n);
}
__global__ void set_int_kernel(int* p, int v) { *p = v; }
void launch_set_int(int* p, int v, hipStream_t st) { hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(1), 0, st, p, v); }
__global__ void add_int_kernel(int* p, int v) { *p += v; }
void launch_add_int(int* p, int v, hipStream_t st) { hipLaunchKernelGGL(add_int_kernel, dim3(1), dim3(1), 0, st, p, v); }

}  // namespace iek
