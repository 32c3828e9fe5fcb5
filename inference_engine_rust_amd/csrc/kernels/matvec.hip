// Decode matvec (M = 1): y[n] = sum_k x[k] * W(k, n) over weights kept in their native GGUF
// block layout (ggml order: element (k, n) at flat k + n*K, src/ops/matmul.rs:1-3).
//
// CDNA4 mapping. A 256-thread workgroup owns 4*R consecutive output rows (R per wave):
//  1. every lane issues the loads of its first quant chunk for all R rows;
//  2. while they fly, the workgroup stages x in LDS once, optionally fused with RMSNorm
//     (rms over the whole vector, y = (x*w)/rms as in src/ops/rmsnorm.rs:25-50);
//  3. lane l walks chunks c = l, l+64, ... of its rows with the next chunk's loads in flight,
//     dequantising in registers; per-sub-block scales are applied once per chunk:
//        sum_k x_k (d*sc*q_k - dmin*m) = (d*sc) * sum x_k q_k - (dmin*m) * sum x_k;
//  4. a wave butterfly leaves the R row sums in every lane; lanes 0..R-1 run the epilogue
//     (store, residual add, SwiGLU pair, RoPE + fp16 KV append, or logits + argmax).
// Weights are streamed exactly once per token as 16-byte coalesced loads; x never leaves LDS.
#include "common.cuh"
#include "mv_args.h"

namespace iek {

// (g * sigmoid(g)) * u, the reference's two-branch sigmoid (src/ops/swiglu.rs:3-36).
IEK_DEV float silu_mul(float g, float u) {
#pragma clang fp contract(off)
  float s;
  if (g >= 0.0f) {
    float z = expf(-g);
    s = 1.0f / (1.0f + z);
  } else {
    float z = expf(g);
    s = z / (1.0f + z);
  }
  return g * s * u;
}

// RoPE on one element of an adjacent pair (t0, t1) (src/ops/rope.rs:52-56), unfused f32 steps.
IEK_DEV float rope_rotate(float v, float partner, float c, float s, bool even) {
#pragma clang fp contract(off)
  return even ? v * c - partner * s : partner * s + v * c;
}

// cap * tanh(z / cap) (src/engine/runtime.rs:110-114).
IEK_DEV float soft_cap(float z, float cap) {
#pragma clang fp contract(off)
  return cap * tanhf(z / cap);
}

template <int I>
IEK_DEV float ubyte_f(uint32_t w) {
  return (float)((w >> (8 * I)) & 0xFFu);
}

IEK_DEV unsigned long long argmax_key_dev(float v, uint32_t idx) {
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}

// rms = sqrt(sum/dim + eps) and y = (x*w)/rms, each step rounded like src/ops/rmsnorm.rs:44-47.
IEK_DEV float rms_of(float sum_sq, int dim, float eps) {
#pragma clang fp contract(off)
  return sqrtf(sum_sq / (float)dim + eps);
}
IEK_DEV float norm_scale(float x, float w, float rms) {
#pragma clang fp contract(off)
  return (x * w) / rms;
}

// ---- prologue: x (optionally RMS-normalised) into LDS ----------------------------------------
IEK_DEV void stage_x(const MvArgs& a, float* xs) {
  const int K = a.K, tid = threadIdx.x;
  if (a.norm_w) {
    __shared__ float red[4];
    float ss = 0.f;
    for (int i = tid; i < K; i += 256) {
      float v = a.x[i];
      ss += v * v;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, WAVE);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float rms = rms_of(tot, K, a.eps);
    for (int i = tid; i < K; i += 256) xs[i] = norm_scale(a.x[i], a.norm_w[i], rms);
  } else {
    for (int i = tid; i < K; i += 256) xs[i] = a.x[i];
  }
  __syncthreads();
}

// ---- epilogue -----------------------------------------------------------------------------------
template <int R>
IEK_DEV void epilogue(const MvArgs& a, int s, int lr0, float (&acc)[R], const float* acc_up, int lane) {
  // The position counter is read by earlier launches of the step only, never by this one.
  if (a.pos_inc && blockIdx.x == 0 && threadIdx.x == 0) *a.pos_inc += 1;
  if (a.epi == EPI_SWIGLU) {
    if (lane < R) {
      float g = acc[0], u = acc_up[0];
#pragma unroll
      for (int r = 1; r < R; ++r)
        if (lane == r) {
          g = acc[r];
          u = acc_up[r];
        }
      a.out[0][lr0 + lane] = silu_mul(g, u);
    }
    return;
  }
  if (a.epi == EPI_QKV) {
    // Rows come in RoPE pairs (2k, 2k+1) of one head (R is even and rows start even).
    if (lane < R) {
      const int n = lr0 + lane;
      float v = acc[0], partner = acc[0];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (lane == r) v = acc[r];
        if ((lane ^ 1) == r) partner = acc[r];
      }
      const int hd = a.head_dim;
      const int d = n % hd;
      const int pos = *a.pos;
      if (s < 2 && d < 2 * a.npairs) {
        const float* e = a.rope_cs + ((size_t)pos * a.npairs + (d >> 1)) * 2;
        const float c = e[0], sn = e[1];
        v = rope_rotate(v, partner, c, sn, (d & 1) == 0);
      }
      if (s == 0) {
        a.out[0][n] = v;
      } else {
        const size_t dst = ((size_t)(n / hd) * a.ctx + pos) * hd + d;
        (s == 1 ? a.kc : a.vc)[dst] = __float2half_rn(v);
      }
    }
    return;
  }
  if (a.epi == EPI_ARGMAX) {
    float v = acc[0];
#pragma unroll
    for (int r = 1; r < R; ++r)
      if (lane == r) v = acc[r];
    if (a.softcap > 0.f) v = soft_cap(v, a.softcap);
    unsigned long long key = 0;
    bool bad = false;
    if (lane < R) {
      a.out[0][lr0 + lane] = v;
      key = argmax_key_dev(v, (uint32_t)(lr0 + lane));
      bad = !isfinite(v);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      unsigned long long o = __shfl_xor(key, off, WAVE);
      key = o > key ? o : key;
    }
    if (lane == 0) atomicMax(a.amax_key, key);
    if (bad) atomicOr(a.amax_flag, 1);
    return;
  }
  if (lane < R) {
    float v = acc[0];
#pragma unroll
    for (int r = 1; r < R; ++r)
      if (lane == r) v = acc[r];
    const int n = lr0 + lane;
    if (a.epi == EPI_RESID) v = a.resid[n] + v;
    a.out[s][n] = v;
  }
}

template <int R>
IEK_DEV void wave_reduce(float (&acc)[R]) {
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
}

// ---- Q4_K -----------------------------------------------------------------------------------
// Chunk j (0..7) of a superblock = qs bytes [16j, 16j+16): 16 low nibbles of sub-block 2g and 16
// high nibbles of sub-block 2g+1 (g = j/2), i.e. elements 64g+16h+t and 64g+32+16h+t, h = j&1.
IEK_DEV float q4k_dot(uint4 hdr, uint4 qv, int j, const float4* xl4, const float4* xh4, float xsl, float xsh) {
  const int g = j >> 1;
  float d = half_bits_to_float(hdr.x), dmin = half_bits_to_float(hdr.x >> 16);
  float sc0, m0, sc1, m1;
  scale_min_k4(2 * g, hdr.y, hdr.z, hdr.w, &sc0, &m0);
  scale_min_k4(2 * g + 1, hdr.y, hdr.z, hdr.w, &sc1, &m1);
  const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
  float sl = 0.f, sh = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t lo = qw[t] & 0x0F0F0F0Fu, hi = (qw[t] >> 4) & 0x0F0F0F0Fu;
    const float4 a = xl4[t], b = xh4[t];
    sl += a.x * ubyte_f<0>(lo) + a.y * ubyte_f<1>(lo) + a.z * ubyte_f<2>(lo) + a.w * ubyte_f<3>(lo);
    sh += b.x * ubyte_f<0>(hi) + b.y * ubyte_f<1>(hi) + b.z * ubyte_f<2>(hi) + b.w * ubyte_f<3>(hi);
  }
  return (d * sc0) * sl - (dmin * m0) * xsl + (d * sc1) * sh - (dmin * m1) * xsh;
}

template <int R, bool DUAL>
__global__ __launch_bounds__(256) void mv_q4k(MvArgs a) {
  extern __shared__ float xs[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * 4 + wave) * R;
  const int total = a.seg_start[a.nseg];
  const bool active = row0 < total;
  const int s = active ? seg_of(a, row0) : 0;
  const int lr0 = row0 - a.seg_start[s];
  const int K = a.K;
  const size_t rb = (size_t)(K / QK_K) * Q4K_BYTES;
  const int nchunk = (K / QK_K) * 8;
  const uint8_t* W0 = a.w[s] + (size_t)lr0 * rb;
  const uint8_t* W1 = DUAL ? a.w[1] + (size_t)lr0 * rb : nullptr;
  constexpr int NR = DUAL ? 2 * R : R;
  auto rowp = [&](int r) { return r < R ? W0 + (size_t)r * rb : W1 + (size_t)(r - R) * rb; };

  uint4 hdr[NR], qv[NR];
  int c = lane;
  if (active && c < nchunk) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const uint8_t* blk = rowp(r) + (size_t)(c >> 3) * Q4K_BYTES;
      hdr[r] = *reinterpret_cast<const uint4*>(blk);
      qv[r] = *reinterpret_cast<const uint4*>(blk + 16 + 16 * (c & 7));
    }
  }
  stage_x(a, xs);
  if (!active) return;

  float acc[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = 0.f;
  for (; c < nchunk; c += WAVE) {
    const int cn = c + WAVE;
    uint4 hdr_n[NR], qv_n[NR];
    if (cn < nchunk) {
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const uint8_t* blk = rowp(r) + (size_t)(cn >> 3) * Q4K_BYTES;
        hdr_n[r] = *reinterpret_cast<const uint4*>(blk);
        qv_n[r] = *reinterpret_cast<const uint4*>(blk + 16 + 16 * (cn & 7));
      }
    }
    const int b = c >> 3, j = c & 7;
    const int e0 = b * QK_K + (j >> 1) * 64 + (j & 1) * 16;
    const float4* xl4 = reinterpret_cast<const float4*>(xs + e0);
    const float4* xh4 = reinterpret_cast<const float4*>(xs + e0 + 32);
    float xsl = 0.f, xsh = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float4 u = xl4[t], v = xh4[t];
      xsl += (u.x + u.y) + (u.z + u.w);
      xsh += (v.x + v.y) + (v.z + v.w);
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] += q4k_dot(hdr[r], qv[r], j, xl4, xh4, xsl, xsh);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      hdr[r] = hdr_n[r];
      qv[r] = qv_n[r];
    }
  }
  float accg[R], accu[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    accg[r] = acc[r];
    accu[r] = DUAL ? acc[R + r] : 0.f;
  }
  wave_reduce<R>(accg);
  if (DUAL) wave_reduce<R>(accu);
  epilogue<R>(a, s, lr0, accg, accu, lane);
}

// ---- Q6_K -----------------------------------------------------------------------------------
// Chunk (h, o8): l = 8*o8..8*o8+7 of half h, all four quarters (32 values). The 210-byte
// superblocks are only 2-byte aligned, so 8-byte fields are read as aligned dword triples and
// re-sliced with v_alignbyte.
struct Q6Raw {
  uint32_t a[3], b[3], h[3], s[3];
  uint32_t d, sh_ql, sh_s;
};

// Three dwords from the aligned address at or below p (the third only when the 8-byte field
// crosses into it), so reads never leave the superblock.
IEK_DEV void load_tri(const uint8_t* p, uint32_t (&o)[3], uint32_t* shift) {
  const uintptr_t ap = reinterpret_cast<uintptr_t>(p);
  const uint32_t* base = reinterpret_cast<const uint32_t*>(ap & ~uintptr_t(3));
  *shift = (uint32_t)(ap & 3u);
  o[0] = base[0];
  o[1] = base[1];
  o[2] = *shift ? base[2] : 0u;
}

IEK_DEV void q6_load(const uint8_t* blk, int h, int o8, Q6Raw& q) {
  uint32_t sh;
  load_tri(blk + 64 * h + 8 * o8, q.a, &q.sh_ql);
  load_tri(blk + 64 * h + 32 + 8 * o8, q.b, &sh);
  load_tri(blk + 128 + 32 * h + 8 * o8, q.h, &sh);
  // scale window: bytes 192 + 8h + o8/2 + {0, 2, 4, 6}; a 7-byte span needs the third dword only
  // when the window starts at offset 2 or 3 of its dword.
  const uintptr_t ap = reinterpret_cast<uintptr_t>(blk + 192 + 8 * h + (o8 >> 1));
  const uint32_t* base = reinterpret_cast<const uint32_t*>(ap & ~uintptr_t(3));
  q.sh_s = (uint32_t)(ap & 3u);
  q.s[0] = base[0];
  q.s[1] = base[1];
  q.s[2] = q.sh_s >= 2 ? base[2] : 0u;
  q.d = *reinterpret_cast<const uint16_t*>(blk + 208);
}

IEK_DEV float q6k_dot(const Q6Raw& q, const float4* x4, const float (&xs4)[4]) {
  const uint32_t sh_ql = q.sh_ql, sh_s = q.sh_s;
  const uint32_t A[2] = {__builtin_amdgcn_alignbyte(q.a[1], q.a[0], sh_ql), __builtin_amdgcn_alignbyte(q.a[2], q.a[1], sh_ql)};
  const uint32_t B[2] = {__builtin_amdgcn_alignbyte(q.b[1], q.b[0], sh_ql), __builtin_amdgcn_alignbyte(q.b[2], q.b[1], sh_ql)};
  const uint32_t H[2] = {__builtin_amdgcn_alignbyte(q.h[1], q.h[0], sh_ql), __builtin_amdgcn_alignbyte(q.h[2], q.h[1], sh_ql)};
  const uint32_t S0 = __builtin_amdgcn_alignbyte(q.s[1], q.s[0], sh_s), S1 = __builtin_amdgcn_alignbyte(q.s[2], q.s[1], sh_s);
  // scales for the four quarters sit at window bytes 0, 2, 4, 6
  const float sc[4] = {(float)(int8_t)(S0 & 0xFF), (float)(int8_t)((S0 >> 16) & 0xFF), (float)(int8_t)(S1 & 0xFF),
                       (float)(int8_t)((S1 >> 16) & 0xFF)};
  const float d = half_bits_to_float(q.d);
  float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const uint32_t qq[4] = {(A[t] & 0x0F0F0F0Fu) | ((H[t] << 4) & 0x30303030u),
                            (B[t] & 0x0F0F0F0Fu) | ((H[t] << 2) & 0x30303030u),
                            ((A[t] >> 4) & 0x0F0F0F0Fu) | (H[t] & 0x30303030u),
                            ((B[t] >> 4) & 0x0F0F0F0Fu) | ((H[t] >> 2) & 0x30303030u)};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 xv = x4[2 * i + t];
      s[i] += xv.x * ubyte_f<0>(qq[i]) + xv.y * ubyte_f<1>(qq[i]) + xv.z * ubyte_f<2>(qq[i]) +
              xv.w * ubyte_f<3>(qq[i]);
    }
  }
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) r += (d * sc[i]) * (s[i] - 32.0f * xs4[i]);
  return r;
}

template <int R, bool DUAL>
__global__ __launch_bounds__(256) void mv_q6k(MvArgs a) {
  extern __shared__ float xs[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * 4 + wave) * R;
  const int total = a.seg_start[a.nseg];
  const bool active = row0 < total;
  const int s = active ? seg_of(a, row0) : 0;
  const int lr0 = row0 - a.seg_start[s];
  const int K = a.K;
  const size_t rb = (size_t)(K / QK_K) * Q6K_BYTES;
  const int nchunk = (K / QK_K) * 8;
  const uint8_t* W0 = a.w[s] + (size_t)lr0 * rb;
  const uint8_t* W1 = DUAL ? a.w[1] + (size_t)lr0 * rb : nullptr;
  constexpr int NR = DUAL ? 2 * R : R;
  auto rowp = [&](int r) { return r < R ? W0 + (size_t)r * rb : W1 + (size_t)(r - R) * rb; };

  Q6Raw q[NR];
  int c = lane;
  if (active && c < nchunk) {
#pragma unroll
    for (int r = 0; r < NR; ++r) q6_load(rowp(r) + (size_t)(c >> 3) * Q6K_BYTES, (c >> 2) & 1, c & 3, q[r]);
  }
  stage_x(a, xs);
  if (!active) return;

  float acc[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = 0.f;
  for (; c < nchunk; c += WAVE) {
    const int cn = c + WAVE;
    Q6Raw qn[NR];
    if (cn < nchunk) {
#pragma unroll
      for (int r = 0; r < NR; ++r) q6_load(rowp(r) + (size_t)(cn >> 3) * Q6K_BYTES, (cn >> 2) & 1, cn & 3, qn[r]);
    }
    const int e0 = (c >> 3) * QK_K + 128 * ((c >> 2) & 1) + 8 * (c & 3);
    float4 x4[8];
    float xs4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x4[2 * i] = *reinterpret_cast<const float4*>(xs + e0 + 32 * i);
      x4[2 * i + 1] = *reinterpret_cast<const float4*>(xs + e0 + 32 * i + 4);
      const float4 u = x4[2 * i], v = x4[2 * i + 1];
      xs4[i] = ((u.x + u.y) + (u.z + u.w)) + ((v.x + v.y) + (v.z + v.w));
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] += q6k_dot(q[r], x4, xs4);
#pragma unroll
    for (int r = 0; r < NR; ++r) q[r] = qn[r];
  }
  float accg[R], accu[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    accg[r] = acc[r];
    accu[r] = DUAL ? acc[R + r] : 0.f;
  }
  wave_reduce<R>(accg);
  if (DUAL) wave_reduce<R>(accu);
  epilogue<R>(a, s, lr0, accg, accu, lane);
}

// ---- generic path: any dtype, any K (blocks may straddle rows when K % block != 0) ----------
__global__ __launch_bounds__(256) void mv_generic(MvArgs a, int dt) {
  extern __shared__ float xs[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.x * 4 + wave;
  stage_x(a, xs);
  const int total = a.seg_start[a.nseg];
  if (row >= total) return;
  const int s = seg_of(a, row);
  const int n = row - a.seg_start[s];
  const bool dual = a.epi == EPI_SWIGLU;
  const int K = a.K;
  float g = 0.f, u = 0.f;
  for (int k = lane; k < K; k += WAVE) {
    const float xv = xs[k];
    const size_t f = (size_t)k + (size_t)n * (size_t)K;
    g += xv * flat_elem(dt, a.w[s], f);
    if (dual) u += xv * flat_elem(dt, a.w[1], f);
  }
  float acc[1] = {wave_sum(g)};
  float accu[1] = {dual ? wave_sum(u) : 0.f};
  epilogue<1>(a, s, n, acc, accu, lane);
}

// ---------------------------------------------------------------------------------------------
void launch_mv(int dt, MvArgs a, hipStream_t st) {
  int total = 0;
  for (int i = 0; i < a.nseg; ++i) {
    a.seg_start[i] = total;
    total += a.n[i];
  }
  a.seg_start[a.nseg] = total;
  const bool dual = a.epi == EPI_SWIGLU;
  if (dual) {
    // the row space is the gate rows; the up weight rides along as w[1]
    a.seg_start[1] = a.n[0];
    a.nseg = 1;
    total = a.n[0];
  }
  bool fast = (dt == DT_Q4K || dt == DT_Q6K) && a.K % QK_K == 0 && (reinterpret_cast<uintptr_t>(a.x) % 16) == 0;
  for (int i = 0; i < (dual ? 2 : a.nseg); ++i) fast = fast && (reinterpret_cast<uintptr_t>(a.w[i]) % 16) == 0;
  const size_t lds = (size_t)a.K * sizeof(float);
  if (lds > 160 * 1024) fail(ST_OP, "matvec: K too large for the LDS-staged input");
  if (fast) {
    int R = dual ? 2 : (total >= 16384 ? 4 : 2);
    bool ok = true;
    for (int i = 0; i < a.nseg; ++i) ok = ok && a.n[i] % R == 0;
    if (!ok) R = 2;
    ok = true;
    for (int i = 0; i < a.nseg; ++i) ok = ok && a.n[i] % R == 0;
    if (!ok) fast = false;
    if (fast) {
      const int blocks = (total + 4 * R - 1) / (4 * R);
#define IEK_L(KER, RR, DD) hipLaunchKernelGGL((KER<RR, DD>), dim3(blocks), dim3(256), lds, st, a)
      if (dt == DT_Q4K) {
        if (dual) IEK_L(mv_q4k, 2, true);
        else if (R == 4) IEK_L(mv_q4k, 4, false);
        else IEK_L(mv_q4k, 2, false);
      } else {
        if (dual) IEK_L(mv_q6k, 2, true);
        else if (R == 4) IEK_L(mv_q6k, 4, false);
        else IEK_L(mv_q6k, 2, false);
      }
#undef IEK_L
      return;
    }
  }
  if (a.epi == EPI_QKV) fail(ST_OP, "matvec: fused Q/K/V epilogue needs the aligned K-quant path");
  hipLaunchKernelGGL(mv_generic, dim3((total + 3) / 4), dim3(256), lds, st, a, dt);
}

void launch_matvec(int dt, const MvSegDesc* segs, int nseg, const float* x, int K, int epi, hipStream_t st) {
  MvArgs a{};
  a.nseg = nseg;
  for (int i = 0; i < nseg; ++i) {
    a.w[i] = (const uint8_t*)segs[i].w;
    a.out[i] = segs[i].out;
    a.n[i] = segs[i].n;
  }
  a.resid = segs[0].resid;
  a.x = x;
  a.K = K;
  a.epi = epi;
  launch_mv(dt, a, st);
}

}  // namespace iek
