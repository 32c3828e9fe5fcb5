// Decode matvec (M = 1) device code of the per-launch kernels (matvec.hip); the decode chain
// (chain.hip) reuses its dequantisation helpers.
//
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
//     (store, residual add, SwiGLU pair, RoPE + KV append, or logits + argmax).
// Weights are streamed exactly once per token as 16-byte coalesced loads; x never leaves LDS.
#pragma once
#include <algorithm>
#include <cstdlib>

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
IEK_DEV float mul_rn(float x, float w) {
#pragma clang fp contract(off)
  return x * w;
}
IEK_DEV float div_rn(float x, float y) {
#pragma clang fp contract(off)
  return x / y;
}

// ---- prologue: x (optionally RMS-normalised) into LDS ----------------------------------------
// x (or x*w, accumulating sum(x^2)) is loaded in batches of 8 float4 per thread with all loads of a
// batch in flight together; the normalised variant then divides the LDS copy by rms in place, i.e.
// y = (x*w)/rms with the reference's two roundings. The epilogue's inputs (residual vector, this
// position's RoPE cos/sin) are staged here too, so the main loop never waits on a global load.
struct Lds {
  float* x;      // K f32
  float* res;    // N (EPI_RESID)
  float* rope;   // 2*npairs (EPI_QKV)
};

// Block-wide sum for the matvec workgroups (NT threads; red holds NT / 64 floats).
template <int NT = 256>
IEK_DEV float block_sum_mv(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = (red[0] + red[1]) + (red[2] + red[3]);
  if constexpr (NT == 512) t += (red[4] + red[5]) + (red[6] + red[7]);
  return t;
}

// Staging with the residual update in front (a.pre_t set; f32 staging): y = x + rmsnorm(pre_t,
// pre_w) [* pre_scale] with the reference's roundings (rmsnorm.rs:44-47, residual_add.rs:3-12,
// ffn.rs:242-278), then the launch's own RMSNorm of y when norm_w is set. Workgroup 0 stores y.
IEK_DEV void stage_pre(const MvArgs& a, const Lds& L, int pos) {
  __shared__ float red[4];
  const int K = a.K, tid = threadIdx.x;
  float st = 0.f;
  for (int i = tid; i < K; i += 256) {
    const float t = a.pre_t[i];
    st += t * t;
  }
  const float rms_t = rms_of(block_sum_mv(st, red), K, a.eps);
  float sy = 0.f;
  for (int i = tid; i < K; i += 256) {
    float y = a.x[i] + div_rn(mul_rn(a.pre_t[i], a.pre_w[i]), rms_t);
    if (a.pre_has_scale) y = mul_rn(y, a.pre_scale);
    if (blockIdx.x == 0) a.pre_out[i] = y;
    sy += y * y;
    L.x[i] = a.norm_w ? mul_rn(y, a.norm_w[i]) : y;
  }
  if (a.norm_w) {
    const float rms = rms_of(block_sum_mv(sy, red), K, a.eps);
    for (int i = tid; i < K; i += 256) L.x[i] = div_rn(L.x[i], rms);
  }
  if (a.epi == EPI_RESID) {
    const int N = a.n[0];
    for (int i = tid; i < N; i += 256) L.res[i] = a.resid[i];
  }
  if (a.epi == EPI_QKV) {
    for (int i = tid; i < 2 * a.npairs; i += 256) L.rope[i] = a.rope_cs[(size_t)pos * a.npairs * 2 + i];
  }
  __syncthreads();
  __builtin_amdgcn_s_waitcnt(0);
}

IEK_DEV void stage(const MvArgs& a, const Lds& L, int pos) {
  if (a.pre_t) {
    stage_pre(a, L, pos);
    return;
  }
  const int K = a.K, tid = threadIdx.x;
  const bool vec = (K & 3) == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
                   (!a.norm_w || (reinterpret_cast<uintptr_t>(a.norm_w) & 15) == 0);
  const int K4 = vec ? K >> 2 : 0;
  const float4* x4 = reinterpret_cast<const float4*>(a.x);
  const float4* w4 = reinterpret_cast<const float4*>(a.norm_w);
  float4* s4 = reinterpret_cast<float4*>(L.x);
  constexpr int B = 8;
  float ss = 0.f;
  for (int base = tid; base < K4; base += 256 * B) {
    float4 v[B], w[B];
#pragma unroll
    for (int b = 0; b < B; ++b) v[b] = x4[min(base + 256 * b, K4 - 1)];
    if (a.norm_w) {
#pragma unroll
      for (int b = 0; b < B; ++b) w[b] = w4[min(base + 256 * b, K4 - 1)];
    }
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const int i = base + 256 * b;
      if (i < K4) {
        if (a.norm_w) {
          ss += (v[b].x * v[b].x + v[b].y * v[b].y) + (v[b].z * v[b].z + v[b].w * v[b].w);
          s4[i] = make_float4(mul_rn(v[b].x, w[b].x), mul_rn(v[b].y, w[b].y), mul_rn(v[b].z, w[b].z),
                              mul_rn(v[b].w, w[b].w));
        } else {
          s4[i] = v[b];
        }
      }
    }
  }
  for (int i = 4 * K4 + tid; i < K; i += 256) {
    const float v = a.x[i];
    if (a.norm_w) {
      ss += v * v;
      L.x[i] = mul_rn(v, a.norm_w[i]);
    } else {
      L.x[i] = v;
    }
  }
  if (a.epi == EPI_RESID) {
    const int N = a.n[0];
    for (int i = tid; i < N; i += 256) L.res[i] = a.resid[i];
  }
  if (a.epi == EPI_QKV) {
    for (int i = tid; i < 2 * a.npairs; i += 256) L.rope[i] = a.rope_cs[(size_t)pos * a.npairs * 2 + i];
  }
  if (a.norm_w) {
    __shared__ float red[4];
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float rms = rms_of((red[0] + red[1]) + (red[2] + red[3]), K, a.eps);
    for (int i = tid; i < K; i += 256) L.x[i] = div_rn(L.x[i], rms);
  }
  __syncthreads();
  // Clamped loads whose values went unused (lanes past K) are still counted as pending; retire
  // them here, where nothing else is in flight, so the main loop's first wait is not a full drain.
  __builtin_amdgcn_s_waitcnt(0);
}

// LDS bytes: x staging (4K), then the residual vector (EPI_RESID) and this position's RoPE
// (cos, sin) pairs (EPI_QKV).
__host__ __device__ inline size_t lds_bytes(const MvArgs& a) {
  return 4 * (size_t)a.K + (a.epi == EPI_RESID ? 4 * (size_t)a.n[0] : 0) + (a.epi == EPI_QKV ? 8 * (size_t)a.npairs : 0);
}

// [x staging][residual][RoPE]
IEK_DEV Lds lds_layout(const MvArgs& a, float* base) {
  Lds L;
  L.x = base;
  L.res = base + a.K;
  L.rope = L.res + (a.epi == EPI_RESID ? a.n[0] : 0);
  return L;
}

IEK_DEV bool res_vec(const MvArgs& a) {
  return a.epi == EPI_RESID && (a.n[0] & 3) == 0 && a.n[0] <= 4096 && (reinterpret_cast<uintptr_t>(a.resid) & 15) == 0;
}

// ---- x staging split in two ------------------------------------------------------------------
// Thread t of an NT-thread workgroup owns the float4 slots t + NT s (s < S, K <= 4 NT S; the host
// picks S) of x, the norm weight and the residual-update inputs (pre_t, pre_w). stage32_issue
// loads them (the conditional ones first, x last, ahead of the weight loads); stage32_finish
// computes the staging with the roundings of stage / stage_pre. The memory counter retires in
// order, so x (an L2 hit) issued after the first weight loads would wait behind the weight stream;
// every load whose issue depends on a runtime condition goes out before the unconditional x slots,
// and the weight loads follow: the compiler counts the loads in flight only along paths with the
// same loads, so a wait for x then leaves the weight loads in flight instead of draining them.
template <int S>
struct XPre32 {
  float4 x[S], w[S], t[S], tw[S];
  float4 res[4];
  float2 rope;
  float ev;
};

template <int S, int NT = 256>
IEK_DEV void stage32_issue(const MvArgs& a, XPre32<S>& p, int pos, int ev_idx) {
  const int tid = threadIdx.x, K4 = a.K >> 2;
  if (a.pre_t) {
    const float4* t4 = reinterpret_cast<const float4*>(a.pre_t);
    const float4* tw4 = reinterpret_cast<const float4*>(a.pre_w);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int i = min(tid + NT * s, K4 - 1);
      p.t[s] = t4[i];
      p.tw[s] = tw4[i];
    }
  }
  if (a.norm_w) {
    const float4* w4 = reinterpret_cast<const float4*>(a.norm_w);
#pragma unroll
    for (int s = 0; s < S; ++s) p.w[s] = w4[min(tid + NT * s, K4 - 1)];
  }
  if (ev_idx >= 0) {
    p.ev = (a.epi == EPI_GELU_MUL ? a.mulv : a.resid)[ev_idx];
  } else if (res_vec(a)) {
    const float4* r4 = reinterpret_cast<const float4*>(a.resid);
    const int n4 = a.n[0] >> 2;
#pragma unroll
    for (int u = 0; u < 1024 / NT; ++u) p.res[u] = r4[min(tid + NT * u, n4 - 1)];
  }
  if (a.epi == EPI_QKV)
    p.rope = reinterpret_cast<const float2*>(a.rope_cs)[(size_t)pos * a.npairs + min(tid, a.npairs - 1)];
  const float4* x4 = reinterpret_cast<const float4*>(a.x);
#pragma unroll
  for (int s = 0; s < S; ++s) p.x[s] = x4[min(tid + NT * s, K4 - 1)];
}

template <int S, int NT = 256>
IEK_DEV void stage32_finish(const MvArgs& a, const Lds& L, int pos, XPre32<S>& p, bool res_lds) {
  __shared__ float red[NT / 64];
  const int tid = threadIdx.x, K = a.K, K4 = K >> 2;
  // the empty asm statements keep the arithmetic below the weight loads (the memory clobber also keeps them
  // from being hoisted among the loads)
  auto pin = [](float4& v) { asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w)::"memory"); };
#pragma unroll
  for (int s = 0; s < S; ++s) pin(p.x[s]);
  float4* L4 = reinterpret_cast<float4*>(L.x);
  float4 y[S];
#pragma unroll
  for (int s = 0; s < S; ++s) y[s] = p.x[s];
  if (a.pre_t) {
    // y = x + (t * w) / rms(t) [* scale], each step rounded as in stage_pre; workgroup 0 stores y
    float st = 0.f;
#pragma unroll
    for (int s = 0; s < S; ++s)
      if (tid + NT * s < K4) {
        const float4 t = p.t[s];
        st += t.x * t.x;
        st += t.y * t.y;
        st += t.z * t.z;
        st += t.w * t.w;
      }
    const float rms_t = rms_of(block_sum_mv<NT>(st, red), K, a.eps);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int i = tid + NT * s;
      if (i < K4) {
        const float4 x = p.x[s], t = p.t[s], w = p.tw[s];
        float4 v = make_float4(x.x + div_rn(mul_rn(t.x, w.x), rms_t), x.y + div_rn(mul_rn(t.y, w.y), rms_t),
                               x.z + div_rn(mul_rn(t.z, w.z), rms_t), x.w + div_rn(mul_rn(t.w, w.w), rms_t));
        if (a.pre_has_scale)
          v = make_float4(mul_rn(v.x, a.pre_scale), mul_rn(v.y, a.pre_scale), mul_rn(v.z, a.pre_scale),
                          mul_rn(v.w, a.pre_scale));
        if (blockIdx.x == 0) reinterpret_cast<float4*>(a.pre_out)[i] = v;
        y[s] = v;
      }
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int i = tid + NT * s;
    if (i < K4) {
      const float4 v = y[s];
      ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
      if (a.norm_w) {
        const float4 w = p.w[s];
        L4[i] = make_float4(mul_rn(v.x, w.x), mul_rn(v.y, w.y), mul_rn(v.z, w.z), mul_rn(v.w, w.w));
      } else {
        L4[i] = v;
      }
    }
  }
  if (a.epi == EPI_RESID && res_lds) {
    const int N = a.n[0];
    if (res_vec(a)) {
      float4* d4 = reinterpret_cast<float4*>(L.res);
#pragma unroll
      for (int u = 0; u < 1024 / NT; ++u)
        if (tid + NT * u < (N >> 2)) d4[tid + NT * u] = p.res[u];
    } else {
      for (int i = tid; i < N; i += NT) L.res[i] = a.resid[i];
    }
  }
  if (a.epi == EPI_QKV) {
    if (tid < a.npairs) reinterpret_cast<float2*>(L.rope)[tid] = p.rope;
    for (int i = NT + tid; i < a.npairs; i += NT)
      reinterpret_cast<float2*>(L.rope)[i] = reinterpret_cast<const float2*>(a.rope_cs)[(size_t)pos * a.npairs + i];
  }
  if (a.norm_w) {
    const float rms = rms_of(block_sum_mv<NT>(ss, red), K, a.eps);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int i = tid + NT * s;
      if (i < K4) {
        const float4 v = L4[i];
        L4[i] = make_float4(div_rn(v.x, rms), div_rn(v.y, rms), div_rn(v.z, rms), div_rn(v.w, rms));
      }
    }
  }
  __syncthreads();
}

// Segment fields picked with constant indices: a dynamic index into the by-value argument block
// becomes a vector memory load, whose wait would also drain the in-flight weight prefetch.
IEK_DEV const uint8_t* seg_w(const MvArgs& a, int s) { return s == 0 ? a.w[0] : (s == 1 ? a.w[1] : a.w[2]); }
IEK_DEV float* seg_out(const MvArgs& a, int s) { return s == 0 ? a.out[0] : (s == 1 ? a.out[1] : a.out[2]); }
IEK_DEV int seg_base(const MvArgs& a, int s) { return s == 0 ? a.seg_start[0] : (s == 1 ? a.seg_start[1] : a.seg_start[2]); }

// ---- epilogue -----------------------------------------------------------------------------------
// Reads only registers and LDS (pos was loaded at kernel start); with ev_reg, lane r < R holds the
// residual (EPI_RESID) or multiplier (EPI_GELU_MUL) of row lr0 + r in ev.
template <int R>
IEK_DEV void epilogue(const MvArgs& a, const Lds& L, int s, int lr0, float (&acc)[R], const float* acc_up, int lane,
                      int pos, unsigned long long& run_key, float ev = 0.f, bool ev_reg = false) {
  if (a.epi == EPI_SWIGLU || a.epi == EPI_GEGLU) {
    if (lane < R) {
      float g = acc[0], u = acc_up[0];
#pragma unroll
      for (int r = 1; r < R; ++r)
        if (lane == r) {
          g = acc[r];
          u = acc_up[r];
        }
      st_f<false>(a.out[0] + lr0 + lane, a.epi == EPI_GEGLU ? gelu_tanh_dev(g) * u : silu_mul(g, u));
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
      if (s < 2 && d < 2 * a.npairs) v = rope_rotate(v, partner, L.rope[d & ~1], L.rope[(d & ~1) + 1], (d & 1) == 0);
      if (s == 0) {
        st_f<false>(a.out[0] + n, v);
      } else {
        const size_t dst = ((size_t)(n / hd) * a.ctx + pos) * hd + d;
        void* c = s == 1 ? a.kc : a.vc;
        if (a.kv_f32) st_f<false>(static_cast<float*>(c) + dst, v);
        else st_h<false>(static_cast<__half*>(c) + dst, __float2half_rn(v));
      }
    }
    return;
  }
  if (a.epi == EPI_ARGMAX) {
    // logits row n: store (soft-capped), fold its packed (value, first-index) key into the lane's
    // running maximum; one atomic per workgroup at the end of the launch (argmax_flush)
    float v = acc[0];
#pragma unroll
    for (int r = 1; r < R; ++r)
      if (lane == r) v = acc[r];
    if (a.softcap > 0.f) v = soft_cap(v, a.softcap);
    if (lane < R) {
      a.out[0][lr0 + lane] = v;
      const unsigned long long key = argmax_key_dev(v, (uint32_t)(lr0 + lane));
      run_key = key > run_key ? key : run_key;
      if (!isfinite(v)) atomicOr(a.amax_flag, 1);
    }
    return;
  }
  if (lane < R) {
    float v = acc[0];
#pragma unroll
    for (int r = 1; r < R; ++r)
      if (lane == r) v = acc[r];
    const int n = lr0 + lane;
    if (a.epi == EPI_RESID) v = (ev_reg ? ev : L.res[n]) + v;
    if (a.epi == EPI_GELU_MUL) v = gelu_tanh_dev(v) * (ev_reg ? ev : a.mulv[n]);
    st_f<false>(seg_out(a, s) + n, v);
  }
}

template <int R>
IEK_DEV void wave_reduce(float (&acc)[R]) {
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
}

// ---- Q4_K -----------------------------------------------------------------------------------
// Chunk g (0..3) of a superblock = qs bytes [32g, 32g+32): 32 low nibbles (sub-block 2g, elements
// 64g+l) and 32 high nibbles (sub-block 2g+1, elements 64g+32+l). The nibbles go straight into
// v_fma_mix_f32 as f16 operands: (w >> s) & 0x000F000F leaves two nibbles in the two halves of a
// register, each the f16 subnormal q * 2^-24, which the instruction widens exactly; the 2^24 is
// folded into the sub-block scale.
IEK_DEV float h_lo(uint32_t w) { return __half2float(__ushort_as_half((unsigned short)(w & 0xFFFFu))); }
IEK_DEV float h_hi(uint32_t w) { return __half2float(__ushort_as_half((unsigned short)(w >> 16))); }

// sum over one qs dword (bytes l..l+3): lo nibbles against xl[0..3], hi nibbles against xh[0..3]
IEK_DEV void q4_dword(uint32_t w, const float4 xl, const float4 xh, float& sl, float& sh) {
  const uint32_t t0 = w & 0x000F000Fu, t1 = (w >> 4) & 0x000F000Fu;
  const uint32_t t2 = (w >> 8) & 0x000F000Fu, t3 = (w >> 12) & 0x000F000Fu;
  sl = fmaf(xl.x, h_lo(t0), sl);
  sl = fmaf(xl.z, h_hi(t0), sl);
  sh = fmaf(xh.x, h_lo(t1), sh);
  sh = fmaf(xh.z, h_hi(t1), sh);
  sl = fmaf(xl.y, h_lo(t2), sl);
  sl = fmaf(xl.w, h_hi(t2), sl);
  sh = fmaf(xh.y, h_lo(t3), sh);
  sh = fmaf(xh.w, h_hi(t3), sh);
}

// get_scale_min_k4 for a per-lane sub-block index without branches (both forms are extracted and
// selected), so every lane of the wave runs one path and every loaded header dword is consumed.
IEK_DEV void scale_min_k4_sel(int j, uint32_t s0, uint32_t s1, uint32_t s2, float* sc, float* m) {
  const int i = j & 3;
  const uint32_t b0 = byte_of(s0, i), b1 = byte_of(s1, i), b2 = byte_of(s2, i);
  const uint32_t sc_lo = b0 & 63u, m_lo = b1 & 63u;
  const uint32_t sc_hi = (b2 & 0xFu) | ((b0 >> 6) << 4), m_hi = (b2 >> 4) | ((b1 >> 6) << 4);
  *sc = (float)(j < 4 ? sc_lo : sc_hi);
  *m = (float)(j < 4 ? m_lo : m_hi);
}

IEK_DEV float q4k_dot(uint4 hdr, uint4 q0, uint4 q1, int g, const float4* xl4, const float4* xh4, float xsl,
                      float xsh) {
  float d = half_bits_to_float(hdr.x), dmin = half_bits_to_float(hdr.x >> 16);
  float sc0, m0, sc1, m1;
  scale_min_k4_sel(2 * g, hdr.y, hdr.z, hdr.w, &sc0, &m0);
  scale_min_k4_sel(2 * g + 1, hdr.y, hdr.z, hdr.w, &sc1, &m1);
  const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
  float sl = 0.f, sh = 0.f;
#pragma unroll
  for (int t = 0; t < 8; ++t) q4_dword(qw[t], xl4[t], xh4[t], sl, sh);
  const float k24 = 16777216.0f;  // 2^24
  return (d * sc0 * k24) * sl - (dmin * m0) * xsl + (d * sc1 * k24) * sh - (dmin * m1) * xsh;
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
  o[2] = base[*shift ? 2 : 1];  // always issued; with shift 0 the third dword is not used
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
  q.s[2] = base[q.sh_s >= 2 ? 2 : 1];  // always issued; unused bytes are never extracted
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
  // 6-bit values (q + 32) are assembled per byte, split into register halves and fed to
  // v_fma_mix_f32 as exact f16 subnormals (value * 2^-24).
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
      const uint32_t e = qq[i] & 0x00FF00FFu, o = (qq[i] >> 8) & 0x00FF00FFu;
      s[i] = fmaf(xv.x, h_lo(e), s[i]);
      s[i] = fmaf(xv.z, h_hi(e), s[i]);
      s[i] = fmaf(xv.y, h_lo(o), s[i]);
      s[i] = fmaf(xv.w, h_hi(o), s[i]);
    }
  }
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) r += (d * sc[i]) * (16777216.0f * s[i] - 32.0f * xs4[i]);
  return r;
}

// End of an EPI_ARGMAX launch: reduce the lanes' running keys over the workgroup and publish one
// atomicMax (the key packs the value's order and the inverted index, so the maximum is the first
// maximal index).
template <int NT = 256>
IEK_DEV void argmax_flush(const MvArgs& a, unsigned long long run_key) {
  __shared__ unsigned long long red_key[NT / 64];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(run_key, off, WAVE);
    run_key = o > run_key ? o : run_key;
  }
  if ((threadIdx.x & 63) == 0) red_key[threadIdx.x >> 6] = run_key;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long k = red_key[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) k = red_key[w] > k ? red_key[w] : k;
    if (k) atomicMax(a.amax_key, k);
  }
}

// ---- streaming driver ------------------------------------------------------------------------
// Wave w of workgroup b owns row groups (4b + w) + k * (4 * gridDim.x). It walks the flattened
// (group, pass) sequence with two register buffers used alternately (no copies of in-flight data),
// issuing the next step's weight loads before computing the current one. Loads are unconditional
// with clamped addresses so the compiler can count them statically and keep them all in flight.
struct Q4Tr {
  static constexpr int CHUNKS = 4;  // 64-value chunks per superblock
  static constexpr int BYTES = Q4K_BYTES;
  IEK_DEV static size_t row_bytes(int nsb) { return (size_t)nsb * BYTES; }
  template <int NR>
  struct Buf {
    uint4 hdr[NR], qa[NR], qb[NR];
  };
  template <int NR>
  IEK_DEV static void load(Buf<NR>& b, const uint8_t* const (&rows)[NR], int c, int nsb) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const uint8_t* blk = rows[r] + (size_t)(c >> 2) * Q4K_BYTES;
      b.hdr[r] = *reinterpret_cast<const uint4*>(blk);
      b.qa[r] = *reinterpret_cast<const uint4*>(blk + 16 + 32 * (c & 3));
      b.qb[r] = *reinterpret_cast<const uint4*>(blk + 32 + 32 * (c & 3));
    }
  }
  template <int NR>
  IEK_DEV static void compute(const Buf<NR>& b, int c, const Lds& L, float (&acc)[NR]) {
    const float* xs = L.x;
    const int e0 = (c >> 2) * QK_K + (c & 3) * 64;
    float4 xl4[8], xh4[8];
    float xsl = 0.f, xsh = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      xl4[t] = *reinterpret_cast<const float4*>(xs + e0 + 4 * t);
      xh4[t] = *reinterpret_cast<const float4*>(xs + e0 + 32 + 4 * t);
      xsl += (xl4[t].x + xl4[t].y) + (xl4[t].z + xl4[t].w);
      xsh += (xh4[t].x + xh4[t].y) + (xh4[t].z + xh4[t].w);
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] += q4k_dot(b.hdr[r], b.qa[r], b.qb[r], c & 3, xl4, xh4, xsl, xsh);
  }
};

struct Q6Tr {
  static constexpr int CHUNKS = 8;  // 32-value chunks per superblock
  static constexpr int BYTES = Q6K_BYTES;
  IEK_DEV static size_t row_bytes(int nsb) { return (size_t)nsb * BYTES; }
  template <int NR>
  struct Buf {
    Q6Raw q[NR];
  };
  template <int NR>
  IEK_DEV static void load(Buf<NR>& b, const uint8_t* const (&rows)[NR], int c, int nsb) {
#pragma unroll
    for (int r = 0; r < NR; ++r) q6_load(rows[r] + (size_t)(c >> 3) * Q6K_BYTES, (c >> 2) & 1, c & 3, b.q[r]);
  }
  template <int NR>
  IEK_DEV static void compute(const Buf<NR>& b, int c, const Lds& L, float (&acc)[NR]) {
    const float* xs = L.x;
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
    for (int r = 0; r < NR; ++r) acc[r] += q6k_dot(b.q[r], x4, xs4);
  }
};

// Q6_K in the regrouped per-row layout (DT_Q6K_R, built once at model load by
// launch_repack_q6k): for superblock j of a row, lane chunk k = 2h + j16 holds the 16 ql bytes of
// quarters 0/2, the 16 ql bytes of quarters 1/3 and the 16 qh bytes for weights l = 16*j16 ..
// 16*j16+15 of half h (48 contiguous, 16-byte aligned bytes), its four sub-block scales as one
// dword and the superblock's d. A lane's 64 weights are thus three coalesced 16-byte loads plus
// two small ones, instead of thirteen dword loads per 32 weights from the 210-byte blocks. The
// values are the same bytes, so the dequantised weights are unchanged.
struct Q6RLayout {
  template <int NR>
  struct Buf {
    uint4 qa[NR], qb[NR], qh[NR];
    uint32_t sc[NR], d[NR];
  };
  template <int NR>
  IEK_DEV static void load(Buf<NR>& b, const uint8_t* const (&rows)[NR], int c, int nsb) {
    const int j = c >> 2, k = c & 3;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const uint8_t* m = rows[r] + (size_t)j * 192 + 48 * k;
      b.qa[r] = *reinterpret_cast<const uint4*>(m);
      b.qb[r] = *reinterpret_cast<const uint4*>(m + 16);
      b.qh[r] = *reinterpret_cast<const uint4*>(m + 32);
      b.sc[r] = *reinterpret_cast<const uint32_t*>(rows[r] + (size_t)nsb * 192 + 16 * j + 4 * k);
      b.d[r] = *reinterpret_cast<const uint16_t*>(rows[r] + (size_t)nsb * 208 + 2 * j);
    }
  }
};

// Q6_K in the regrouped per-row layout (DT_Q6K_R) against f32 x. Per lane chunk (64 weights of
// one half: l = 16*j16 .. 16*j16+15 in each of the four quarters) the 6-bit values q + 32 are
// assembled per byte, split into register halves and fed to v_fma_mix_f32 as exact f16 subnormals
// (value * 2^-24), so each quarter's sum is S = sum x * (q + 32) in f32; the quarter then adds
// (d * sc) * (2^24 * S - 32 * sum x), the reference's sum of x * (d * sc * q) reassociated.
struct Q6RTr {
  static constexpr int CHUNKS = 4;
  static constexpr int BYTES = 208;
  IEK_DEV static size_t row_bytes(int nsb) { return q6r_row_bytes(nsb); }
  template <int NR>
  using Buf = Q6RLayout::Buf<NR>;
  template <int NR>
  IEK_DEV static void load(Buf<NR>& b, const uint8_t* const (&rows)[NR], int c, int nsb) {
    Q6RLayout::load<NR>(b, rows, c, nsb);
  }
  template <int NR>
  IEK_DEV static void compute(const Buf<NR>& b, int c, const Lds& L, float (&acc)[NR]) {
    const int j = c >> 2, k = c & 3, h = k >> 1, j16 = k & 1;
    const int e0 = j * QK_K + 128 * h + 16 * j16;
    // x of quarter qd, weights l = 16*j16 + 4t .. +3: X[qd][t]
    float4 X[4][4];
    float xs[4];
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const float4* p = reinterpret_cast<const float4*>(L.x + e0 + 32 * qd);
      float s = 0.f;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        X[qd][t] = p[t];
        s += (X[qd][t].x + X[qd][t].y) + (X[qd][t].z + X[qd][t].w);
      }
      xs[qd] = s;
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const uint32_t A[4] = {b.qa[r].x, b.qa[r].y, b.qa[r].z, b.qa[r].w};
      const uint32_t B[4] = {b.qb[r].x, b.qb[r].y, b.qb[r].z, b.qb[r].w};
      const uint32_t H[4] = {b.qh[r].x, b.qh[r].y, b.qh[r].z, b.qh[r].w};
      float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t qq[4] = {(A[t] & 0x0F0F0F0Fu) | ((H[t] << 4) & 0x30303030u),
                                (B[t] & 0x0F0F0F0Fu) | ((H[t] << 2) & 0x30303030u),
                                ((A[t] >> 4) & 0x0F0F0F0Fu) | (H[t] & 0x30303030u),
                                ((B[t] >> 4) & 0x0F0F0F0Fu) | ((H[t] >> 2) & 0x30303030u)};
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const float4 xv = X[qd][t];
          const uint32_t e = qq[qd] & 0x00FF00FFu, o = (qq[qd] >> 8) & 0x00FF00FFu;
          s[qd] = fmaf(xv.x, h_lo(e), s[qd]);
          s[qd] = fmaf(xv.z, h_hi(e), s[qd]);
          s[qd] = fmaf(xv.y, h_lo(o), s[qd]);
          s[qd] = fmaf(xv.w, h_hi(o), s[qd]);
        }
      }
      const float d = half_bits_to_float(b.d[r]);
      float sum = 0.f;
#pragma unroll
      for (int qd = 0; qd < 4; ++qd)
        sum += (d * (float)(int8_t)((b.sc[r] >> (8 * qd)) & 0xFF)) * (16777216.0f * s[qd] - 32.0f * xs[qd]);
      acc[r] += sum;
    }
  }
};

// Q8_0 in a regrouped per-row layout (DT_Q8_0_R, built once at model load by launch_repack_q80):
// a row's nb = K/32 blocks keep their 32 int8 quants as nb contiguous 32-byte runs, followed by
// the nb f16 scales (padded to 16 bytes), so one lane's block is two 16-byte loads and one short
// load instead of 34 bytes at 2-byte alignment. The bytes are the native ones, rearranged.
// x stays f32 here (the Gemma-4 models that use Q8_0 have a score scale of 1 on normalised q/k,
// which turns the int8 staging's 2^-16 activation rounding into ~1e-3 of logit error): each quant
// byte is read as the unsigned q + 128 (v_cvt_f32_ubyte after flipping the sign bits), and the
// offset comes back as one term per block, d * (sum x*(q+128) - 128 * sum x).
struct Q8RTr {
  static constexpr int CHUNKS = 8;  // 32-value blocks per 256
  static constexpr int BYTES = 34;
  IEK_DEV static size_t row_bytes(int nsb) { return q8r_row_bytes((size_t)nsb * 8); }
  template <int NR>
  struct Buf {
    uint4 qa[NR], qb[NR];
    uint32_t d[NR];
  };
  template <int NR>
  IEK_DEV static void load(Buf<NR>& b, const uint8_t* const (&rows)[NR], int c, int nsb) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const uint8_t* m = rows[r] + (size_t)c * 32;
      b.qa[r] = *reinterpret_cast<const uint4*>(m);
      b.qb[r] = *reinterpret_cast<const uint4*>(m + 16);
      b.d[r] = *reinterpret_cast<const uint16_t*>(rows[r] + (size_t)nsb * 256 + 2 * c);
    }
  }
  template <int NR>
  IEK_DEV static void compute(const Buf<NR>& b, int c, const Lds& L, float (&acc)[NR]) {
    const float4* x4 = reinterpret_cast<const float4*>(L.x + 32 * c);
    float4 xv[8];
    float xsum = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      xv[t] = x4[t];
      xsum += (xv[t].x + xv[t].y) + (xv[t].z + xv[t].w);
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const uint32_t q[8] = {b.qa[r].x, b.qa[r].y, b.qa[r].z, b.qa[r].w, b.qb[r].x, b.qb[r].y, b.qb[r].z, b.qb[r].w};
      float s = 0.f;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint32_t u = q[t] ^ 0x80808080u;  // bytes q + 128
        s += xv[t].x * ubyte_f<0>(u) + xv[t].y * ubyte_f<1>(u) + xv[t].z * ubyte_f<2>(u) + xv[t].w * ubyte_f<3>(u);
      }
      acc[r] += half_bits_to_float(b.d[r]) * (s - 128.f * xsum);
    }
  }
};

// Geometry of one streaming pass over a launch's rows: wave w of workgroup b owns row groups
// (4b + w) + k * (4 * gridDim.x) and walks its flattened (group, K pass) steps.
template <class Tr, int R, bool DUAL, int NW = 4>
struct MvGeom {
  static constexpr int NR = DUAL ? 2 * R : R;
  int lane, g0, stride, groups, nsb, nchunk, npass, steps;
  size_t rb;
  IEK_DEV MvGeom(const MvArgs& a) {
    lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int total = a.nseg == 1 ? a.seg_start[1] : (a.nseg == 2 ? a.seg_start[2] : a.seg_start[3]);
    groups = total / R;
    stride = gridDim.x * NW;
    g0 = blockIdx.x * NW + wave;
    nsb = a.K / QK_K;
    rb = Tr::row_bytes(nsb);
    nchunk = (a.K / QK_K) * Tr::CHUNKS;
    npass = (nchunk + WAVE - 1) / WAVE;
    const int my_groups = g0 < groups ? (groups - 1 - g0) / stride + 1 : 0;
    steps = my_groups * npass;
  }
  // Row pointers and chunk of step `it`, clamped into the wave's steps and the launch's row groups
  // so every load is valid (a wave without steps reads the last group).
  IEK_DEV void rows_of(const MvArgs& a, int it, const uint8_t* (&rows)[NR], int& c) const {
    const int k = max(0, min(it, steps - 1));
    const int g = min(g0 + (k / npass) * stride, groups - 1), p = k % npass;
    c = min(lane + WAVE * p, nchunk - 1);
    const int row0 = g * R;
    const int s = DUAL ? 0 : seg_of(a, row0);
    const int lr0 = row0 - seg_base(a, s);
    const uint8_t* w0 = seg_w(a, s);
#pragma unroll
    for (int r = 0; r < NR; ++r) rows[r] = r < R ? w0 + (size_t)lr0 * rb + (size_t)r * rb : a.w[1] + (size_t)(lr0 + r - R) * rb;
  }
};

// The streaming matvec of one launch's rows.
//
// Load order and waits. The compiler waits for a load by counting the memory operations issued
// after it, which it can only do along paths that issued the same ones; a load issued on some
// paths only makes every later wait conservative (a full drain of the weight stream). So: the
// conditional staging loads go first, then x, then the weight buffers, and in the stream the
// other buffer is always in flight while one is computed. MULTI (the host's choice, when some
// wave has more than one step) keeps two buffers in flight from the start; single-step launches
// carry only one. XS > 0 selects the split staging (x slots issued ahead of the weight loads).
template <class Tr, int R, bool DUAL, bool MULTI = true, int NT = 256, int XS = 0>
IEK_DEV void mv_body(const MvArgs& a, float* lds, int pos) {
  static_assert(NT == 256 || (NT == 512 && XS > 0), "512-thread workgroups need the split staging");
  constexpr int NW = NT / 64;
  constexpr int NR = DUAL ? 2 * R : R;
  const int lane = threadIdx.x & 63;
  const Lds L = lds_layout(a, lds);
  const MvGeom<Tr, R, DUAL, NW> G(a);
  const int npass = G.npass, nchunk = G.nchunk, steps = G.steps;
  typename Tr::template Buf<NR> A, B;
  unsigned long long run_key = 0;
  float acc[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = 0.f;
  // the epilogue's residual / multiplier in a register when every wave has at most one row group
  const bool ev_reg = XS > 0 && (a.epi == EPI_RESID || a.epi == EPI_GELU_MUL) && G.groups <= G.stride;
  int ev_idx = -1;
  if (ev_reg) {
    const int row0 = min(G.g0, G.groups - 1) * R;
    const int s0 = seg_of(a, row0);
    ev_idx = max(0, min(row0 - seg_base(a, s0) + min(lane, R - 1), a.n[0] - 1));
  }
  XPre32<(XS > 0 ? XS : 1)> xq;
  xq.ev = 0.f;

  auto finish = [&](int it) {
    const int p = it % npass;
    if (p != npass - 1) return;
    const int g = G.g0 + (it / npass) * G.stride;
    float accg[R], accu[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      accg[r] = acc[r];
      accu[r] = DUAL ? acc[R + r] : 0.f;
    }
    wave_reduce<R>(accg);
    if (DUAL) wave_reduce<R>(accu);
    const int row0 = g * R;
    const int s = DUAL ? 0 : seg_of(a, row0);
    epilogue<R>(a, L, s, row0 - seg_base(a, s), accg, accu, lane, pos, run_key, xq.ev, ev_reg);
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = 0.f;
  };
  auto step = [&](const typename Tr::template Buf<NR>& buf, int it) {
    const int p = it % npass;
    const int c = lane + WAVE * p;
    float part[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) part[r] = 0.f;
    Tr::template compute<NR>(buf, min(c, nchunk - 1), L, part);
    // The empty asm pins the dot products as computed on every path: otherwise the compiler sinks
    // them under the c < nchunk branch and a wave whose lanes all skip it leaves the buffer's loads
    // unretired, which costs a full drain at the next reuse of those registers.
#pragma unroll
    for (int r = 0; r < NR; ++r) asm volatile("" : "+v"(part[r]));
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] += c < nchunk ? part[r] : 0.f;
    finish(it);
  };
  auto load = [&](typename Tr::template Buf<NR>& buf, int it) {
    const uint8_t* rows[NR];
    int c;
    G.rows_of(a, it, rows, c);
    Tr::template load<NR>(buf, rows, c, G.nsb);
  };

  // x / residual / RoPE loads go out first, then the weight buffers, so the staging work overlaps
  // the weight fetch instead of queueing behind it.
  if constexpr (XS > 0) stage32_issue<XS, NT>(a, xq, pos, ev_idx);
  load(A, 0);
  if constexpr (MULTI) load(B, 1);
  // keep the staging arithmetic below the weight loads: scheduled among them, its first use of x
  // would hold the remaining weight loads back until x has arrived
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (XS > 0) stage32_finish<XS, NT>(a, L, pos, xq, !ev_reg);
  else stage(a, L, pos);
  if (steps > 0) {
    if constexpr (MULTI) {
      // Each buffer's refill is issued right after it was computed, unconditionally (the last one
      // re-reads the wave's final step and is never waited for), so every path into a step has
      // the same loads in flight behind it.
      for (int it = 0;; it += 2) {
        step(A, it);
        if (it + 1 >= steps) break;
        load(A, it + 2);
        step(B, it + 1);
        if (it + 2 >= steps) break;
        load(B, it + 3);
      }
    } else {
      step(A, 0);
    }
  }
  if (a.epi == EPI_ARGMAX) argmax_flush<NT>(a, run_key);
}

}  // namespace iek
