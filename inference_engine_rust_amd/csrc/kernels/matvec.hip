// Decode matvec (M = 1): y[n] = sum_k x[k] * W(k, n) over weights kept in their native GGUF
// block layout (ggml order: element (k, n) at flat k + n*K, src/ops/matmul.rs:1-3).
//
// Mapping (wave64, CDNA4): one wave owns R consecutive output rows; lane l takes the 16-byte
// quant chunks c = l, l+64, ... of each row, so a wave streams R rows as fully coalesced
// 1 KiB-per-instruction bursts while the lane's slice of x stays in VGPRs across the R rows.
// Dequant happens in registers; per-32-value sub-block scales are applied once per chunk:
//   sum_k x_k (d*sc*q_k - dmin*m) = (d*sc) * sum x_k q_k - (dmin*m) * sum x_k.
// Row sums end in a wave butterfly; lanes 0..R-1 write the R outputs through the epilogue.
#include "common.cuh"
#include "../iek_internal.h"

namespace iek {

struct MvSeg {
  const uint8_t* w;
  float* out;
  const float* resid;  // EPI_RESID: out[n] = resid[n] + dot (may alias out)
  int n;
};

struct MvParams {
  MvSeg seg[3];
  int seg_start[4];
  int nseg;
  const float* x;
  int K;
  int epi;
};

enum : int { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };

IEK_DEV float silu_mul(float g, float u) {
  // (g * sigmoid(g)) * u with the reference's two-branch sigmoid (src/ops/swiglu.rs:3-36).
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

// Byte i of a dword as f32; the compiler selects v_cvt_f32_ubyte{0..3}.
template <int I>
IEK_DEV float ubyte_f(uint32_t w) {
  return (float)((w >> (8 * I)) & 0xFFu);
}

template <int R>
IEK_DEV void reduce_rows(float (&acc)[R]) {
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
}

// Locate the segment that holds `row` (rows of a wave never straddle segments).
IEK_DEV int find_seg(const MvParams& p, int row) {
  int s = 0;
  if (p.nseg > 1 && row >= p.seg_start[1]) s = 1;
  if (p.nseg > 2 && row >= p.seg_start[2]) s = 2;
  return s;
}

// ---------------------------------------------------------------------------------------------
// Q4_K chunk dot: chunk j (0..7) of a superblock = 16 qs bytes covering 16 low-nibble values of
// sub-block 2g and 16 high-nibble values of sub-block 2g+1 (g = j/2).
// ---------------------------------------------------------------------------------------------
IEK_DEV float q4k_chunk_dot(uint4 hdr, uint4 qv, int j, const float (&xl)[16], const float (&xh)[16], float xsl,
                            float xsh) {
  const int g = j >> 1;
  float d = half_bits_to_float(hdr.x), dmin = half_bits_to_float(hdr.x >> 16);
  float sc0, m0, sc1, m1;
  scale_min_k4(2 * g, hdr.y, hdr.z, hdr.w, &sc0, &m0);
  scale_min_k4(2 * g + 1, hdr.y, hdr.z, hdr.w, &sc1, &m1);
  uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
  float sl = 0.f, sh = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    uint32_t lo = qw[t] & 0x0F0F0F0Fu, hi = (qw[t] >> 4) & 0x0F0F0F0Fu;
    sl += xl[4 * t + 0] * ubyte_f<0>(lo) + xl[4 * t + 1] * ubyte_f<1>(lo) +
          xl[4 * t + 2] * ubyte_f<2>(lo) + xl[4 * t + 3] * ubyte_f<3>(lo);
    sh += xh[4 * t + 0] * ubyte_f<0>(hi) + xh[4 * t + 1] * ubyte_f<1>(hi) +
          xh[4 * t + 2] * ubyte_f<2>(hi) + xh[4 * t + 3] * ubyte_f<3>(hi);
  }
  return (d * sc0) * sl - (dmin * m0) * xsl + (d * sc1) * sh - (dmin * m1) * xsh;
}

template <int R, bool DUAL>
__global__ __launch_bounds__(256) void mv_q4k_kernel(MvParams p) {
  const int lane = threadIdx.x & 63;
  const int wid = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int row0 = wid * R;
  const int total = DUAL ? p.seg[0].n : p.seg_start[p.nseg];
  if (row0 >= total) return;
  const int s = DUAL ? 0 : find_seg(p, row0);
  const int lr0 = row0 - (DUAL ? 0 : p.seg_start[s]);
  const int K = p.K;
  const size_t row_bytes = (size_t)(K / QK_K) * Q4K_BYTES;
  const int nchunk = (K / QK_K) * 8;
  const uint8_t* W0 = p.seg[s].w + (size_t)lr0 * row_bytes;
  const uint8_t* W1 = DUAL ? p.seg[1].w + (size_t)lr0 * row_bytes : nullptr;
  constexpr int NR = DUAL ? 2 * R : R;
  float acc[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = 0.f;

  for (int c = lane; c < nchunk; c += WAVE) {
    const int b = c >> 3, j = c & 7, g = j >> 1, hh = j & 1;
    const int e0 = b * QK_K + g * 64 + hh * 16;
    uint4 hdr[NR], qv[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const uint8_t* blk = (r < R ? W0 + (size_t)r * row_bytes : W1 + (size_t)(r - R) * row_bytes) + (size_t)b * Q4K_BYTES;
      hdr[r] = *reinterpret_cast<const uint4*>(blk);
      qv[r] = *reinterpret_cast<const uint4*>(blk + 16 + 16 * j);
    }
    float xl[16], xh[16];
    const float4* xp = reinterpret_cast<const float4*>(p.x + e0);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float4 a = xp[t], bb = xp[8 + t];
      xl[4 * t] = a.x; xl[4 * t + 1] = a.y; xl[4 * t + 2] = a.z; xl[4 * t + 3] = a.w;
      xh[4 * t] = bb.x; xh[4 * t + 1] = bb.y; xh[4 * t + 2] = bb.z; xh[4 * t + 3] = bb.w;
    }
    float xsl = 0.f, xsh = 0.f;
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      xsl += xl[t];
      xsh += xh[t];
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] += q4k_chunk_dot(hdr[r], qv[r], j, xl, xh, xsl, xsh);
  }
  reduce_rows<NR>(acc);
  if constexpr (DUAL) {
    if (lane < R) {
      float gv = acc[0], uv = acc[R];
#pragma unroll
      for (int r = 1; r < R; ++r)
        if (lane == r) {
          gv = acc[r];
          uv = acc[R + r];
        }
      p.seg[0].out[lr0 + lane] = silu_mul(gv, uv);
    }
  } else if (lane < R) {
    float v = acc[0];
#pragma unroll
    for (int r = 1; r < R; ++r)
      if (lane == r) v = acc[r];
    const int n = lr0 + lane;
    if (p.epi == EPI_RESID) v = p.seg[s].resid[n] + v;
    p.seg[s].out[n] = v;
  }
}

// ---------------------------------------------------------------------------------------------
// Q6_K: chunk (h, o8) of a superblock = 8 consecutive l of half h, covering the four quarters
// (32 values): ql[64h+8o8..+8], ql[64h+32+8o8..+8], qh[32h+8o8..+8]. Superblocks are 210 B, so
// these 8-byte fields are only 2-byte aligned; they are read as aligned dwords and re-sliced
// with v_alignbyte.
// ---------------------------------------------------------------------------------------------
IEK_DEV void load8_u2(const uint8_t* p, uint32_t& w0, uint32_t& w1) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t* base = reinterpret_cast<const uint32_t*>(a & ~uintptr_t(3));
  const uint32_t sh = (uint32_t)(a & 3u);
  uint32_t d0 = base[0], d1 = base[1], d2 = base[2];
  w0 = __builtin_amdgcn_alignbyte(d1, d0, sh);
  w1 = __builtin_amdgcn_alignbyte(d2, d1, sh);
}

IEK_DEV float q6k_chunk_dot(const uint8_t* blk, int h, int o8, const float (&x)[32], const float (&xs)[4]) {
  uint32_t a0, a1, b0, b1, h0, h1;
  load8_u2(blk + 64 * h + 8 * o8, a0, a1);
  load8_u2(blk + 64 * h + 32 + 8 * o8, b0, b1);
  load8_u2(blk + 128 + 32 * h + 8 * o8, h0, h1);
  const int isb = 8 * h + (o8 >> 1);
  float sc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) sc[i] = (float)(int8_t)blk[192 + isb + 2 * i];
  float d = half_bits_to_float(load_u16(blk + 208));
  uint32_t A[2] = {a0, a1}, B[2] = {b0, b1}, H[2] = {h0, h1};
  float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    uint32_t q0 = (A[t] & 0x0F0F0F0Fu) | ((H[t] << 4) & 0x30303030u);
    uint32_t q1 = (B[t] & 0x0F0F0F0Fu) | ((H[t] << 2) & 0x30303030u);
    uint32_t q2 = ((A[t] >> 4) & 0x0F0F0F0Fu) | (H[t] & 0x30303030u);
    uint32_t q3 = ((B[t] >> 4) & 0x0F0F0F0Fu) | ((H[t] >> 2) & 0x30303030u);
    uint32_t qq[4] = {q0, q1, q2, q3};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float* xi = &x[8 * i + 4 * t];
      s[i] += xi[0] * ubyte_f<0>(qq[i]) + xi[1] * ubyte_f<1>(qq[i]) +
              xi[2] * ubyte_f<2>(qq[i]) + xi[3] * ubyte_f<3>(qq[i]);
    }
  }
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) r += (d * sc[i]) * (s[i] - 32.0f * xs[i]);
  return r;
}

template <int R, bool DUAL>
__global__ __launch_bounds__(256) void mv_q6k_kernel(MvParams p) {
  const int lane = threadIdx.x & 63;
  const int wid = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int row0 = wid * R;
  const int total = DUAL ? p.seg[0].n : p.seg_start[p.nseg];
  if (row0 >= total) return;
  const int s = DUAL ? 0 : find_seg(p, row0);
  const int lr0 = row0 - (DUAL ? 0 : p.seg_start[s]);
  const int K = p.K;
  const size_t row_bytes = (size_t)(K / QK_K) * Q6K_BYTES;
  const int nchunk = (K / QK_K) * 8;
  const uint8_t* W0 = p.seg[s].w + (size_t)lr0 * row_bytes;
  const uint8_t* W1 = DUAL ? p.seg[1].w + (size_t)lr0 * row_bytes : nullptr;
  constexpr int NR = DUAL ? 2 * R : R;
  float acc[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = 0.f;
  for (int c = lane; c < nchunk; c += WAVE) {
    const int b = c >> 3, h = (c >> 2) & 1, o8 = c & 3;
    const int e0 = b * QK_K + 128 * h + 8 * o8;
    float x[32], xs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4* xp = reinterpret_cast<const float4*>(p.x + e0 + 32 * i);
      float4 u = xp[0], v = xp[1];
      x[8 * i + 0] = u.x; x[8 * i + 1] = u.y; x[8 * i + 2] = u.z; x[8 * i + 3] = u.w;
      x[8 * i + 4] = v.x; x[8 * i + 5] = v.y; x[8 * i + 6] = v.z; x[8 * i + 7] = v.w;
      float t = 0.f;
#pragma unroll
      for (int q = 0; q < 8; ++q) t += x[8 * i + q];
      xs[i] = t;
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const uint8_t* blk = (r < R ? W0 + (size_t)r * row_bytes : W1 + (size_t)(r - R) * row_bytes) + (size_t)b * Q6K_BYTES;
      acc[r] += q6k_chunk_dot(blk, h, o8, x, xs);
    }
  }
  reduce_rows<NR>(acc);
  if constexpr (DUAL) {
    if (lane < R) {
      float gv = acc[0], uv = acc[R];
#pragma unroll
      for (int r = 1; r < R; ++r)
        if (lane == r) {
          gv = acc[r];
          uv = acc[R + r];
        }
      p.seg[0].out[lr0 + lane] = silu_mul(gv, uv);
    }
  } else if (lane < R) {
    float v = acc[0];
#pragma unroll
    for (int r = 1; r < R; ++r)
      if (lane == r) v = acc[r];
    const int n = lr0 + lane;
    if (p.epi == EPI_RESID) v = p.seg[s].resid[n] + v;
    p.seg[s].out[n] = v;
  }
}

// ---------------------------------------------------------------------------------------------
// Generic path: any dtype, any K (including superblocks that straddle rows when K % 256 != 0,
// e.g. a 1408-wide FFN). One wave per row; lanes stride the row element by element and decode
// each weight from its flat block index.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void mv_generic_kernel(MvParams p, int dt) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int total = p.epi == EPI_SWIGLU ? p.seg[0].n : p.seg_start[p.nseg];
  if (row >= total) return;
  const int s = p.epi == EPI_SWIGLU ? 0 : find_seg(p, row);
  const int n = row - (p.epi == EPI_SWIGLU ? 0 : p.seg_start[s]);
  const int K = p.K;
  float a0 = 0.f, a1 = 0.f;
  for (int k = lane; k < K; k += WAVE) {
    const float xv = p.x[k];
    const size_t f = (size_t)k + (size_t)n * (size_t)K;
    a0 += xv * flat_elem(dt, p.seg[s].w, f);
    if (p.epi == EPI_SWIGLU) a1 += xv * flat_elem(dt, p.seg[1].w, f);
  }
  a0 = wave_sum(a0);
  if (p.epi == EPI_SWIGLU) a1 = wave_sum(a1);
  if (lane == 0) {
    if (p.epi == EPI_SWIGLU) p.seg[0].out[n] = silu_mul(a0, a1);
    else if (p.epi == EPI_RESID) p.seg[s].out[n] = p.seg[s].resid[n] + a0;
    else p.seg[s].out[n] = a0;
  }
}

// ---------------------------------------------------------------------------------------------
// Host launcher. `segs` describe up to three weights sharing K (fused Q/K/V) or a gate/up pair.
// ---------------------------------------------------------------------------------------------
static int pick_rows(int nmin, bool dual) {
  // Rows per wave: keep >= ~8 waves per CU for latency hiding on the largest layers.
  if (dual) return 2;
  if (nmin % 4 == 0 && nmin >= 16384) return 4;
  return 2;
}

void launch_matvec(int dt, const MvSegDesc* segs, int nseg, const float* x, int K, int epi, hipStream_t st) {
  MvParams p{};
  p.nseg = nseg;
  p.x = x;
  p.K = K;
  p.epi = epi;
  int start = 0, nmin = 1 << 30;
  for (int i = 0; i < nseg; ++i) {
    p.seg[i] = MvSeg{(const uint8_t*)segs[i].w, segs[i].out, segs[i].resid, segs[i].n};
    p.seg_start[i] = start;
    start += segs[i].n;
    nmin = std::min(nmin, segs[i].n);
  }
  p.seg_start[nseg] = start;
  const bool dual = epi == EPI_SWIGLU;
  const int be = dt == DT_Q8_0 ? Q8_0_ELEMS : (dt == DT_F32 ? 1 : QK_K);
  bool aligned = (dt == DT_Q4K || dt == DT_Q6K) && K % QK_K == 0;
  for (int i = 0; i < nseg && aligned; ++i)
    aligned = (reinterpret_cast<uintptr_t>(segs[i].w) % 16) == 0;
  aligned = aligned && (reinterpret_cast<uintptr_t>(x) % 16) == 0;
  (void)be;
  if (aligned) {
    int R = pick_rows(nmin, dual);
    bool ok = true;
    for (int i = 0; i < nseg; ++i) ok = ok && segs[i].n % R == 0;
    if (!ok) R = 1;
    const int rows = dual ? segs[0].n : start;
    const int waves = (rows + R - 1) / R;
    dim3 grid((waves + 3) / 4), block(256);
#define IEK_MV(KER)                                                                   \
  do {                                                                                \
    if (R == 4) hipLaunchKernelGGL((KER<4, false>), grid, block, 0, st, p);           \
    else if (R == 2 && dual) hipLaunchKernelGGL((KER<2, true>), grid, block, 0, st, p); \
    else if (R == 2) hipLaunchKernelGGL((KER<2, false>), grid, block, 0, st, p);      \
    else if (dual) hipLaunchKernelGGL((KER<1, true>), grid, block, 0, st, p);         \
    else hipLaunchKernelGGL((KER<1, false>), grid, block, 0, st, p);                  \
  } while (0)
    if (dt == DT_Q4K) IEK_MV(mv_q4k_kernel);
    else IEK_MV(mv_q6k_kernel);
#undef IEK_MV
  } else {
    const int rows = dual ? segs[0].n : start;
    dim3 grid((rows + 3) / 4), block(256);
    hipLaunchKernelGGL(mv_generic_kernel, grid, block, 0, st, p, dt);
  }
}

}  // namespace iek
