// Prefill matmul for K-quant / Q8_0 weights on the matrix cores with the block scales kept out of
// the fp16 operands: out[m, n] = sum_k a[m, k] * W(k, n).
//
// Algebra (per row n of W, per scale block): the reference dequantises
//   Q4_K  w = (d*sc)*q - dmin*m      (quant_k_handler.rs:38-82; q 4-bit, sc/m 6-bit per 32)
//   Q6_K  w = (d*sc)*(q - 32)        (:85-135; q 6-bit, sc int8 per 16)
//   Q8_0  w = d*q                    (:21-35; q int8 per 32)
// so sum_k a_k w_k = d * sum_k a_k w'_k - dmin * sum_b m_b * (sum_{k in b} a_k) with the integer
// w' = sc*q, sc*(q-32) or q. Q4_K's |w'| <= 945 and Q8_0's |w'| <= 128 are exact in fp16; Q6_K's
// |w'| <= 4096 is exact as an fp16 pair (hi + lo, |lo| <= 1). The activation is the fp16 pair
// (hi, lo) of f32, so MFMA products are exact and only f32 accumulation order differs from the
// reference: Q4_K / Q8_0 take two v_mfma_f32_16x16x32_f16 per K step (a_hi*w', a_lo*w'), Q6_K
// three (+ a_hi*w'_lo). The superblock factor d (Q8_0: per 32) multiplies a per-superblock MFMA
// accumulator into the output accumulator; Q4_K's min term uses the per-32 row sums of a.
//
// Tiling: BM x BN outputs per 256-thread workgroup (64x64 .. 128x128), four waves stacked along M;
// 32-wide K stages double-buffered in LDS (one barrier per stage) with the next stage's raw bytes
// in flight in registers while the current stage's MFMAs run. Up to three weight matrices that
// share the activation (Q/K/V) run as one launch; M tiles of one N tile share an XCD's L2.
#include <cstdlib>

#include "common.cuh"
#include "../iek_internal.h"

namespace iek {

struct GemmQArgs {
  const uint8_t* w[3];
  float* out[3];
  int n[3];
  int tile_start[4];  // first N tile of each segment; tile_start[nseg] = total N tiles
  int nseg;
  int M, K;
  size_t row_bytes;
  const __half* xh;
  const __half* xl;
  const float* xs;
  const float* resid;  // segment 0 only
  int xcd_remap;
};

namespace {

typedef _Float16 qh8_t __attribute__((ext_vector_type(8)));
typedef float qf4_t __attribute__((ext_vector_type(4)));
typedef uint32_t qu4_t __attribute__((ext_vector_type(4)));

constexpr int QBK = 32, QROW = 40;  // K per stage, LDS row (halves, padded)

IEK_DEV uint32_t hpack(_Float16 a, _Float16 b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// Raw bytes of 8 consecutive weights k0..k0+7 of row n (k0 % 8 == 0), fetched a stage ahead, and
// their decode into the integer w' (as fp16, exact), the stage's column scale and Q4_K's dmin*m.
template <int DT>
struct QDeq;

template <>
struct QDeq<DT_Q4K> {
  static constexpr int PERIOD = 8;  // stages per d block
  static constexpr bool LO = false;
  uint4 hdr;
  uint2 qs;
  IEK_DEV void load(const uint8_t* w, size_t row_bytes, int n, int k0, int nsb) {
    const uint8_t* blk = w + (size_t)n * row_bytes + (size_t)(k0 >> 8) * Q4K_BYTES;
    const int e = k0 & 255, g = e >> 6, l0 = e & 31;
    hdr = *reinterpret_cast<const uint4*>(blk);
    qs = *reinterpret_cast<const uint2*>(blk + 16 + 32 * g + l0);
  }
  IEK_DEV void decode(int k0, uint4& hi, uint4& lo, float& d, float& dm) const {
#pragma clang fp contract(off)
    const int e = k0 & 255, sb = e >> 5, nib = sb & 1;
    d = half_bits_to_float(hdr.x);
    const float dmin = half_bits_to_float(hdr.x >> 16);
    float sc, m;
    scale_min_k4(sb, hdr.y, hdr.z, hdr.w, &sc, &m);
    dm = dmin * m;
    const uint32_t isc = (uint32_t)sc;
    _Float16 h[8];
    const uint32_t w2[2] = {qs.x, qs.y};
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = (_Float16)(int)(((w2[i >> 2] >> (8 * (i & 3) + 4 * nib)) & 0xFu) * isc);
    hi = make_uint4(hpack(h[0], h[1]), hpack(h[2], h[3]), hpack(h[4], h[5]), hpack(h[6], h[7]));
    lo = make_uint4(0, 0, 0, 0);
  }
};

// Q6_K weights from the regrouped per-row layout (DT_Q6K_R: lane chunks of [ql 0/2 | ql 1/3 | qh]
// 16 bytes each, then per-chunk scale dwords, then d per superblock; see matvec.hip).
template <>
struct QDeq<DT_Q6K_R> {
  static constexpr int PERIOD = 8;
  static constexpr bool LO = true;
  uint2 ql, qh;
  uint32_t sc, d16;
  IEK_DEV void load(const uint8_t* w, size_t row_bytes, int n, int k0, int nsb) {
    const uint8_t* row = w + (size_t)n * row_bytes;
    const int j = k0 >> 8, e = k0 & 255, h = e >> 7, r = e & 127, qd = r >> 5, l = r & 31;
    const int kc = 2 * h + (l >> 4), i0 = l & 15;
    const uint8_t* m = row + (size_t)j * 192 + 48 * kc;
    ql = *reinterpret_cast<const uint2*>(m + ((qd & 1) ? 16 : 0) + i0);
    qh = *reinterpret_cast<const uint2*>(m + 32 + i0);
    sc = *reinterpret_cast<const uint32_t*>(row + (size_t)nsb * 192 + 16 * j + 4 * kc);
    d16 = *reinterpret_cast<const uint16_t*>(row + (size_t)nsb * 208 + 2 * j);
  }
  IEK_DEV void decode(int k0, uint4& hi, uint4& lo, float& d, float& dm) const {
    const int qd = ((k0 & 255) & 127) >> 5;
    d = half_bits_to_float(d16);
    dm = 0.f;
    const int isc = (int)(int8_t)((sc >> (8 * qd)) & 0xFF);
    const uint32_t lw[2] = {ql.x, ql.y}, hw[2] = {qh.x, qh.y};
    _Float16 h[8], l[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t lb = (lw[i >> 2] >> (8 * (i & 3))) & 0xFFu, hb = (hw[i >> 2] >> (8 * (i & 3))) & 0xFFu;
      const uint32_t nib = qd < 2 ? (lb & 0xFu) : (lb >> 4);
      const int wq = ((int)(nib | (((hb >> (2 * qd)) & 3u) << 4)) - 32) * isc;
      h[i] = (_Float16)wq;
      l[i] = (_Float16)(wq - (int)h[i]);
    }
    hi = make_uint4(hpack(h[0], h[1]), hpack(h[2], h[3]), hpack(h[4], h[5]), hpack(h[6], h[7]));
    lo = make_uint4(hpack(l[0], l[1]), hpack(l[2], l[3]), hpack(l[4], l[5]), hpack(l[6], l[7]));
  }
};

// Q6_K from the native 210-byte blocks (2-byte aligned: u16 loads).
template <>
struct QDeq<DT_Q6K> {
  static constexpr int PERIOD = 8;
  static constexpr bool LO = true;
  uint32_t ql[4], qh[4], sd;
  IEK_DEV void load(const uint8_t* w, size_t row_bytes, int n, int k0, int nsb) {
    const uint8_t* blk = w + (size_t)n * row_bytes + (size_t)(k0 >> 8) * Q6K_BYTES;
    const int e = k0 & 255, h = e >> 7, r = e & 127, quarter = r >> 5, l0 = r & 31;
    const uint16_t* pl = reinterpret_cast<const uint16_t*>(blk + 64 * h + 32 * (quarter & 1) + l0);
    const uint16_t* ph = reinterpret_cast<const uint16_t*>(blk + 128 + 32 * h + l0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ql[i] = pl[i];
      qh[i] = ph[i];
    }
    const int si = 192 + 8 * h + (l0 >> 4) + 2 * quarter;
    const uint16_t s2 = *reinterpret_cast<const uint16_t*>(blk + (si & ~1));
    sd = ((si & 1) ? (uint32_t)(s2 >> 8) : (uint32_t)(s2 & 0xFF)) |
         ((uint32_t)*reinterpret_cast<const uint16_t*>(blk + 208) << 16);
  }
  IEK_DEV void decode(int k0, uint4& hi, uint4& lo, float& d, float& dm) const {
    const int quarter = ((k0 & 255) & 127) >> 5;
    d = half_bits_to_float(sd >> 16);
    dm = 0.f;
    const int isc = (int)(int8_t)(sd & 0xFF);
    _Float16 h[8], l[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t lb = (ql[i >> 1] >> (8 * (i & 1))) & 0xFFu, hb = (qh[i >> 1] >> (8 * (i & 1))) & 0xFFu;
      const uint32_t nib = quarter < 2 ? (lb & 0xFu) : (lb >> 4);
      const int wq = ((int)(nib | (((hb >> (2 * quarter)) & 3u) << 4)) - 32) * isc;
      h[i] = (_Float16)wq;
      l[i] = (_Float16)(wq - (int)h[i]);
    }
    hi = make_uint4(hpack(h[0], h[1]), hpack(h[2], h[3]), hpack(h[4], h[5]), hpack(h[6], h[7]));
    lo = make_uint4(hpack(l[0], l[1]), hpack(l[2], l[3]), hpack(l[4], l[5]), hpack(l[6], l[7]));
  }
};

template <>
struct QDeq<DT_Q8_0> {
  static constexpr int PERIOD = 1;
  static constexpr bool LO = false;
  uint32_t q[4], d16;
  IEK_DEV void load(const uint8_t* w, size_t row_bytes, int n, int k0, int nsb) {
    const uint8_t* blk = w + (size_t)n * row_bytes + (size_t)(k0 >> 5) * Q8_0_BYTES;
    const uint16_t* p = reinterpret_cast<const uint16_t*>(blk + 2 + (k0 & 31));
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = p[i];
    d16 = *reinterpret_cast<const uint16_t*>(blk);
  }
  IEK_DEV void decode(int, uint4& hi, uint4& lo, float& d, float& dm) const {
    d = half_bits_to_float(d16);
    dm = 0.f;
    _Float16 h[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = (_Float16)(int)(int8_t)((q[i >> 1] >> (8 * (i & 1))) & 0xFFu);
    hi = make_uint4(hpack(h[0], h[1]), hpack(h[2], h[3]), hpack(h[4], h[5]), hpack(h[6], h[7]));
    lo = make_uint4(0, 0, 0, 0);
  }
};

// Per-32 row sums of the activation (Q4_K's min term): xs[m * (K/32) + b] = sum of a[m, 32b..].
__global__ __launch_bounds__(256) void block_sums_kernel(const float* __restrict__ a, size_t nb, float* __restrict__ xs) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nb) return;
  const float4* p = reinterpret_cast<const float4*>(a + 32 * i);
  float s = 0.f;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const float4 v = p[t];
    s += (v.x + v.y) + (v.z + v.w);
  }
  xs[i] = s;
}

template <int DT, int BM, int BN>
__global__ __launch_bounds__(256) void gemm_q_kernel(GemmQArgs g) {
  constexpr int WM = BM / 4, MT = WM / 16, NT = BN / 16;
  constexpr int BR = BN / 64;  // weight rows staged per thread per stage
  constexpr int AU = BM * 4 / 256;  // uint4 per thread per plane per stage (BM rows x 4 uint4)
  constexpr bool LO = QDeq<DT>::LO;
  constexpr int PERIOD = QDeq<DT>::PERIOD;
  __shared__ __align__(16) _Float16 as_h[2][BM][QROW];
  __shared__ __align__(16) _Float16 as_l[2][BM][QROW];
  __shared__ __align__(16) _Float16 bs_h[2][BN][QROW];
  __shared__ __align__(16) _Float16 bs_l[LO ? 2 : 1][BN][QROW];
  __shared__ float sd[2][BN], sdm[2][BN], sxs[2][BM];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int M = g.M, K = g.K, nk = K / QBK, nsb = K / QK_K;
  const int mtiles = (M + BM - 1) / BM;
  // Workgroup b runs on XCD b % 8. xcd_remap 2 (mtiles % 8 == 0): XCD x takes the M tiles
  // m % 8 == x and every N tile, so its activation rows stay resident in its L2 while the
  // weights stream (each XCD reads the weights once; the activation is read once per XCD instead
  // of once per N tile). xcd_remap 1: XCD x takes a contiguous run of tiles (all M tiles of its
  // N tiles share the weight tile in L2).
  int mt, ntile;
  if (g.xcd_remap == 2) {
    const int x = blockIdx.x % 8, j = blockIdx.x / 8, mpx = mtiles / 8;
    mt = x + 8 * (j % mpx);
    ntile = j / mpx;
  } else {
    int tile = blockIdx.x;
    if (g.xcd_remap == 1) {
      const int per = gridDim.x / 8;
      tile = (blockIdx.x % 8) * per + blockIdx.x / 8;
    }
    mt = tile % mtiles;
    ntile = tile / mtiles;
  }
  const int s = ntile < g.tile_start[1] ? 0 : (ntile < g.tile_start[2] ? 1 : 2);
  const uint8_t* w = s == 0 ? g.w[0] : (s == 1 ? g.w[1] : g.w[2]);
  float* out = s == 0 ? g.out[0] : (s == 1 ? g.out[1] : g.out[2]);
  const int N = s == 0 ? g.n[0] : (s == 1 ? g.n[1] : g.n[2]);
  const int ts = s == 0 ? 0 : (s == 1 ? g.tile_start[1] : g.tile_start[2]);
  const int m0 = mt * BM, n0 = (ntile - ts) * BN;
  const size_t row_bytes = g.row_bytes;

  const int b_row = tid >> 2, b_run = tid & 3;
  int b_n[BR];
#pragma unroll
  for (int r = 0; r < BR; ++r) b_n[r] = min(n0 + b_row + 64 * r, N - 1);
  // D stages of raw operand bytes in flight: slot i of the register ring holds stage kt with
  // kt % D == i; a slot is refilled with stage kt + D right after stage kt is moved to LDS.
  constexpr int D = 4;
  struct Slot {
    qu4_t arh[AU], arl[AU];
    float axs;
    QDeq<DT> braw[BR];
  };
  Slot ring[D];

  auto fetch = [&](int kt, Slot& sl) {
    const int k0 = kt * QBK;
#pragma unroll
    for (int u = 0; u < AU; ++u) {
      const int idx = tid + 256 * u, row = idx >> 2, c8 = idx & 3;
      const size_t off = (size_t)min(m0 + row, M - 1) * K + k0 + 8 * c8;
      sl.arh[u] = *reinterpret_cast<const qu4_t*>(g.xh + off);
      sl.arl[u] = *reinterpret_cast<const qu4_t*>(g.xl + off);
    }
    if (DT == DT_Q4K && tid < BM) sl.axs = g.xs[(size_t)min(m0 + tid, M - 1) * (K / 32) + kt];
#pragma unroll
    for (int r = 0; r < BR; ++r) sl.braw[r].load(w, row_bytes, b_n[r], k0 + 8 * b_run, nsb);
  };
  auto stage = [&](int kt, int buf, const Slot& sl) {
#pragma unroll
    for (int u = 0; u < AU; ++u) {
      const int idx = tid + 256 * u, row = idx >> 2, c8 = idx & 3;
      *reinterpret_cast<qu4_t*>(&as_h[buf][row][8 * c8]) = sl.arh[u];
      *reinterpret_cast<qu4_t*>(&as_l[buf][row][8 * c8]) = sl.arl[u];
    }
    if (DT == DT_Q4K && tid < BM) sxs[buf][tid] = sl.axs;
#pragma unroll
    for (int r = 0; r < BR; ++r) {
      uint4 hi, lo;
      float d, dm;
      sl.braw[r].decode(kt * QBK + 8 * b_run, hi, lo, d, dm);
      const int row = b_row + 64 * r;
      *reinterpret_cast<uint4*>(&bs_h[buf][row][8 * b_run]) = hi;
      if constexpr (LO) *reinterpret_cast<uint4*>(&bs_l[LO ? buf : 0][row][8 * b_run]) = lo;
      if (b_run == 0) {
        sd[buf][row] = d;
        sdm[buf][row] = dm;
      }
    }
  };

  qf4_t acc[MT][NT], part[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      acc[i][j] = qf4_t{0.f, 0.f, 0.f, 0.f};
      part[i][j] = qf4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
  for (int i = 0; i < D; ++i) fetch(min(i, nk - 1), ring[i]);
  stage(0, 0, ring[0]);
  fetch(min(D, nk - 1), ring[0]);
  __syncthreads();
  const int fr = lane & 15, fk = 8 * (lane >> 4);
  for (int kt0 = 0; kt0 < nk; kt0 += D) {
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const int kt = kt0 + u;
      if (kt >= nk) break;
      const int buf = kt & 1;
      qu4_t ah[MT], al[MT], bh[NT], bl[NT];
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        ah[i] = *reinterpret_cast<const qu4_t*>(&as_h[buf][wave * WM + 16 * i + fr][fk]);
        al[i] = *reinterpret_cast<const qu4_t*>(&as_l[buf][wave * WM + 16 * i + fr][fk]);
      }
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        bh[j] = *reinterpret_cast<const qu4_t*>(&bs_h[buf][16 * j + fr][fk]);
        if constexpr (LO) bl[j] = *reinterpret_cast<const qu4_t*>(&bs_l[LO ? buf : 0][16 * j + fr][fk]);
      }
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const qh8_t a_h = __builtin_bit_cast(qh8_t, ah[i]), a_l = __builtin_bit_cast(qh8_t, al[i]);
          const qh8_t b_h = __builtin_bit_cast(qh8_t, bh[j]);
          part[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_h, b_h, part[i][j], 0, 0, 0);
          part[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_l, b_h, part[i][j], 0, 0, 0);
          if constexpr (LO) {
            const qh8_t b_l = __builtin_bit_cast(qh8_t, bl[j]);
            part[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_h, b_l, part[i][j], 0, 0, 0);
          }
        }
      // Q4_K min term of this 32-block: acc[m][n] -= (dmin*m_b)[n] * sum_b a[m]
      if constexpr (DT == DT_Q4K) {
        float xsv[MT][4];
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) xsv[i][r] = sxs[buf][wave * WM + 16 * i + 4 * (lane >> 4) + r];
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const float dmn = sdm[buf][16 * j + fr];
#pragma unroll
          for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] -= dmn * xsv[i][r];
        }
      }
      // end of a d block: fold d[n] * (its partial) into the output accumulator
      if ((kt + 1) % PERIOD == 0) {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const float dn = sd[buf][16 * j + fr];
#pragma unroll
          for (int i = 0; i < MT; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] += dn * part[i][j][r];
            part[i][j] = qf4_t{0.f, 0.f, 0.f, 0.f};
          }
        }
      }
      {
        // unconditional with clamped stage indices, so the number of loads in flight is the same
        // on every path and each stage waits only for its own slot (the tail re-reads the last
        // stage and stages it into the idle buffer)
        Slot& sl = ring[(u + 1) % D];
        stage(min(kt + 1, nk - 1), buf ^ 1, sl);
        fetch(min(kt + 1 + D, nk - 1), sl);
      }
      __syncthreads();
    }
  }

  const float* resid = s == 0 ? g.resid : nullptr;
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int n = n0 + 16 * j + fr;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wave * WM + 16 * i + 4 * (lane >> 4) + r;
        if (m < M && n < N) {
          float v = acc[i][j][r];
          if (resid) v = resid[(size_t)m * N + n] + v;
          out[(size_t)m * N + n] = v;
        }
      }
    }
}

}  // namespace

bool gemm_q_ok(int dt, const void* w, int K) {
  switch (dt) {
    case DT_Q4K: return K % QK_K == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0;
    case DT_Q6K: return K % QK_K == 0 && (reinterpret_cast<uintptr_t>(w) & 1) == 0;
    case DT_Q6K_R: return K % QK_K == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0;
    case DT_Q8_0: return K % 32 == 0 && (reinterpret_cast<uintptr_t>(w) & 1) == 0;
    default: return false;
  }
}

void launch_block_sums(const float* a, int M, int K, float* xs, hipStream_t st) {
  if (K % 32 != 0) fail(ST_OP, "block_sums: K must be a multiple of 32");
  const size_t nb = (size_t)M * (K / 32);
  hipLaunchKernelGGL(block_sums_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, st, a, nb, xs);
}

template <int DT, int BM, int BN>
static void gemm_q_launch(GemmQArgs g, hipStream_t st) {
  int t = 0;
  for (int i = 0; i < g.nseg; ++i) {
    g.tile_start[i] = t;
    t += (g.n[i] + BN - 1) / BN;
  }
  for (int i = g.nseg; i <= 3; ++i) g.tile_start[i] = t;
  const int mtiles = (g.M + BM - 1) / BM;
  const int tiles = mtiles * t;
  static int mode = -1;
  if (mode < 0) {
    const char* e = getenv("IEK_GEMM_XCD");  // 1: N-tile runs per XCD (tuning)
    mode = e ? atoi(e) : 2;
  }
  g.xcd_remap = (mode == 2 && mtiles % 8 == 0) ? 2 : (tiles % 8 == 0 ? 1 : 0);
  hipLaunchKernelGGL((gemm_q_kernel<DT, BM, BN>), dim3(tiles), dim3(256), 0, st, g);
}

// Tile shape: 64 x 64 by default (measured fastest at the Mistral-7B prefill shapes: the larger
// tiles lose more to occupancy than they gain in operand reuse); IEK_GEMM_TILE overrides.
template <int DT>
static void gemm_q_dt(GemmQArgs g, hipStream_t st) {
  auto tiles = [&](int bm, int bn) {
    size_t n = 0;
    for (int i = 0; i < g.nseg; ++i) n += (g.n[i] + bn - 1) / bn;
    return (size_t)((g.M + bm - 1) / bm) * n;
  };
  static int force = -2;
  if (force == -2) {
    const char* e = getenv("IEK_GEMM_TILE");  // 0: 64x64, 1: 64x128, 2: 128x128 (tuning)
    force = e ? atoi(e) : -1;
  }
  (void)tiles;
  if (force == 2) gemm_q_launch<DT, 128, 128>(g, st);
  else if (force == 1) gemm_q_launch<DT, 64, 128>(g, st);
  else gemm_q_launch<DT, 64, 64>(g, st);
}

void launch_gemm_q(int dt, const GemmQSeg* segs, int nseg, const __half* xh, const __half* xl, const float* xs, int M,
                   int K, const float* resid, hipStream_t st) {
  if (nseg < 1 || nseg > 3 || M < 1) fail(ST_OP, "gemm_q: 1..3 segments and M >= 1");
  GemmQArgs g{};
  g.nseg = nseg;
  for (int i = 0; i < nseg; ++i) {
    if (!gemm_q_ok(dt, segs[i].w, K) || segs[i].n < 1) fail(ST_OP, "gemm_q: unsupported weight type, alignment or shape");
    g.w[i] = (const uint8_t*)segs[i].w;
    g.out[i] = segs[i].out;
    g.n[i] = segs[i].n;
  }
  g.M = M;
  g.K = K;
  g.xh = xh;
  g.xl = xl;
  g.xs = xs;
  g.resid = resid;
  const size_t nsb = (size_t)(K / QK_K);
  switch (dt) {
    case DT_Q4K: g.row_bytes = nsb * Q4K_BYTES; break;
    case DT_Q6K: g.row_bytes = nsb * Q6K_BYTES; break;
    case DT_Q6K_R: g.row_bytes = q6r_row_bytes(nsb); break;
    default: g.row_bytes = (size_t)(K / 32) * Q8_0_BYTES; break;
  }
  if (dt == DT_Q4K && !xs) fail(ST_OP, "gemm_q: Q4_K needs the per-32 activation sums");
  switch (dt) {
    case DT_Q4K: gemm_q_dt<DT_Q4K>(g, st); break;
    case DT_Q6K: gemm_q_dt<DT_Q6K>(g, st); break;
    case DT_Q6K_R: gemm_q_dt<DT_Q6K_R>(g, st); break;
    default: gemm_q_dt<DT_Q8_0>(g, st); break;
  }
}

}  // namespace iek
