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
  // split-K (wave-tiled kernel, one segment): the second half of the superblocks writes its
  // partial sums to kpart [M, N], which a follow-up pass adds to out
  int ksplit;
  float* kpart;
  // gate/up + SwiGLU (wave-tiled kernel instantiated with GLU, segments 0 = gate and 1 = up of
  // equal N): each wave computes 32 gate and the same 32 up columns; the epilogue writes
  // act = silu(gate) * up as the down projection's input: fp16 (hi, lo) planes [M][N], their
  // per-32 sums (glu_sums, optional) and the f32 act (glu_out, optional)
  _Float16 *glu_h, *glu_l, *glu_sums;
  float* glu_out;
  int* ovf;  // GLU: set when an act value or per-32 sum is beyond the fp16 pair's range
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
  IEK_DEV void decode(int k0, uint4& hi, uint4& lo, float& d) const {
    const int quarter = ((k0 & 255) & 127) >> 5;
    d = half_bits_to_float(sd >> 16);
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
  IEK_DEV void decode(int, uint4& hi, uint4& lo, float& d) const {
    d = half_bits_to_float(d16);
    _Float16 h[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = (_Float16)(int)(int8_t)((q[i >> 1] >> (8 * (i & 1))) & 0xFFu);
    hi = make_uint4(hpack(h[0], h[1]), hpack(h[2], h[3]), hpack(h[4], h[5]), hpack(h[6], h[7]));
    lo = make_uint4(0, 0, 0, 0);
  }
};

// Per-32 row sums of the activation (Q4_K's min term), summed in f32 and stored as an fp16 pair
// over two planes of nb halves: hi[m * (K/32) + b] + lo[...] = sum of a[m, 32b .. 32b+31].
__global__ __launch_bounds__(256) void block_sums_kernel(const float* __restrict__ a, size_t nb,
                                                         _Float16* __restrict__ hi, _Float16* __restrict__ lo) {
#pragma clang fp contract(off)
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nb) return;
  const float4* p = reinterpret_cast<const float4*>(a + 32 * i);
  float s = 0.f;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const float4 v = p[t];
    s += (v.x + v.y) + (v.z + v.w);
  }
  const _Float16 h = (_Float16)s;
  hi[i] = h;
  lo[i] = (_Float16)(s - (float)h);
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
  __shared__ float sd[2][BN];

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
#pragma unroll
    for (int r = 0; r < BR; ++r) {
      uint4 hi, lo;
      float d;
      sl.braw[r].decode(kt * QBK + 8 * b_run, hi, lo, d);
      const int row = b_row + 64 * r;
      *reinterpret_cast<uint4*>(&bs_h[buf][row][8 * b_run]) = hi;
      if constexpr (LO) *reinterpret_cast<uint4*>(&bs_l[LO ? buf : 0][row][8 * b_run]) = lo;
      if (b_run == 0) sd[buf][row] = d;
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

// ---- K-quants: 64 x 64 wave tiles, weights dequantised straight into MFMA operand registers ----
//
// A workgroup of four waves owns a BM x BN output tile (waves WGM x WGN, each 64 x 64 = 4 x 4
// MFMA tiles). K advances in 64-wide stages (one Q4_K sub-block pair). The activation pair is
// staged through LDS (double-buffered, XOR-swizzled 16-byte chunks); each wave decodes the weights
// of its own 64 columns into registers: lane (column n, k group g) holds k = 8g .. 8g+7 of the
// stage's two sub-blocks, built as exact fp16 integers w' = sc * q from the nibbles by a byte
// permute under the exponent byte 0x64 (1024 + q) and one packed fp16 FMA (1024 + q) * sc -
// 1024 * sc, which is exact because the result sc * q <= 945 is. An MFMA output column is the
// lane's own weight column, so the superblock factors d and dmin apply per lane. The min term
// -dmin * sum_b m_b * sum(a over sub-block b) runs on the matrix cores once per superblock: the
// per-32 activation sums (fp16 pair) against the eight 6-bit mins.
typedef _Float16 qh2_t __attribute__((ext_vector_type(2)));

IEK_DEV uint32_t pk_fma16(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(qh2_t, a), __builtin_bit_cast(qh2_t, b),
                                                                __builtin_bit_cast(qh2_t, c)));
}
// (1024 + byte) as fp16 in each half: bytes of x picked by the selector's bytes 0 and 2.
IEK_DEV uint32_t mag16(uint32_t x, uint32_t sel) { return __builtin_amdgcn_perm(0x64646464u, x, sel); }
constexpr uint32_t SEL01 = 0x04010400u, SEL23 = 0x04030402u;
constexpr uint32_t H2_M1024 = 0xE400E400u;  // (-1024, -1024)
constexpr uint32_t H2_ONE = 0x3C003C00u;    // (1, 1)

// {sc, sc} and {-1024 sc, -1024 sc} for the 6-bit scale in byte `i` of `scs`.
IEK_DEV void q4k_scale2(uint32_t scs, uint32_t i, uint32_t& s2, uint32_t& c2) {
  s2 = pk_fma16(mag16(scs, 0x04000400u | i | (i << 16)), H2_ONE, H2_M1024);
  c2 = pk_fma16(s2, H2_M1024, 0u);
}

// B operand of sub-block 2P + H (H = 0: low nibbles, 1: high nibbles) for one 16-column tile.
template <int P, int H>
IEK_DEV qu4_t q4k_b(const uint4& hdr, uint2 q) {
  const uint32_t scs = P < 2 ? (hdr.y & 0x3F3F3F3Fu) : ((hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u));
  uint32_t sc, c;
  q4k_scale2(scs, 2 * (P & 1) + H, sc, c);
  const uint32_t x = (q.x >> (4 * H)) & 0x0F0F0F0Fu, y = (q.y >> (4 * H)) & 0x0F0F0F0Fu;
  return qu4_t{pk_fma16(mag16(x, SEL01), sc, c), pk_fma16(mag16(x, SEL23), sc, c), pk_fma16(mag16(y, SEL01), sc, c),
               pk_fma16(mag16(y, SEL23), sc, c)};
}

// The eight 6-bit mins of a superblock as fp16 (k groups 0 and 1; zero for groups 2 and 3).
IEK_DEV qu4_t q4k_mins(const uint4& hdr, bool live) {
  const uint32_t m03 = hdr.z & 0x3F3F3F3Fu;
  const uint32_t m47 = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
  qu4_t r{pk_fma16(mag16(m03, SEL01), H2_ONE, H2_M1024), pk_fma16(mag16(m03, SEL23), H2_ONE, H2_M1024),
          pk_fma16(mag16(m47, SEL01), H2_ONE, H2_M1024), pk_fma16(mag16(m47, SEL23), H2_ONE, H2_M1024)};
  return live ? r : qu4_t{0u, 0u, 0u, 0u};
}

IEK_DEV qf4_t mfma16(qu4_t a, qu4_t b, qf4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(qh8_t, a), __builtin_bit_cast(qh8_t, b), c, 0, 0, 0);
}

// Buffer resource over `bytes` bytes at `p` (raw, unswizzled; word 3 as gfx9 data loads expect).
IEK_DEV __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
IEK_DEV qu4_t ld_b128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}
IEK_DEV uint2 ld_b64(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}

IEK_DEV uint32_t ld_b32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
IEK_DEV uint32_t ld_b16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}

// Weight formats of the wave-tiled kernel. Each provides the raw bytes of one 64-wide stage for
// the lane's four columns (`Raw`), the per-superblock factors (`Hdr`), and the B operands of
// half-step (P, H): hi, plus lo when the integer weight w' does not fit fp16 (LO).
struct Q4KB {
  static constexpr bool LO = false, MINS = true;
  struct Raw {
    uint2 q[4];
  };
  struct Hdr {
    uint4 h[4];
  };
  IEK_DEV static void fetch(__amdgpu_buffer_rsrc_t r0, __amdgpu_buffer_rsrc_t r1, const uint32_t (&vb)[4], int lg,
                            int kt, Raw& o) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o.q[j] = ld_b64(j < 2 ? r0 : r1, vb[j] + 16 + 8 * lg, (uint32_t)((kt >> 2) * Q4K_BYTES + 32 * (kt & 3)));
  }
  IEK_DEV static void fetch_hdr(__amdgpu_buffer_rsrc_t r0, __amdgpu_buffer_rsrc_t r1, const uint32_t (&vb)[4], int,
                                int sb, int, Hdr& o) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o.h[j] = __builtin_bit_cast(uint4, ld_b128(j < 2 ? r0 : r1, vb[j], (uint32_t)(sb * Q4K_BYTES)));
  }
  template <int P, int H>
  IEK_DEV static void deq(const Hdr& hd, const Raw& q, qu4_t (&bh)[4], qu4_t (&)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) bh[j] = q4k_b<P, H>(hd.h[j], q.q[j]);
  }
  IEK_DEV static float d(const Hdr& hd, int j) { return half_bits_to_float(hd.h[j].x); }
  IEK_DEV static float dmin(const Hdr& hd, int j) { return half_bits_to_float(hd.h[j].x >> 16); }
  // A superblock with d = +-0 contributes only its min term: zero its eight scales (the mins,
  // in z and the high nibbles of w, stay).
  IEK_DEV static void zero_d_scales(Hdr& hd) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if ((hd.h[j].x & 0x7FFFu) == 0) {
        hd.h[j].y = 0u;
        hd.h[j].w &= 0xF0F0F0F0u;
      }
  }
  IEK_DEV static qu4_t mins(const Hdr& hd, int j, bool live) { return q4k_mins(hd.h[j], live); }
};

// Q6_K from the regrouped rows (DT_Q6K_R: per superblock four 48-byte lane chunks [ql of quarters
// 0/2 | ql of quarters 1/3 | qh], then per-chunk scale dwords, then d). Stage P covers half
// P >> 1 and quarters 2(P & 1) + H; lane group g reads chunk 2(P >> 1) + (g >> 1), bytes 8(g & 1).
// w' = sc * (q - 32) reaches 4096, so it is an fp16 pair: hi = fp16(w'), lo = w' - hi (|lo| <= 1).
struct Q6RB {
  static constexpr bool LO = true, MINS = false;
  struct Raw {
    uint2 l0[4], l1[4], h[4];
  };
  struct Hdr {
    uint32_t sc[2][4], d[4];
  };
  IEK_DEV static void fetch(__amdgpu_buffer_rsrc_t r0, __amdgpu_buffer_rsrc_t r1, const uint32_t (&vb)[4], int lg,
                            int kt, Raw& o) {
    const uint32_t so = (uint32_t)((kt >> 2) * 192 + 48 * 2 * ((kt & 3) >> 1));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const __amdgpu_buffer_rsrc_t r = j < 2 ? r0 : r1;
      const uint32_t v = vb[j] + 48 * (lg >> 1) + 8 * (lg & 1);
      o.l0[j] = ld_b64(r, v, so);
      o.l1[j] = ld_b64(r, v + 16, so);
      o.h[j] = ld_b64(r, v + 32, so);
    }
  }
  IEK_DEV static void fetch_hdr(__amdgpu_buffer_rsrc_t r0, __amdgpu_buffer_rsrc_t r1, const uint32_t (&vb)[4], int lg,
                                int sb, int nsb, Hdr& o) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const __amdgpu_buffer_rsrc_t r = j < 2 ? r0 : r1;
      const uint32_t v = vb[j] + (uint32_t)nsb * 192 + 4 * (lg >> 1);
      o.sc[0][j] = ld_b32(r, v, 16u * sb);
      o.sc[1][j] = ld_b32(r, v + 8, 16u * sb);
      o.d[j] = ld_b16(r, vb[j] + (uint32_t)nsb * 208, 2u * sb);
    }
  }
  template <int P, int H>
  IEK_DEV static void deq(const Hdr& hd, const Raw& q, qu4_t (&bh)[4], qu4_t (&bl)[4]) {
    constexpr int qd = 2 * (P & 1) + H;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // {sc, sc} from the signed scale byte: (sc + 128) under the exponent byte, minus 1152
      const uint32_t scb = hd.sc[P >> 1][j] ^ 0x80808080u;
      const qh2_t s2 = __builtin_bit_cast(qh2_t, mag16(scb, 0x04000400u | qd | (qd << 16))) - qh2_t{1152.0f16, 1152.0f16};
      const uint2 l = H ? q.l1[j] : q.l0[j], hb = q.h[j];
      const uint32_t qx = ((l.x >> (4 * (P & 1))) & 0x0F0F0F0Fu) | (((hb.x >> (2 * qd)) << 4) & 0x30303030u);
      const uint32_t qy = ((l.y >> (4 * (P & 1))) & 0x0F0F0F0Fu) | (((hb.y >> (2 * qd)) << 4) & 0x30303030u);
      const uint32_t v[4] = {mag16(qx, SEL01), mag16(qx, SEL23), mag16(qy, SEL01), mag16(qy, SEL23)};
      uint32_t hi[4], lo[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const qh2_t qm = __builtin_bit_cast(qh2_t, v[t]) - qh2_t{1056.0f16, 1056.0f16};  // q - 32, exact
        const qh2_t h = qm * s2;
        hi[t] = __builtin_bit_cast(uint32_t, h);
        lo[t] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(qm, s2, -h));  // exact remainder
      }
      bh[j] = qu4_t{hi[0], hi[1], hi[2], hi[3]};
      bl[j] = qu4_t{lo[0], lo[1], lo[2], lo[3]};
    }
  }
  IEK_DEV static float d(const Hdr& hd, int j) { return half_bits_to_float(hd.d[j]); }
  IEK_DEV static float dmin(const Hdr&, int) { return 0.f; }
  IEK_DEV static void zero_d_scales(Hdr& hd) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if ((hd.d[j] & 0x7FFFu) == 0) hd.sc[0][j] = hd.sc[1][j] = 0u;
  }
  IEK_DEV static qu4_t mins(const Hdr&, int, bool) { return qu4_t{0u, 0u, 0u, 0u}; }
};

template <class T>
IEK_DEV void kq_deq(int p, int h, const typename T::Hdr& hd, const typename T::Raw& q, qu4_t (&bh)[4], qu4_t (&bl)[4]) {
  switch (2 * p + h) {
    case 0: T::template deq<0, 0>(hd, q, bh, bl); break;
    case 1: T::template deq<0, 1>(hd, q, bh, bl); break;
    case 2: T::template deq<1, 0>(hd, q, bh, bl); break;
    case 3: T::template deq<1, 1>(hd, q, bh, bl); break;
    case 4: T::template deq<2, 0>(hd, q, bh, bl); break;
    case 5: T::template deq<2, 1>(hd, q, bh, bl); break;
    case 6: T::template deq<3, 0>(hd, q, bh, bl); break;
    default: T::template deq<3, 1>(hd, q, bh, bl); break;
  }
}

// SwiGLU epilogue of a gate/up tile (GLU): column groups 0-1 of a wave are gate columns and 2-3
// the same up columns, so each lane holds matching gate / up sums. act = silu(g) * u with the
// arithmetic of swiglu_split_kernel (src/ops/swiglu.rs:24-36: two-branch stable sigmoid,
// (g * s) * u), then its fp16 (hi, lo) pair and, per 32 columns, the sum in emit_split8's order
// (pairs, pairs of pairs, then the eight quarter sums one after the other from zero), so the down
// projection's input has the bits the separate pass would write.
// (Staging the fp16 pair through LDS for 16-byte stores measured no faster.)
template <int TM, typename AccT>
IEK_DEV void glu_epilogue(const GemmQArgs& g, const AccT& acc, const float (&Dc)[4], bool rescaled, int m0, int wcol,
                          int lane) {
#pragma clang fp contract(off)
  const int lr = lane & 15, lg = lane >> 4;
  const int M = g.M, N = g.n[0];
  const size_t nb = (size_t)N / 32;
  bool big = false;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + 16 * i + 4 * lg + r;
      float vv[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = wcol + 16 * j + lr;
        const float x = rescaled ? acc[i][j][r] * Dc[j] : acc[i][j][r];
        const float u = rescaled ? acc[i][j + 2][r] * Dc[j + 2] : acc[i][j + 2][r];
        float sg;
        if (x >= 0.0f) {
          const float z = expf(-x);
          sg = 1.0f / (1.0f + z);
        } else {
          const float z = expf(x);
          sg = z / (1.0f + z);
        }
        const float v = x * sg * u;
        if (m < M && n < N) {
          const size_t o = (size_t)m * N + n;
          const _Float16 h = (_Float16)v;
          g.glu_h[o] = h;
          g.glu_l[o] = (_Float16)(v - (float)h);
          if (g.glu_out) g.glu_out[o] = v;
          big |= fabsf(v) > F16_PAIR_MAX;
        }
        vv[j] = v;
      }
      if (g.glu_sums) {
        // (v0 + v1) + (v2 + v3) over each aligned group of four columns, at the group's first lane
        float qs[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float s1 = vv[j] + __shfl_xor(vv[j], 1, 64);
          qs[j] = s1 + __shfl_xor(s1, 2, 64);
        }
        // the wave's 32 columns are one block; its eight quarter sums sit at lanes 0, 4, 8, 12 of
        // the lane's row of 16 (same m) for j = 0, then j = 1
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int t = 0; t < 4; ++t) sum += __shfl(qs[j], (lane & ~15) + 4 * t, 64);
        if (lr == 0 && m < M && wcol < N) {
          const size_t o = (size_t)m * nb + wcol / 32;
          const _Float16 h = (_Float16)sum;
          g.glu_sums[o] = h;
          g.glu_sums[(size_t)M * nb + o] = (_Float16)(sum - (float)h);
          big |= fabsf(sum) > F16_PAIR_MAX;
        }
      }
    }
  if (big && g.ovf) *g.ovf = 1;
}

// TM: 16-row MFMA tiles per wave along M (a wave owns 16 TM x 64); WGM x WGN waves.
// OCC: waves per SIMD the register allocation must allow (2 caps each wave at 256 registers).
// FM, how the superblock factor d enters the f32 sum:
//  0: per superblock, acc += d * part (a second full set of accumulators, the partials);
//  2: rescaled: the MFMAs accumulate straight into acc, which holds sum / D (D = d of the current
//     superblock); at a superblock end acc = acc * (D / D') - (dmin / D') * mins-term with D' the
//     next superblock's d, and the output is acc * D. Two VALU ops per element per superblock, no
//     partials. A superblock with d = 0 keeps D (its scales are zeroed, so only its min term
//     counts); the rescale's rounding (a few ulp of the running sum per superblock) is far inside
//     the f32 reordering bound.
// GLU: gate/up with the SwiGLU epilogue (GemmQArgs::glu); a tile is 32 * WGN act columns.
template <class T, int WGM, int WGN, int DA, int TM, int OCC = 1, int FM = 0, bool GLU = false>
__global__ __launch_bounds__(64 * WGM * WGN, OCC) void gemm_kq_kernel(GemmQArgs g) {
  constexpr int NT = 64 * WGM * WGN;  // threads
  constexpr int WR = 16 * TM;         // rows per wave
  constexpr int BM = WR * WGM, BN = 64 * WGN;
  constexpr int PL = BM * 8;        // 16-byte chunks per plane per stage (BM rows x 64 halves)
  constexpr int AR = PL / NT;       // chunk rows per thread per plane per stage
  static_assert(AR >= 1 && PL % NT == 0, "activation tile must divide over the threads");
  constexpr int DB = 2;             // stages of raw weight bytes in flight and (DA) of activation
                                    // stages; both divide the 4 stages of a superblock, so ring
                                    // slots are static
  static_assert(4 % DA == 0 && 4 % DB == 0, "ring slots are indexed by stage within the superblock");
  __shared__ __align__(16) qu4_t As[2][2 * PL];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int M = g.M, K = g.K, kb = K / 32, nsb = K / QK_K;
  const int mtiles = (M + BM - 1) / BM;
  // split-K: workgroups [ks * per_split, (ks + 1) * per_split) take superblocks [sb_lo, sb_hi)
  const int per_split = gridDim.x / g.ksplit, ks = blockIdx.x / per_split;
  const int sb_lo = ks == 0 ? 0 : nsb / 2, sb_hi = (g.ksplit == 1 || ks == 1) ? nsb : nsb / 2;
  const int kt_last = 4 * sb_hi - 1;
  int tile = blockIdx.x - ks * per_split;
  if (g.xcd_remap == 1) {
    const int per = per_split / 8;
    tile = (tile % 8) * per + tile / 8;
  }
  const int mt = tile % mtiles, ntile = tile / mtiles;
  const int s = GLU ? 0 : (ntile < g.tile_start[1] ? 0 : (ntile < g.tile_start[2] ? 1 : 2));
  const uint8_t* w = s == 0 ? g.w[0] : (s == 1 ? g.w[1] : g.w[2]);
  float* out = s == 0 ? g.out[0] : (s == 1 ? g.out[1] : g.out[2]);
  const int N = s == 0 ? g.n[0] : (s == 1 ? g.n[1] : g.n[2]);
  const int ts = s == 0 ? 0 : (s == 1 ? g.tile_start[1] : g.tile_start[2]);
  const int m0 = mt * BM;
  // GLU: the wave's 32 act columns (column groups 0-1 read gate rows, 2-3 the same up rows)
  const int wcol = GLU ? (BN / 2) * ntile + 32 * wn : (ntile - ts) * BN + 64 * wn;
  const int lr = lane & 15, lg = lane >> 4;

  // Operand streams as buffer loads: one descriptor per array, 32-bit per-lane offsets, the
  // stage's advance in the scalar offset.
  const __amdgpu_buffer_rsrc_t rw = buf_rsrc(w, (uint32_t)(g.row_bytes * (size_t)N));
  const __amdgpu_buffer_rsrc_t rw2 = GLU ? buf_rsrc(g.w[1], (uint32_t)(g.row_bytes * (size_t)N)) : rw;
  const __amdgpu_buffer_rsrc_t rxh = buf_rsrc(g.xh, (uint32_t)((size_t)M * K * 2));
  const __amdgpu_buffer_rsrc_t rxl = buf_rsrc(g.xl, (uint32_t)((size_t)M * K * 2));
  const __amdgpu_buffer_rsrc_t rxs = buf_rsrc(g.xs, T::MINS ? (uint32_t)((size_t)M * kb * 4) : 0u);
  uint32_t vb[4];  // weight row of the lane's column in each 16-column tile
#pragma unroll
  for (int j = 0; j < 4; ++j)
    vb[j] = (uint32_t)((size_t)min(wcol + 16 * (GLU ? (j & 1) : j) + lr, N - 1) * g.row_bytes);
  uint32_t va[AR];  // activation rows staged by this thread (both planes)
#pragma unroll
  for (int u = 0; u < AR; ++u)
    va[u] = (uint32_t)(min(m0 + (tid >> 3) + (NT / 8) * u, M - 1) * K + 8 * (tid & 7)) * 2u;
  uint32_t vx[TM];  // per-32 sums: k group 0 reads the hi plane, 1 the lo plane
#pragma unroll
  for (int i = 0; i < TM; ++i)
    vx[i] = (uint32_t)(min(m0 + WR * wm + 16 * i + lr, M - 1) * kb + ((lg & 1) ? M * kb : 0)) * 2u;

  struct ASlot {
    qu4_t a[2 * AR];
  };
  ASlot ra[DA];
  typename T::Raw rb[DB];
  typename T::Hdr hdr, hdrn;  // factors of the current and the next superblock
  qu4_t xsv[TM];

  auto fetch_a = [&](int kt, ASlot& sl) {
#pragma unroll
    for (int u = 0; u < AR; ++u) {
      sl.a[u] = ld_b128(rxh, va[u], 128u * kt);
      sl.a[AR + u] = ld_b128(rxl, va[u], 128u * kt);
    }
  };
  auto store_a = [&](int buf, const ASlot& sl) {
    const int c = tid & 7;
#pragma unroll
    for (int u = 0; u < AR; ++u) {
      const int row = (tid >> 3) + (NT / 8) * u;
      As[buf][row * 8 + (c ^ (row & 7))] = sl.a[u];
      As[buf][PL + row * 8 + (c ^ (row & 7))] = sl.a[AR + u];
    }
  };
  auto fetch_xs = [&](int sb) {
#pragma unroll
    for (int i = 0; i < TM; ++i) xsv[i] = ld_b128(rxs, vx[i], 16u * sb);
  };

  qf4_t acc[TM][4], part[TM][4];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[i][j] = qf4_t{0.f, 0.f, 0.f, 0.f};
      part[i][j] = qf4_t{0.f, 0.f, 0.f, 0.f};
    }

  // prologue: A(0) in LDS, A(1) .. A(DA) and B(0) .. B(DB-1) in flight. The loads leave in the
  // order the loop's last stage issues them (an activation stage, then a weight stage), so the
  // wait counts at the loop head are the same on entry and on the back edge.
  const int kt_lo = 4 * sb_lo;
  T::fetch_hdr(rw, rw2, vb, lg, sb_lo, nsb, hdr);
  float Dc[4] = {1.f, 1.f, 1.f, 1.f};  // FM 2: the scale acc is held at, per column tile
#pragma unroll
  for (int i = 0; i < DB - 1; ++i) T::fetch(rw, rw2, vb, lg, min(kt_lo + i, kt_last), rb[i]);
  fetch_a(kt_lo, ra[0]);
  store_a(0, ra[0]);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 1; i <= DA; ++i) fetch_a(min(kt_lo + i, kt_last), ra[i % DA]);
  __builtin_amdgcn_sched_barrier(0);
  T::fetch(rw, rw2, vb, lg, min(kt_lo + DB - 1, kt_last), rb[DB - 1]);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();

  for (int sb = sb_lo; sb < sb_hi; ++sb) {
    const int kt0 = 4 * sb;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int kt = kt0 + p, buf = p & 1;
      // A(kt+1) into the other LDS buffer (last read before the previous barrier), then refill
      // (scheduling fences keep every fetch where it is written: the compiler would otherwise sink
      // loads next to their use and expose their latency)
      store_a(buf ^ 1, ra[(p + 1) % DA]);
      __builtin_amdgcn_sched_barrier(0);
      fetch_a(min(kt + 1 + DA, kt_last), ra[(p + 1) % DA]);
      // the next superblock's factors go out ahead of this stage's weight refill, so waiting
      // for them at the superblock end never waits for a younger load
      if (p == 0) T::fetch_hdr(rw, rw2, vb, lg, min(sb + 1, sb_hi - 1), nsb, hdrn);
      if (T::MINS && p == 2) fetch_xs(sb);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (FM == 2) {
        if (p == 0) T::zero_d_scales(hdr);
        qu4_t bh[2][4], bl[2][4];
        kq_deq<T>(p, 0, hdr, rb[p % DB], bh[0], bl[0]);
        kq_deq<T>(p, 1, hdr, rb[p % DB], bh[1], bl[1]);
        __builtin_amdgcn_sched_barrier(0);
        T::fetch(rw, rw2, vb, lg, min(kt + DB, kt_last), rb[p % DB]);
        __builtin_amdgcn_sched_barrier(0);
        qu4_t a4[2][4];
        auto rd4 = [&](int i, qu4_t (&x)[4]) {
          const int row = WR * wm + 16 * i + lr;
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const int ch = row * 8 + ((4 * hh + lg) ^ (row & 7));
            x[2 * hh] = As[buf][ch];
            x[2 * hh + 1] = As[buf][PL + ch];
          }
        };
        rd4(0, a4[0]);
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          if (i < TM - 1) rd4(i + 1, a4[(i + 1) & 1]);
          const qu4_t(&x)[4] = a4[i & 1];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc[i][j] = mfma16(x[0], bh[0][j], acc[i][j]);
            acc[i][j] = mfma16(x[1], bh[0][j], acc[i][j]);
            if constexpr (T::LO) acc[i][j] = mfma16(x[0], bl[0][j], acc[i][j]);
            acc[i][j] = mfma16(x[2], bh[1][j], acc[i][j]);
            acc[i][j] = mfma16(x[3], bh[1][j], acc[i][j]);
            if constexpr (T::LO) acc[i][j] = mfma16(x[2], bl[1][j], acc[i][j]);
          }
        }
        if (p == 3) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float dcur = T::d(hdr, j), dnext = T::d(hdrn, j);
            const float D = sb == sb_lo ? (dcur != 0.f ? dcur : 1.f) : Dc[j];
            const float Dn = dnext != 0.f ? dnext : D;
            const float inv = __builtin_amdgcn_rcpf(Dn);
            const float r = D * inv;
            if constexpr (T::MINS) {
              const float cm = T::dmin(hdr, j) * inv;
              const qu4_t mb = T::mins(hdr, j, lg < 2);
#pragma unroll
              for (int i = 0; i < TM; ++i) {
                const qf4_t mp = mfma16(xsv[i], mb, qf4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[i][j][e] = acc[i][j][e] * r - cm * mp[e];
              }
            } else {
#pragma unroll
              for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[i][j][e] *= r;
            }
            Dc[j] = Dn;
          }
          hdr = hdrn;
        }
        __syncthreads();
        continue;
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        qu4_t bh[4], bl[4];
        kq_deq<T>(p, h, hdr, rb[p % DB], bh, bl);
        if (h == 1) {
          __builtin_amdgcn_sched_barrier(0);
          T::fetch(rw, rw2, vb, lg, min(kt + DB, kt_last), rb[p % DB]);
          __builtin_amdgcn_sched_barrier(0);
        }
        // activation operands one m-tile ahead of the MFMAs that use them
        qu4_t ah[2], al[2];
        auto rd = [&](int i, qu4_t& x, qu4_t& y) {
          const int row = WR * wm + 16 * i + lr, ch = row * 8 + ((4 * h + lg) ^ (row & 7));
          x = As[buf][ch];
          y = As[buf][PL + ch];
        };
        rd(0, ah[0], al[0]);
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          if (i < TM - 1) rd(i + 1, ah[(i + 1) & 1], al[(i + 1) & 1]);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            part[i][j] = mfma16(ah[i & 1], bh[j], (p == 0 && h == 0) ? qf4_t{0.f, 0.f, 0.f, 0.f} : part[i][j]);
            part[i][j] = mfma16(al[i & 1], bh[j], part[i][j]);
            if constexpr (T::LO) part[i][j] = mfma16(ah[i & 1], bl[j], part[i][j]);
          }
        }
      }
      if (p == 3) {
        // superblock end: acc += d * part (- dmin * sum_b m_b * xs_b for Q4_K; the mins are zero
        // in k groups 2 and 3, so those lanes' activation sums drop out)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float d = T::d(hdr, j);
          if constexpr (T::MINS) {
            const float dmin = T::dmin(hdr, j);
            const qu4_t mb = T::mins(hdr, j, lg < 2);
#pragma unroll
            for (int i = 0; i < TM; ++i) {
              const qf4_t mp = mfma16(xsv[i], mb, qf4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[i][j][r] = (acc[i][j][r] + d * part[i][j][r]) - dmin * mp[r];
            }
          } else {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[i][j][r] += d * part[i][j][r];
          }
        }
        hdr = hdrn;
      }
      __syncthreads();
    }
  }

  if constexpr (GLU) {
    glu_epilogue<TM>(g, acc, Dc, FM == 2, m0, wcol, lane);
    return;
  }
  const float* resid = s == 0 && ks == 0 ? g.resid : nullptr;
  float* dst = ks == 0 ? out : g.kpart;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = wcol + 16 * j + lr;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + WR * wm + 16 * i + 4 * lg + r;
        if (m < M && n < N) {
          float v = FM == 2 ? acc[i][j][r] * Dc[j] : acc[i][j][r];
          if (resid) v = resid[(size_t)m * N + n] + v;
          dst[(size_t)m * N + n] = v;
        }
      }
    }
}

// out[i] += part[i]: the split-K reduction (after the first half wrote resid + its sum).
__global__ __launch_bounds__(256) void add_part_kernel(float* __restrict__ out, const float* __restrict__ part,
                                                      size_t n4) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
    float4 o = reinterpret_cast<float4*>(out)[i];
    const float4 q = reinterpret_cast<const float4*>(part)[i];
    o.x += q.x;
    o.y += q.y;
    o.z += q.z;
    o.w += q.w;
    reinterpret_cast<float4*>(out)[i] = o;
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
  _Float16* h = reinterpret_cast<_Float16*>(xs);
  hipLaunchKernelGGL(block_sums_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, st, a, nb, h, h + nb);
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
  g.xcd_remap = mtiles % 8 == 0 ? 2 : (tiles % 8 == 0 ? 1 : 0);
  hipLaunchKernelGGL((gemm_q_kernel<DT, BM, BN>), dim3(tiles), dim3(256), 0, st, g);
}

template <class T, int WGM, int WGN, int DA, int TM = 4, int OCC = 1, int FM = 0, bool GLU = false>
static bool gemm_kq_launch(GemmQArgs g, hipStream_t st, bool defer_add) {
  constexpr int BM = 16 * TM * WGM, BN = 64 * WGN;
  int t = 0;
  if (GLU) {
    t = (g.n[0] + BN / 2 - 1) / (BN / 2);  // 32 act columns per wave
    for (int i = 0; i <= 3; ++i) g.tile_start[i] = i == 0 ? 0 : t;
  } else {
    for (int i = 0; i < g.nseg; ++i) {
      g.tile_start[i] = t;
      t += (g.n[i] + BN - 1) / BN;
    }
    for (int i = g.nseg; i <= 3; ++i) g.tile_start[i] = t;
  }
  const int tiles = ((g.M + BM - 1) / BM) * t;
  g.xcd_remap = tiles % 8 == 0 ? 1 : 0;
  // split K in two when one workgroup per tile would leave most CUs idle (the M x N of the O and
  // down projections at a 512-token prompt fill half the chip)
  const size_t mn = (size_t)g.M * g.n[0];
  g.ksplit = (!GLU && g.kpart && g.nseg == 1 && 2 * tiles <= num_cus() && g.K / QK_K >= 2 && mn % 4 == 0) ? 2 : 1;
  hipLaunchKernelGGL((gemm_kq_kernel<T, WGM, WGN, DA, TM, OCC, FM, GLU>), dim3(tiles * g.ksplit), dim3(64 * WGM * WGN),
                     0, st, g);
  if (g.ksplit == 2) {
    if (defer_add) return true;
    launch_add_f32(g.out[0], g.kpart, mn, st);
  }
  return false;
}

// K-quant tile: 64 x 256 (1 x 4 waves; each wave streams its own 64 weight columns, the
// activation tile is shared) with one activation stage in flight: measured 15% faster than
// 128 x 128 at the Mistral-7B prefill shapes, and deeper activation prefetch (two or four stages)
// or eight waves of 32 x 64 gained nothing. Q4_K GEMMs with at least two tiles per CU (gate/up at
// a 512-token prompt: 896 tiles) keep a rescaled accumulator instead of superblock partials, so
// two waves share each SIMD (d applied per 64-wide stage the same way was 3% slower: four times
// the folding); on smaller grids, which then pack two workgroups on some CUs and none on others,
// it is slower (Q/K/V at 512 rows: 74 -> 80 us). Q6_K's fp16 weight pairs do not fit two waves
// per SIMD (the rescaled form spills there and is 30% slower; at one wave per SIMD 7% slower).
template <class T, bool GLU = false>
static bool gemm_kq(GemmQArgs g, hipStream_t st, bool defer_add) {
  size_t nt = 0;
  for (int i = 0; i < g.nseg; ++i) nt += (g.n[i] + 255) / 256;
  const size_t tiles = nt * (size_t)((g.M + 63) / 64);
  if constexpr (T::MINS) {
    if (tiles >= 2 * (size_t)num_cus()) return gemm_kq_launch<T, 1, 4, 1, 4, 2, 2, GLU>(g, st, defer_add);
  }
  return gemm_kq_launch<T, 1, 4, 1, 4, 1, 0, GLU>(g, st, defer_add);
}

// Tile shape 64 x 64 (measured fastest at the Mistral-7B prefill shapes: the larger tiles lose
// more to occupancy than they gain in operand reuse).
template <int DT>
static void gemm_q_dt(GemmQArgs g, hipStream_t st) {
  gemm_q_launch<DT, 64, 64>(g, st);
}

bool launch_gemm_q_glu(int dt, const void* w_gate, const void* w_up, int N, const __half* xh, const __half* xl,
                       const float* xs, int M, int K, __half* act_hi, __half* act_lo, float* act_sums, float* act_f32,
                       int* ovf, hipStream_t st) {
  if (dt != DT_Q4K && dt != DT_Q6K_R) return false;
  if (M < 1 || N < 32 || N % 32 != 0 || !gemm_q_ok(dt, w_gate, K) || !gemm_q_ok(dt, w_up, K)) return false;
  if (dt == DT_Q4K && !xs) fail(ST_OP, "gemm_q: Q4_K needs the per-32 activation sums");
  GemmQArgs g{};
  g.nseg = 2;
  g.w[0] = (const uint8_t*)w_gate;
  g.w[1] = (const uint8_t*)w_up;
  g.n[0] = g.n[1] = N;
  g.M = M;
  g.K = K;
  g.xh = xh;
  g.xl = xl;
  g.xs = xs;
  g.ksplit = 1;
  g.row_bytes = dt == DT_Q4K ? (size_t)(K / QK_K) * Q4K_BYTES : q6r_row_bytes((size_t)(K / QK_K));
  g.glu_h = reinterpret_cast<_Float16*>(act_hi);
  g.glu_l = reinterpret_cast<_Float16*>(act_lo);
  g.glu_sums = reinterpret_cast<_Float16*>(act_sums);
  g.glu_out = act_f32;
  g.ovf = ovf;
  if (dt == DT_Q4K) gemm_kq<Q4KB, true>(g, st, false);
  else gemm_kq<Q6RB, true>(g, st, false);
  return true;
}

void launch_add_f32(float* out, const float* part, size_t n, hipStream_t st) {
  if (n == 0) return;
  if (n % 4 != 0 || (reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(part)) % 16)
    fail(ST_OP, "add_f32: n % 4 and 16-byte aligned arrays");
  const int blocks = (int)std::min<size_t>((n / 4 + 255) / 256, 2048);
  hipLaunchKernelGGL(add_part_kernel, dim3(blocks), dim3(256), 0, st, out, part, n / 4);
}

bool launch_gemm_q(int dt, const GemmQSeg* segs, int nseg, const __half* xh, const __half* xl, const float* xs, int M,
                   int K, const float* resid, hipStream_t st, float* kpart, bool defer_add) {
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
  g.kpart = kpart;
  g.ksplit = 1;
  const size_t nsb = (size_t)(K / QK_K);
  switch (dt) {
    case DT_Q4K: g.row_bytes = nsb * Q4K_BYTES; break;
    case DT_Q6K: g.row_bytes = nsb * Q6K_BYTES; break;
    case DT_Q6K_R: g.row_bytes = q6r_row_bytes(nsb); break;
    default: g.row_bytes = (size_t)(K / 32) * Q8_0_BYTES; break;
  }
  if (dt == DT_Q4K && !xs) fail(ST_OP, "gemm_q: Q4_K needs the per-32 activation sums");
  switch (dt) {
    case DT_Q4K: return gemm_kq<Q4KB>(g, st, defer_add);
    case DT_Q6K: gemm_q_dt<DT_Q6K>(g, st); return false;
    case DT_Q6K_R: return gemm_kq<Q6RB>(g, st, defer_add);
    default: gemm_q_dt<DT_Q8_0>(g, st); return false;
  }
}

}  // namespace iek
