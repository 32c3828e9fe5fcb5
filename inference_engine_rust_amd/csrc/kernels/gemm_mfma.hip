// Prefill matmul on the CDNA4 matrix cores: out[m, n] = sum_k a[m, k] * W(k, n) for K-quant, Q8_0
// and F32 weights, using v_mfma_f32_16x16x32_f16.
//
// Precision. The reference multiplies f32 activations by f32 dequantised weights
// (src/ops/matmul.rs, src/ops/quant/quant_k_handler.rs). Both operands are split here into an fp16
// pair, v = hi + lo with hi = fp16(v) and lo = fp16(v - hi), which carries 22 significant bits,
// and three MFMAs per K step accumulate hi*hi + hi*lo + lo*hi in f32 (the dropped lo*lo term is
// ~2^-22 relative). Products of fp16 values are exact in f32, so the result differs from the
// reference only by f32 accumulation order plus ~2^-21 relative representation error, well inside
// the fp32 reordering bound the parity tests apply.
//
// Tiling. A 256-thread workgroup owns a BM x 64 output tile (BM = 128 or 256, four waves stacked
// along M, each 16-row subtiles x four 16-column subtiles). Each 32-wide K stage stages the
// activation pair (pre-split in HBM) and the weight rows, dequantised exactly as the reference
// does and split into fp16 pairs, in LDS; the next stage's raw bytes are in flight in registers
// while the current stage's MFMAs run. Workgroups are mapped so that all M tiles of one weight
// N tile land on the same XCD and share its L2.
#include <type_traits>

#include "common.cuh"
#include "../iek_internal.h"

namespace iek {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));  // native vector: stays in registers

constexpr int MBK = 32;       // K per stage (one MFMA step)
constexpr int MBN = 64;       // N per workgroup
constexpr int LDS_ROW = 40;   // halves per LDS row: 32 + 8 padding (80 B rows spread the banks)

// ---- fp16 pair split --------------------------------------------------------------------------
IEK_DEV uint32_t pack2(_Float16 a, _Float16 b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

IEK_DEV void split8(const float (&v)[8], uint4& hi, uint4& lo) {
#pragma clang fp contract(off)
  _Float16 h[8], l[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    h[i] = (_Float16)v[i];
    l[i] = (_Float16)(v[i] - (float)h[i]);
  }
  hi = make_uint4(pack2(h[0], h[1]), pack2(h[2], h[3]), pack2(h[4], h[5]), pack2(h[6], h[7]));
  lo = make_uint4(pack2(l[0], l[1]), pack2(l[2], l[3]), pack2(l[4], l[5]), pack2(l[6], l[7]));
}

__global__ __launch_bounds__(256) void split_f16_kernel(const float* __restrict__ x, size_t n8, uint4* __restrict__ hi,
                                                        uint4* __restrict__ lo) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (size_t)gridDim.x * 256) {
    const float4 a = reinterpret_cast<const float4*>(x)[2 * i], b = reinterpret_cast<const float4*>(x)[2 * i + 1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint4 h, l;
    split8(v, h, l);
    hi[i] = h;
    lo[i] = l;
  }
}

void launch_split_f16(const float* x, size_t n, __half* hi, __half* lo, hipStream_t st) {
  if (n % 8 != 0) fail(ST_OP, "split_f16: length must be a multiple of 8");
  const size_t n8 = n / 8;
  const int blocks = (int)std::min<size_t>((n8 + 255) / 256, 4096);
  hipLaunchKernelGGL(split_f16_kernel, dim3(std::max(blocks, 1)), dim3(256), 0, st, x, n8, (uint4*)hi, (uint4*)lo);
}

// ---- exact dequantisation of 8 consecutive flat elements f0 .. f0+7 (f0 % 8 == 0) ----------
// Raw bytes are fetched first (raw_load) and decoded after the current stage's MFMAs (decode), so
// the fetch latency hides behind the matrix work.
template <int DT>
struct Deq;

template <>
struct Deq<DT_Q4K> {
  uint4 hdr;
  uint2 qs;
  IEK_DEV void raw_load(const uint8_t* w, size_t f0) {
    const uint8_t* blk = w + (f0 / QK_K) * Q4K_BYTES;
    const int e = (int)(f0 % QK_K), g = e >> 6, l0 = e & 31;
    hdr = *reinterpret_cast<const uint4*>(blk);
    qs = *reinterpret_cast<const uint2*>(blk + 16 + 32 * g + l0);
  }
  IEK_DEV void decode(size_t f0, float (&o)[8]) const {
    const int e = (int)(f0 % QK_K), g = e >> 6, hi = (e >> 5) & 1;
    const float d = half_bits_to_float(hdr.x), dmin = half_bits_to_float(hdr.x >> 16);
    float sc, m;
    scale_min_k4(2 * g + hi, hdr.y, hdr.z, hdr.w, &sc, &m);
    const uint32_t w2[2] = {qs.x, qs.y};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t q = (w2[i >> 2] >> (8 * (i & 3) + 4 * hi)) & 0xFu;
      o[i] = q4k_value(d, dmin, sc, m, q);
    }
  }
};

template <>
struct Deq<DT_Q6K> {
  uint32_t ql[4], qh[4], sd;  // u16 pairs of ql / qh bytes; sd = scale byte | d << 16
  IEK_DEV void raw_load(const uint8_t* w, size_t f0) {
    const uint8_t* blk = w + (f0 / QK_K) * Q6K_BYTES;
    const int e = (int)(f0 % QK_K), h = e >> 7, r = e & 127, quarter = r >> 5, l0 = r & 31;
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
  IEK_DEV void decode(size_t f0, float (&o)[8]) const {
#pragma clang fp contract(off)
    const int e = (int)(f0 % QK_K), quarter = (e & 127) >> 5;
    const float d = half_bits_to_float(sd >> 16);
    const float ds = d * (float)(int8_t)(sd & 0xFF);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t lb = (ql[i >> 1] >> (8 * (i & 1))) & 0xFFu, hb = (qh[i >> 1] >> (8 * (i & 1))) & 0xFFu;
      const uint32_t nib = quarter < 2 ? (lb & 0xFu) : (lb >> 4);
      const int q = (int)(nib | (((hb >> (2 * quarter)) & 3u) << 4)) - 32;
      o[i] = q == 0 ? 0.0f : ds * (float)q;
    }
  }
};

template <>
struct Deq<DT_Q8_0> {
  uint32_t q[4], d;
  IEK_DEV void raw_load(const uint8_t* w, size_t f0) {
    const uint8_t* blk = w + (f0 / Q8_0_ELEMS) * Q8_0_BYTES;
    const uint16_t* p = reinterpret_cast<const uint16_t*>(blk + 2 + (f0 % Q8_0_ELEMS));
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = p[i];
    d = *reinterpret_cast<const uint16_t*>(blk);
  }
  IEK_DEV void decode(size_t, float (&o)[8]) const {
#pragma clang fp contract(off)
    const float df = half_bits_to_float(d);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = df * (float)(int8_t)((q[i >> 1] >> (8 * (i & 1))) & 0xFFu);
  }
};

template <>
struct Deq<DT_F32> {
  float4 a, b;
  IEK_DEV void raw_load(const uint8_t* w, size_t f0) {
    const float4* p = reinterpret_cast<const float4*>(w + f0 * 4);
    a = p[0];
    b = p[1];
  }
  IEK_DEV void decode(size_t, float (&o)[8]) const {
    o[0] = a.x, o[1] = a.y, o[2] = a.z, o[3] = a.w, o[4] = b.x, o[5] = b.y, o[6] = b.z, o[7] = b.w;
  }
};

// ---- stage helpers ----------------------------------------------------------------------------
// activation pair rows m0 .. m0+BM-1 (clamped to M-1), K columns k0 .. k0+31: AU uint4 per plane
template <int AU>
IEK_DEV void fetch_a(const __half* xh, const __half* xl, int m0, int M, int K, int k0, int tid, u4_t (&arh)[AU],
                     u4_t (&arl)[AU]) {
#pragma unroll
  for (int u = 0; u < AU; ++u) {
    const int idx = tid + 256 * u, row = idx >> 2, c8 = idx & 3;
    const size_t off = (size_t)min(m0 + row, M - 1) * K + k0 + 8 * c8;
    arh[u] = *reinterpret_cast<const u4_t*>(xh + off);
    arl[u] = *reinterpret_cast<const u4_t*>(xl + off);
  }
}

template <int BM, int AU>
IEK_DEV void stage_a(_Float16 (*as_h)[LDS_ROW], _Float16 (*as_l)[LDS_ROW], int tid, const u4_t (&arh)[AU],
                     const u4_t (&arl)[AU]) {
#pragma unroll
  for (int u = 0; u < AU; ++u) {
    const int idx = tid + 256 * u, row = idx >> 2, c8 = idx & 3;
    *reinterpret_cast<u4_t*>(&as_h[row][8 * c8]) = arh[u];
    *reinterpret_cast<u4_t*>(&as_l[row][8 * c8]) = arl[u];
  }
}

template <int DT>
IEK_DEV void stage_b(_Float16 (*bs_h)[LDS_ROW], _Float16 (*bs_l)[LDS_ROW], int row, int run, const Deq<DT>& braw,
                     size_t f0) {
  float v[8];
  braw.decode(f0, v);
  uint4 hi, lo;
  split8(v, hi, lo);
  *reinterpret_cast<uint4*>(&bs_h[row][8 * run]) = hi;
  *reinterpret_cast<uint4*>(&bs_l[row][8 * run]) = lo;
}

// ---- the GEMM -------------------------------------------------------------------------------
template <int DT, int BM>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(const uint8_t* __restrict__ w, const __half* __restrict__ xh,
                                                        const __half* __restrict__ xl, int M, int K, int N,
                                                        float* __restrict__ out, const float* __restrict__ resid,
                                                        int xcd_remap) {
  constexpr int WM = BM / 4;        // rows per wave
  constexpr int MT = WM / 16;       // 16-row subtiles per wave
  constexpr int NT = MBN / 16;      // 16-column subtiles
  constexpr int AU = BM * 4 / 256;  // uint4 per thread per plane per stage
  __shared__ __align__(16) _Float16 as_h[BM][LDS_ROW];
  __shared__ __align__(16) _Float16 as_l[BM][LDS_ROW];
  __shared__ __align__(16) _Float16 bs_h[MBN][LDS_ROW];
  __shared__ __align__(16) _Float16 bs_l[MBN][LDS_ROW];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int mtiles = (M + BM - 1) / BM;
  int tile = blockIdx.x;
  if (xcd_remap) {
    // hardware hands workgroup b to XCD b % 8; give each XCD a contiguous range of tiles (N-major,
    // M-minor) so the M tiles sharing one weight tile sit behind the same L2
    const int per = gridDim.x / 8;
    tile = (blockIdx.x % 8) * per + blockIdx.x / 8;
  }
  const int mt = tile % mtiles, nt = tile / mtiles;
  const int m0 = mt * BM, n0 = nt * MBN;
  const int nk = K / MBK;

  // per-thread staging assignments
  const int b_row = tid >> 2, b_run = tid & 3;  // weight row within the tile, 8-element run
  const size_t b_f = (size_t)min(n0 + b_row, N - 1) * K + 8 * b_run;
  u4_t arh[AU], arl[AU];
  Deq<DT> braw;
  f4_t acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  fetch_a<AU>(xh, xl, m0, M, K, 0, tid, arh, arl);
  braw.raw_load(w, b_f);
  stage_a<BM, AU>(as_h, as_l, tid, arh, arl);
  stage_b<DT>(bs_h, bs_l, b_row, b_run, braw, b_f);
  __syncthreads();
  const int fr = lane & 15, fk = 8 * (lane >> 4);
  for (int kt = 0; kt < nk; ++kt) {
    {
      const int k1 = min(kt + 1, nk - 1) * MBK;
      fetch_a<AU>(xh, xl, m0, M, K, k1, tid, arh, arl);
      braw.raw_load(w, b_f + k1);
    }
    u4_t ah[MT], al[MT], bh[NT], bl[NT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      ah[i] = *reinterpret_cast<const u4_t*>(&as_h[wave * WM + 16 * i + fr][fk]);
      al[i] = *reinterpret_cast<const u4_t*>(&as_l[wave * WM + 16 * i + fr][fk]);
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      bh[j] = *reinterpret_cast<const u4_t*>(&bs_h[16 * j + fr][fk]);
      bl[j] = *reinterpret_cast<const u4_t*>(&bs_l[16 * j + fr][fk]);
    }
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const h8_t a_h = __builtin_bit_cast(h8_t, ah[i]), a_l = __builtin_bit_cast(h8_t, al[i]);
        const h8_t b_h = __builtin_bit_cast(h8_t, bh[j]), b_l = __builtin_bit_cast(h8_t, bl[j]);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_h, b_h, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_h, b_l, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_l, b_h, acc[i][j], 0, 0, 0);
      }
    __syncthreads();
    if (kt + 1 < nk) {
      stage_a<BM, AU>(as_h, as_l, tid, arh, arl);
      stage_b<DT>(bs_h, bs_l, b_row, b_run, braw, b_f + (size_t)(kt + 1) * MBK);
    }
    __syncthreads();
  }

  // D layout of the 16x16 MFMA: lane holds column lane % 16, rows 4 * (lane / 16) + r
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int n = n0 + 16 * j + (lane & 15);
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

bool gemm_mfma_ok(int dt, const void* w, int K, int N) {
  if (K % MBK != 0 || N < 1) return false;
  switch (dt) {
    case DT_Q4K:
    case DT_F32:
      return (reinterpret_cast<uintptr_t>(w) & 15) == 0;
    case DT_Q6K:
    case DT_Q8_0:
      return (reinterpret_cast<uintptr_t>(w) & 1) == 0;
    default:
      return false;
  }
}

template <int DT>
static void gemm_mfma_dt(const void* w, const __half* xh, const __half* xl, int M, int K, int N, float* out,
                         const float* resid, hipStream_t st) {
  const int ntiles = (N + MBN - 1) / MBN;
  // BM = 256 when that still gives at least one workgroup per CU, else 128 (more workgroups)
  const bool big = (size_t)((M + 255) / 256) * ntiles >= 256;
  const int BM = big ? 256 : 128;
  const int tiles = ((M + BM - 1) / BM) * ntiles;
  const int remap = tiles % 8 == 0 ? 1 : 0;
  if (big)
    hipLaunchKernelGGL((gemm_mfma_kernel<DT, 256>), dim3(tiles), dim3(256), 0, st, (const uint8_t*)w, xh, xl, M, K, N,
                       out, resid, remap);
  else
    hipLaunchKernelGGL((gemm_mfma_kernel<DT, 128>), dim3(tiles), dim3(256), 0, st, (const uint8_t*)w, xh, xl, M, K, N,
                       out, resid, remap);
}

void launch_gemm_mfma(int dt, const void* w, const __half* xh, const __half* xl, int M, int K, int N, float* out,
                      const float* resid, hipStream_t st) {
  if (!gemm_mfma_ok(dt, w, K, N) || M < 1) fail(ST_OP, "gemm_mfma: unsupported weight type, alignment or shape");
  switch (dt) {
    case DT_Q4K: gemm_mfma_dt<DT_Q4K>(w, xh, xl, M, K, N, out, resid, st); break;
    case DT_Q6K: gemm_mfma_dt<DT_Q6K>(w, xh, xl, M, K, N, out, resid, st); break;
    case DT_Q8_0: gemm_mfma_dt<DT_Q8_0>(w, xh, xl, M, K, N, out, resid, st); break;
    default: gemm_mfma_dt<DT_F32>(w, xh, xl, M, K, N, out, resid, st); break;
  }
}

}  // namespace iek
