// Attention over a KV cache laid out per layer as [n_kv][ctx][head_dim] (f32 in the sessions; fp16
// through the op-level entry).
//
// Decode (src/layers/attention.rs:462-655): split-K flash-decode over 64-key slices, GQA groups
// sharing one K/V stream; the slice count is fixed by the cache capacity so the launch shape
// never changes between captured decode steps, and the live length is read from device memory.
//
// Prefill (attention.rs:175-422): causal attention over the f32 K/V of the prompt (the
// reference attends to the layer's own k_data/v_data, not the cache).
#include <cstdlib>
#include <type_traits>

#include "attn_core.cuh"

namespace iek {

template <int HD, bool EARLY, int SETS, bool COH, typename T>
__global__ __launch_bounds__(256 * SETS) void attn_decode_kernel(const float* __restrict__ q, const T* __restrict__ kc,
                                                                 const T* __restrict__ vc, float* __restrict__ part,
                                                                 float* __restrict__ out, int* __restrict__ counters,
                                                                 int n_heads, int n_kv, int ctx, const int* pos_dev,
                                                                 int window, float scale, int nsplit, int spc,
                                                                 int HG) {
  __shared__ __align__(16) char smem[AttnSmem<HD, SETS, T>::BYTES];
  // all arguments in one batch of scalar loads, ahead of the position they depend on
  asm volatile("" ::"s"(q), "s"(kc), "s"(vc), "s"(part), "s"(out), "s"(counters), "s"(n_heads), "s"(n_kv), "s"(ctx),
               "s"(pos_dev), "s"(window), "s"(scale), "s"(nsplit), "s"(spc), "s"(HG));
  attn_chunk<HD, COH, EARLY, SETS, T>(q, kc, vc, part, out, counters, n_heads, n_kv, ctx, pos_dev, 0, window, scale,
                                      nsplit, blockIdx.x / HG, blockIdx.y, spc, smem, blockIdx.x % HG, HG);
}

template <int HD, typename T>
static void attn_decode_hd(dim3 grid, hipStream_t st, const float* q, const T* kc, const T* vc, float* out, float* part,
                           int* counters, int n_heads, int n_kv, int ctx, const int* pos_dev, int window, float scale,
                           int nsplit) {
  // chunks of spc slices (about 32 chunks per KV head); one partial slot per chunk
  const int spc = attn_slices_per_chunk(nsplit * SPLIT, window, 32);
  const int nchunk = (nsplit + spc - 1) / spc;
  // Chunks of several slices (long contexts) run two slice streams per workgroup (head dims up to
  // 128: the doubled K / V buffers still fit in LDS), and publish their partials with coherent
  // stores and a relaxed count (no L2 write-back / invalidate around the arrival, measured faster
  // there; one-slice chunks are faster with plain stores).
  const bool two = HD <= 128 && spc >= 2;
  // A group of 8 query heads splits over two workgroups per chunk (four heads each, one per
  // wave) when there are few KV heads to spread over the machine (Gemma-4-E2B: one KV head);
  // each half has its own arrival counter (2 * n_kv counters) and merge.
  const int HG = (n_heads / n_kv == 8 && n_kv < 4) ? 2 : 1;
  auto go = [&](auto kern, int nt) {
    hipLaunchKernelGGL(kern, dim3(grid.x * HG, nchunk), dim3(nt), 0, st, q, kc, vc, part, out, counters, n_heads, n_kv,
                       ctx, pos_dev, window, scale, nchunk, spc, HG);
  };
  // without a window the first slice's loads go out before the position is known
  constexpr int S2 = HD <= 128 ? 2 : 1;
  if (window <= 0)
    two ? go(attn_decode_kernel<HD, true, S2, true, T>, 512) : go(attn_decode_kernel<HD, true, 1, false, T>, 256);
  else
    two ? go(attn_decode_kernel<HD, false, S2, true, T>, 512) : go(attn_decode_kernel<HD, false, 1, false, T>, 256);
}

size_t attn_decode_part_floats(int n_heads, int head_dim, int max_len) {
  // one (max, sum, o[head_dim]) slot per query head and 64-key slice bounds both kernels' partials
  return (size_t)n_heads * ((max_len + SPLIT - 1) / SPLIT) * (head_dim + 2);
}

void launch_attn_decode(const float* q, const void* kc, const void* vc, bool kv_f32, float* out, float* part,
                        int* counters, int n_heads, int n_kv, int head_dim, int ctx, const int* pos_dev, int window,
                        float scale, int max_len, hipStream_t st) {
  const int nsplit = (max_len + SPLIT - 1) / SPLIT;
  dim3 grid(n_kv, nsplit);
  if (n_kv <= 0 || n_heads % n_kv != 0 || n_heads / n_kv > 8)
    fail(ST_OP, "attention: GQA group must divide the heads and be at most 8");
  switch (head_dim) {
#define IEK_AD(HD)                                                                                                 \
  kv_f32 ? attn_decode_hd<HD>(grid, st, q, (const float*)kc, (const float*)vc, out, part, counters, n_heads, n_kv, ctx, \
                              pos_dev, window, scale, nsplit)                                                         \
         : attn_decode_hd<HD>(grid, st, q, (const __half*)kc, (const __half*)vc, out, part, counters, n_heads, n_kv,   \
                              ctx, pos_dev, window, scale, nsplit)
    case 64:
      IEK_AD(64);
      break;
    case 128:
      IEK_AD(128);
      break;
    case 256:
      IEK_AD(256);
      break;
    case 512:
      IEK_AD(512);
      break;
#undef IEK_AD
    default:
      fail(ST_OP, "attention: head_dim must be 64, 128, 256 or 512");
  }
}

// Prefill on the matrix cores (v_mfma_f32_16x16x32_f16): one 256-thread workgroup per (head,
// 64-query tile), each wave owning 16 queries; 64-key blocks of K (row-major) and V (transposed)
// are staged in LDS as fp16 (hi, lo) pairs, S = Q K^T and O += P V each take three MFMAs per step
// (hi*hi + hi*lo + lo*hi, products exact in f32), and the softmax is the online form (running max
// per query row, sum rescaled whenever the max grows).
typedef _Float16 ah8_t __attribute__((ext_vector_type(8)));
typedef float af4_t __attribute__((ext_vector_type(4)));
typedef uint32_t au4_t __attribute__((ext_vector_type(4)));

IEK_DEV uint32_t apack2(_Float16 a, _Float16 b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

IEK_DEV void asplit(float v, _Float16& h, _Float16& l) {
#pragma clang fp contract(off)
  h = (_Float16)v;
  l = (_Float16)(v - (float)h);
}

IEK_DEV af4_t mma3(au4_t ah, au4_t al, au4_t bh, au4_t bl, af4_t c) {
  const ah8_t a_h = __builtin_bit_cast(ah8_t, ah), a_l = __builtin_bit_cast(ah8_t, al);
  const ah8_t b_h = __builtin_bit_cast(ah8_t, bh), b_l = __builtin_bit_cast(ah8_t, bl);
  c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_h, b_h, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_h, b_l, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_l, b_h, c, 0, 0, 0);
  return c;
}

// KB keys per block: 64 up to head_dim 128; 32 at 256 and 512, where the (hi, lo) K block, the
// transposed V block and the P tiles must still fit the 160 KB of LDS.
template <int HD, int KB>
__global__ __launch_bounds__(256) void attn_prefill_mfma_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                                const float* __restrict__ v, float* __restrict__ out,
                                                                int M, int n_heads, int n_kv, int window, float scale) {
  constexpr int JN = KB / 16;    // 16-key column tiles of S
  constexpr int KS = HD / 32;    // MFMA K steps of S = Q K^T
  constexpr int NS = HD / 16;    // 16-wide head-dim subtiles of O
  constexpr int KROW = HD + 8;   // padded LDS rows (halves)
  constexpr int VROW = KB + 8;
  __shared__ __align__(16) _Float16 kh[KB][KROW];
  __shared__ __align__(16) _Float16 kl[KB][KROW];
  __shared__ __align__(16) _Float16 vth[HD][VROW];
  __shared__ __align__(16) _Float16 vtl[HD][VROW];
  __shared__ __align__(16) _Float16 ph[4][16][VROW];
  __shared__ __align__(16) _Float16 pl[4][16][VROW];

  const int h = blockIdx.x, qt = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = n_heads / n_kv, kvh = h / G;
  const int qd = n_heads * HD, kvd = n_kv * HD;
  const int q0 = qt * 64 + 16 * wave;
  const int fr = lane & 15, fk = 8 * (lane >> 4);

  // Q fragments (A operand): row q0 + fr, dims 32 s + fk .. +7, split into fp16 pairs
  au4_t qah[KS], qal[KS];
  {
    const float* qrow = q + (size_t)min(q0 + fr, M - 1) * qd + h * HD;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const float4 a = *reinterpret_cast<const float4*>(qrow + 32 * s + fk);
      const float4 b = *reinterpret_cast<const float4*>(qrow + 32 * s + fk + 4);
      const float vv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      _Float16 hh[8], ll[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) asplit(vv[t], hh[t], ll[t]);
      qah[s] = au4_t{apack2(hh[0], hh[1]), apack2(hh[2], hh[3]), apack2(hh[4], hh[5]), apack2(hh[6], hh[7])};
      qal[s] = au4_t{apack2(ll[0], ll[1]), apack2(ll[2], ll[3]), apack2(ll[4], ll[5]), apack2(ll[6], ll[7])};
    }
  }
  af4_t o[NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) o[j] = af4_t{0.f, 0.f, 0.f, 0.f};
  float mrow[4], lrow[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    mrow[r] = -INFINITY;
    lrow[r] = 0.f;
  }
  const int last_q = min(M - 1, qt * 64 + 63);
  const int jmin_tile = window > 0 ? max(0, qt * 64 - (window - 1)) : 0;
  for (int kb0 = (jmin_tile / KB) * KB; kb0 <= last_q; kb0 += KB) {
    __syncthreads();  // the previous block's LDS reads are done
    for (int e = tid; e < KB * HD / 4; e += 256) {
      const int j = e / (HD / 4), d4 = 4 * (e % (HD / 4));
      const size_t row = (size_t)min(kb0 + j, M - 1) * kvd + kvh * HD + d4;
      const float4 kk = *reinterpret_cast<const float4*>(k + row);
      const float4 vv = *reinterpret_cast<const float4*>(v + row);
      const float kf[4] = {kk.x, kk.y, kk.z, kk.w}, vf[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        asplit(kf[t], kh[j][d4 + t], kl[j][d4 + t]);
        asplit(vf[t], vth[d4 + t][j], vtl[d4 + t][j]);
      }
    }
    __syncthreads();
    if (kb0 > q0 + 15) continue;  // every query of this wave precedes the block
    // S = Q K^T for the wave's 16 queries x KB keys
    af4_t sacc[JN];
#pragma unroll
    for (int jn = 0; jn < JN; ++jn) {
      sacc[jn] = af4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const au4_t bh = *reinterpret_cast<const au4_t*>(&kh[16 * jn + fr][32 * s + fk]);
        const au4_t bl = *reinterpret_cast<const au4_t*>(&kl[16 * jn + fr][32 * s + fk]);
        sacc[jn] = mma3(qah[s], qal[s], bh, bl, sacc[jn]);
      }
    }
    // mask, scale, online softmax; lane holds rows 4 * (lane >> 4) + r, key column 16 jn + fr
    float p[JN][4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = q0 + 4 * (lane >> 4) + r;
      const int jlo = window > 0 ? max(0, i - (window - 1)) : 0;
      float mx = -INFINITY;
#pragma unroll
      for (int jn = 0; jn < JN; ++jn) {
        const int j = kb0 + 16 * jn + fr;
        const bool ok = j <= i && j >= jlo && j < M && i < M;
        const float sv = sacc[jn][r] * scale;
        p[jn][r] = ok ? sv : -INFINITY;
        mx = fmaxf(mx, p[jn][r]);
      }
      mx = row16_max(mx);
      const float mn = fmaxf(mrow[r], mx);
      const float corr = mn == -INFINITY ? 1.f : expf(mrow[r] - mn);
      float sum = 0.f;
#pragma unroll
      for (int jn = 0; jn < JN; ++jn) {
        const float e = p[jn][r] == -INFINITY ? 0.f : expf(p[jn][r] - mn);
        p[jn][r] = e;
        sum += e;
      }
      sum = row16_sum(sum);
      lrow[r] = lrow[r] * corr + sum;
      mrow[r] = mn;
#pragma unroll
      for (int j = 0; j < NS; ++j) o[j][r] *= corr;
    }
    // P to LDS in A-operand order [query][key] (this wave's slice only)
#pragma unroll
    for (int jn = 0; jn < JN; ++jn)
#pragma unroll
      for (int r = 0; r < 4; ++r) asplit(p[jn][r], ph[wave][4 * (lane >> 4) + r][16 * jn + fr], pl[wave][4 * (lane >> 4) + r][16 * jn + fr]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // O += P V
#pragma unroll
    for (int ks = 0; ks < KB / 32; ++ks) {
      const au4_t pah = *reinterpret_cast<const au4_t*>(&ph[wave][fr][32 * ks + fk]);
      const au4_t pal = *reinterpret_cast<const au4_t*>(&pl[wave][fr][32 * ks + fk]);
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const au4_t bh = *reinterpret_cast<const au4_t*>(&vth[16 * j + fr][32 * ks + fk]);
        const au4_t bl = *reinterpret_cast<const au4_t*>(&vtl[16 * j + fr][32 * ks + fk]);
        o[j] = mma3(pah, pal, bh, bl, o[j]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = q0 + 4 * (lane >> 4) + r;
    if (i < M) {
#pragma unroll
      for (int j = 0; j < NS; ++j) out[(size_t)i * qd + h * HD + 16 * j + fr] = o[j][r] / lrow[r];
    }
  }
}

// ---- prefill attention sharing each K/V block across the query heads of a KV head --------------
// K and V (f32 rows [M][n_kv * HD]) are split once per layer into fp16 (hi, lo) planes laid out for
// the MFMA B operands: K per KV head as [n_kv][M][HD], V transposed as [n_kv][HD][Mp] (Mp = M
// rounded up to 64; the padding is zero). One 64 x 64 tile per workgroup, through LDS for V.
__global__ __launch_bounds__(256) void kv_split_kernel(const float* __restrict__ k, const float* __restrict__ v, int M,
                                                       int n_kv, int hd, int Mp, _Float16* __restrict__ kh,
                                                       _Float16* __restrict__ kl, _Float16* __restrict__ vh,
                                                       _Float16* __restrict__ vl) {
  __shared__ float tile[64][65];
  const int h = blockIdx.z, d0 = blockIdx.y * 64, p0 = blockIdx.x * 64, tid = threadIdx.x;
  const size_t kvd = (size_t)n_kv * hd;
#pragma unroll 4
  for (int r = 0; r < 16; ++r) {
    const int pl = (tid >> 6) + 4 * r, dl = tid & 63, p = p0 + pl, d = d0 + dl;
    float vv = 0.f;
    if (p < M && d < hd) {
      const size_t src = (size_t)p * kvd + (size_t)h * hd + d;
      vv = v[src];
      _Float16 a, b;
      asplit(k[src], a, b);
      const size_t kd = ((size_t)h * M + p) * hd + d;
      kh[kd] = a;
      kl[kd] = b;
    }
    tile[pl][dl] = vv;
  }
  __syncthreads();
#pragma unroll 4
  for (int r = 0; r < 16; ++r) {
    const int dl = (tid >> 6) + 4 * r, pl = tid & 63, d = d0 + dl, p = p0 + pl;
    if (d < hd && p < Mp) {
      _Float16 a, b;
      asplit(tile[pl][dl], a, b);
      const size_t vd = ((size_t)h * hd + d) * Mp + p;
      vh[vd] = a;
      vl[vd] = b;
    }
  }
}

// The prompt's attention inputs in one pass (replaces RoPE on Q and on K, the KV append and
// kv_split_kernel): workgroup (position tile, 64-dim tile, z); a thread takes four consecutive head
// dims (two RoPE pairs, the arithmetic of rotate() in ops.hip, src/ops/rope.rs:11-59) of rows
// (tid >> 4) + 16 r. z < n_kv: KV head z, whose K rows get RoPE at the prompt positions 0..M-1 in
// registers, then go to the cache at pos0 + p (f32 or fp16, as kv_store_kernel) and to the K
// planes; V goes to the cache and, through LDS, to the transposed V planes. z >= n_kv: query head
// z - n_kv gets RoPE in place.
IEK_DEV void rope4(float4& x, const float* cs, int p, int npairs, int d) {
#pragma clang fp contract(off)
  const float2* e = reinterpret_cast<const float2*>(cs) + (size_t)p * npairs + (d >> 1);
  if (d < 2 * npairs) {
    const float2 c = e[0];
    const float t0 = x.x, t1 = x.y;
    x.x = t0 * c.x - t1 * c.y;
    x.y = t0 * c.y + t1 * c.x;
  }
  if (d + 2 < 2 * npairs) {
    const float2 c = e[1];
    const float t0 = x.z, t1 = x.w;
    x.z = t0 * c.x - t1 * c.y;
    x.w = t0 * c.y + t1 * c.x;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void attn_prep_kernel(float* __restrict__ q, const float* __restrict__ k,
                                                        const float* __restrict__ v, int M, int n_heads, int n_kv,
                                                        int hd, int Mp, const float* __restrict__ cs, int npairs,
                                                        T* __restrict__ kc, T* __restrict__ vc, int ctx, int pos0,
                                                        _Float16* __restrict__ kh, _Float16* __restrict__ kl,
                                                        _Float16* __restrict__ vh, _Float16* __restrict__ vl,
                                                        int* __restrict__ ovf) {
  __shared__ float tile[64][65];
  const int z = blockIdx.z, d0 = blockIdx.y * 64, p0 = blockIdx.x * 64, tid = threadIdx.x;
  const int c4 = 4 * (tid & 15), d = d0 + c4;  // the thread's four head dims
  auto big4 = [](const float4& x) {
    return fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w))) > F16_PAIR_MAX;
  };
  if (z >= n_kv) {
    const int h = z - n_kv;
    const size_t qd = (size_t)n_heads * hd;
    bool big = false;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int p = p0 + (tid >> 4) + 16 * r;
      if (p < M && d < hd) {
        float4* e = reinterpret_cast<float4*>(q + (size_t)p * qd + (size_t)h * hd + d);
        float4 x = *e;
        rope4(x, cs, p, npairs, d);
        *e = x;
        big |= big4(x);
      }
    }
    if (big) *ovf = 1;
    return;
  }
  bool big = false;
  const int h = z;
  const size_t kvd = (size_t)n_kv * hd;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int pl = (tid >> 4) + 16 * r, p = p0 + pl;
    float4 vv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (p < M && d < hd) {
      const size_t src = (size_t)p * kvd + (size_t)h * hd + d;
      float4 kx = *reinterpret_cast<const float4*>(k + src);
      vv = *reinterpret_cast<const float4*>(v + src);
      rope4(kx, cs, p, npairs, d);
      big |= big4(kx) || big4(vv);
      const size_t dst = ((size_t)h * ctx + pos0 + p) * hd + d;
      if constexpr (std::is_same<T, float>::value) {
        *reinterpret_cast<float4*>(kc + dst) = kx;
        *reinterpret_cast<float4*>(vc + dst) = vv;
      } else {
        kc[dst] = __float2half_rn(kx.x);
        kc[dst + 1] = __float2half_rn(kx.y);
        kc[dst + 2] = __float2half_rn(kx.z);
        kc[dst + 3] = __float2half_rn(kx.w);
        vc[dst] = __float2half_rn(vv.x);
        vc[dst + 1] = __float2half_rn(vv.y);
        vc[dst + 2] = __float2half_rn(vv.z);
        vc[dst + 3] = __float2half_rn(vv.w);
      }
      _Float16 a[4], b[4];
      asplit(kx.x, a[0], b[0]);
      asplit(kx.y, a[1], b[1]);
      asplit(kx.z, a[2], b[2]);
      asplit(kx.w, a[3], b[3]);
      const size_t kd = ((size_t)h * M + p) * hd + d;
      *reinterpret_cast<uint2*>(kh + kd) = make_uint2(apack2(a[0], a[1]), apack2(a[2], a[3]));
      *reinterpret_cast<uint2*>(kl + kd) = make_uint2(apack2(b[0], b[1]), apack2(b[2], b[3]));
    }
    tile[pl][c4] = vv.x;
    tile[pl][c4 + 1] = vv.y;
    tile[pl][c4 + 2] = vv.z;
    tile[pl][c4 + 3] = vv.w;
  }
  if (big) *ovf = 1;
  __syncthreads();
#pragma unroll 4
  for (int r = 0; r < 16; ++r) {
    const int dt = (tid >> 6) + 4 * r, pl = tid & 63, dd = d0 + dt, p = p0 + pl;
    if (dd < hd && p < Mp) {
      _Float16 a, b;
      asplit(tile[pl][dt], a, b);
      const size_t vd = ((size_t)h * hd + dd) * Mp + p;
      vh[vd] = a;
      vl[vd] = b;
    }
  }
}

// One workgroup of NW waves per (KV head, group of up to 4 query heads, query tile): wave w takes
// query head w % G4 and query sub-tile w / G4 (G4 = min(G, 4)), TMQ 16-query MFMA tiles of it. Each
// KB-key block (64; 32 at head_dim 256) of K and V^T is staged once in LDS (16-byte copies of the split planes, the next
// block's loads in flight during the current block's MFMAs) and serves every query head of the
// KV head. The scores are computed transposed, S^T = K Q^T with the keys as MFMA rows: a lane's
// 16 scores of a block then all belong to one query (lane & 15), and with the K rows staged in the
// order krow() gives, the lane's keys of block steps 2t and 2t + 1 are exactly the 8 consecutive
// keys 32t + 8(lane >> 4) .. + 7 that it supplies as the B operand of O^T += V^T P^T. P stays in
// registers (no LDS round trip, no wave barrier), and 72 KB of LDS lets two workgroups share a
// CU (NW = 4) or gives eight waves one staged block (NW = 8). Every product takes three MFMAs (hi*hi + hi*lo + lo*hi of the fp16 pairs, exact in f32);
// the softmax is the online form per query. The longest (latest) query tiles are dispatched first.
template <int HD, int TMQ, int NW, int KB>
__global__ __launch_bounds__(64 * NW, 8 / NW) void attn_prefill_gqa_kernel(const float* __restrict__ q,
                                                                  const _Float16* __restrict__ kh,
                                                                  const _Float16* __restrict__ kl,
                                                                  const _Float16* __restrict__ vh,
                                                                  const _Float16* __restrict__ vl,
                                                                  float* __restrict__ out, int M, int Mp, int n_heads,
                                                                  int n_kv, int window, float scale) {
  static_assert(KB == 32 || KB == 64, "keys per block");
  constexpr int JN = KB / 16;    // 16-key row tiles of S^T
  constexpr int KS = HD / 32;    // MFMA K steps of S^T
  constexpr int NS = HD / 16;    // 16-wide head-dim row tiles of O^T
  constexpr int KROW = HD + 8;   // padded LDS rows (halves)
  constexpr int VROW = KB + 8;
  constexpr int QW = 16 * TMQ;   // queries per wave
  constexpr int NT = 64 * NW;
  constexpr int CPT = KB * HD / 8 / NT;  // 16-byte chunks per thread per plane of a K (or V^T) block
  static_assert(CPT >= 1 && (KB * HD / 8) % NT == 0, "block must divide over the threads");
  __shared__ __align__(16) _Float16 ksh[KB][KROW];
  __shared__ __align__(16) _Float16 ksl[KB][KROW];
  __shared__ __align__(16) _Float16 vsh[HD][VROW];
  __shared__ __align__(16) _Float16 vsl[HD][VROW];

  const int G = n_heads / n_kv, G4 = min(G, 4), HG = (G + 3) / 4;
  const int kvh = blockIdx.x / HG, hg = blockIdx.x % HG;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = wave % G4, qs = wave / G4, h = 4 * hg + hl;
  const bool active = h < G && qs < NW / G4;
  const int QT = QW * (NW / G4);
  const int qt = gridDim.y - 1 - blockIdx.y;  // latest tiles first
  const int wq0 = qt * QT, wq1 = min(M - 1, wq0 + QT - 1);
  const int q0 = wq0 + qs * QW;
  const int hq = kvh * G + min(h, G - 1);
  const int qd = n_heads * HD;
  const int fr = lane & 15, lg = lane >> 4, fk = 8 * lg;

  // Q fragments (B operand of S^T: lane = query fr, dims fk .. fk + 7 of each 32-dim step) of the
  // wave's TMQ query tiles, scaled by scale * log2(e) so that the scores come out in base-2 units
  // (the softmax below is exp2(s - max), the same function), split into fp16 pairs
  const float qscale = scale * 1.44269504088896341f;
  au4_t qah[TMQ][KS], qal[TMQ][KS];
#pragma unroll
  for (int i = 0; i < TMQ; ++i) {
    const float* qrow = q + (size_t)min(q0 + 16 * i + fr, M - 1) * qd + (size_t)hq * HD;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const float4 a = *reinterpret_cast<const float4*>(qrow + 32 * s + fk);
      const float4 b = *reinterpret_cast<const float4*>(qrow + 32 * s + fk + 4);
      const float vv[8] = {a.x * qscale, a.y * qscale, a.z * qscale, a.w * qscale,
                           b.x * qscale, b.y * qscale, b.z * qscale, b.w * qscale};
      _Float16 hh[8], ll[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) asplit(vv[t], hh[t], ll[t]);
      qah[i][s] = au4_t{apack2(hh[0], hh[1]), apack2(hh[2], hh[3]), apack2(hh[4], hh[5]), apack2(hh[6], hh[7])};
      qal[i][s] = au4_t{apack2(ll[0], ll[1]), apack2(ll[2], ll[3]), apack2(ll[4], ll[5]), apack2(ll[6], ll[7])};
    }
  }
  // O^T accumulators (lane: query fr, dims 16j + 4lg .. + 3) and the lane's query's softmax state
  // (running max in base-2 units, running sum)
  af4_t o[TMQ][NS];
  float mrow[TMQ], lrow[TMQ];
#pragma unroll
  for (int i = 0; i < TMQ; ++i) {
#pragma unroll
    for (int j = 0; j < NS; ++j) o[i][j] = af4_t{0.f, 0.f, 0.f, 0.f};
    mrow[i] = -INFINITY;
    lrow[i] = 0.f;
  }

  // staged block: K rows [row][dim] in krow order and V^T rows [dim][key], both planes
  const _Float16* khp = kh + (size_t)kvh * M * HD;
  const _Float16* klp = kl + (size_t)kvh * M * HD;
  const _Float16* vhp = vh + (size_t)kvh * HD * Mp;
  const _Float16* vlp = vl + (size_t)kvh * HD * Mp;
  // LDS row of key j of a block: key 32t + 8g + 4u + e goes to row 16(2t + u) + 4g + e, so that S^T
  // row tile jn = 2t + u holds, in lane group g's four output rows, keys 32t + 8g + 4u .. + 3
  auto krow = [](int j) { return (j & 32) + 16 * ((j >> 2) & 1) + 4 * ((j >> 3) & 3) + (j & 3); };
  au4_t rk[2][CPT], rv[2][CPT];
  auto fetch = [&](int kb0) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int e = tid + NT * c;
      const int j = e / (HD / 8), kc = e % (HD / 8);
      const size_t ks = (size_t)min(kb0 + j, M - 1) * HD + 8 * kc;
      rk[0][c] = *reinterpret_cast<const au4_t*>(khp + ks);
      rk[1][c] = *reinterpret_cast<const au4_t*>(klp + ks);
      const int d = e / (KB / 8), vc = e % (KB / 8);
      const size_t vs = (size_t)d * Mp + kb0 + 8 * vc;
      rv[0][c] = *reinterpret_cast<const au4_t*>(vhp + vs);
      rv[1][c] = *reinterpret_cast<const au4_t*>(vlp + vs);
    }
  };
  const int kb_start = window > 0 ? (max(0, wq0 - (window - 1)) / KB) * KB : 0;
  fetch(kb_start);
  for (int kb0 = kb_start; kb0 <= wq1; kb0 += KB) {
    __syncthreads();  // the previous block's LDS reads are done
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int e = tid + NT * c;
      const int j = e / (HD / 8), kc = e % (HD / 8);
      *reinterpret_cast<au4_t*>(&ksh[krow(j)][8 * kc]) = rk[0][c];
      *reinterpret_cast<au4_t*>(&ksl[krow(j)][8 * kc]) = rk[1][c];
      const int d = e / (KB / 8), vc = e % (KB / 8);
      *reinterpret_cast<au4_t*>(&vsh[d][8 * vc]) = rv[0][c];
      *reinterpret_cast<au4_t*>(&vsl[d][8 * vc]) = rv[1][c];
    }
    __syncthreads();
    if (kb0 + KB <= wq1) fetch(kb0 + KB);
    // the wave's queries all precede the block, or the block is older than all their windows
    if (!active || kb0 > q0 + QW - 1 || (window > 0 && kb0 + KB - 1 < q0 - (window - 1))) continue;
    // query tiles that reach into the block (uniform); each K and V^T fragment is read from LDS
    // once and serves all of them
    bool live[TMQ];
#pragma unroll
    for (int i = 0; i < TMQ; ++i) live[i] = kb0 <= q0 + 16 * i + 15;
    af4_t sacc[TMQ][JN];
#pragma unroll
    for (int i = 0; i < TMQ; ++i)
#pragma unroll
      for (int jn = 0; jn < JN; ++jn) sacc[i][jn] = af4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int jn = 0; jn < JN; ++jn)
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const au4_t ah = *reinterpret_cast<const au4_t*>(&ksh[16 * jn + fr][32 * s + fk]);
        const au4_t al = *reinterpret_cast<const au4_t*>(&ksl[16 * jn + fr][32 * s + fk]);
#pragma unroll
        for (int i = 0; i < TMQ; ++i)
          if (live[i]) sacc[i][jn] = mma3(ah, al, qah[i][s], qal[i][s], sacc[i][jn]);
        // keeps the fragment loads next to their MFMAs (hoisted, they would not fit the registers)
        if (TMQ > 1) __builtin_amdgcn_sched_barrier(0);
      }
    // per query tile: the online softmax of the lane's query, then P^T as the B operands of the two
    // 32-key steps (fp16 pairs); sacc[i][jn][r] is key kb0 + 32(jn >> 1) + 8lg + 4(jn & 1) + r
    au4_t pbh[TMQ][KB / 32], pbl[TMQ][KB / 32];
#pragma unroll
    for (int i = 0; i < TMQ; ++i) {
      if (!live[i]) continue;
      const int qi0 = q0 + 16 * i, qi = qi0 + fr;
      // every key of the block is visible to every query of the tile: no per-score mask
      const bool interior = kb0 + KB - 1 <= qi0 && kb0 + KB <= M && (window <= 0 || kb0 >= qi0 + 16 - window);
      float p[JN][4];
      float mx = -INFINITY;
      if (interior) {
#pragma unroll
        for (int jn = 0; jn < JN; ++jn)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            p[jn][r] = sacc[i][jn][r];
            mx = fmaxf(mx, p[jn][r]);
          }
      } else {
        const int jlo = window > 0 ? max(0, qi - (window - 1)) : 0;
#pragma unroll
        for (int jn = 0; jn < JN; ++jn)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int j = kb0 + 32 * (jn >> 1) + fk + 4 * (jn & 1) + r;
            const bool ok = j <= qi && j >= jlo && j < M && qi < M;
            p[jn][r] = ok ? sacc[i][jn][r] : -INFINITY;
            mx = fmaxf(mx, p[jn][r]);
          }
      }
      // lanes fr, fr + 16, fr + 32, fr + 48 hold the same query
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mn = fmaxf(mrow[i], mx);
      float sum = 0.f;
      if (mn == -INFINITY) {  // no visible key yet
#pragma unroll
        for (int jn = 0; jn < JN; ++jn)
#pragma unroll
          for (int r = 0; r < 4; ++r) p[jn][r] = 0.f;
      } else {
#pragma unroll
        for (int jn = 0; jn < JN; ++jn)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            p[jn][r] = __builtin_amdgcn_exp2f(p[jn][r] - mn);  // exp2(-inf) = 0 for a hidden key
            sum += p[jn][r];
          }
      }
      sum += __shfl_xor(sum, 16);
      sum += __shfl_xor(sum, 32);
      // the running max grows in a few blocks only: rescale when some lane's did
      if (__any(mn != mrow[i])) {
        const float corr = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(mrow[i] - mn);
        lrow[i] *= corr;
#pragma unroll
        for (int j = 0; j < NS; ++j) o[i][j] *= corr;
      }
      lrow[i] += sum;
      mrow[i] = mn;
#pragma unroll
      for (int t = 0; t < KB / 32; ++t) {
        _Float16 ph[8], pl[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) asplit(p[2 * t + (e >> 2)][e & 3], ph[e], pl[e]);
        pbh[i][t] = au4_t{apack2(ph[0], ph[1]), apack2(ph[2], ph[3]), apack2(ph[4], ph[5]), apack2(ph[6], ph[7])};
        pbl[i][t] = au4_t{apack2(pl[0], pl[1]), apack2(pl[2], pl[3]), apack2(pl[4], pl[5]), apack2(pl[6], pl[7])};
      }
    }
    // O^T += V^T P^T over the block's two 32-key steps; the B operand is the lane's own P
#pragma unroll
    for (int t = 0; t < KB / 32; ++t)
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const au4_t ah = *reinterpret_cast<const au4_t*>(&vsh[16 * j + fr][32 * t + fk]);
        const au4_t al = *reinterpret_cast<const au4_t*>(&vsl[16 * j + fr][32 * t + fk]);
#pragma unroll
        for (int i = 0; i < TMQ; ++i)
          if (live[i]) o[i][j] = mma3(ah, al, pbh[i][t], pbl[i][t], o[i][j]);
        if (TMQ > 1) __builtin_amdgcn_sched_barrier(0);
      }
  }
  if (!active) return;
#pragma unroll
  for (int i = 0; i < TMQ; ++i) {
    const int qi = q0 + 16 * i + fr;
    if (qi < M) {
      const float l = lrow[i];
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const af4_t v = o[i][j];
        *reinterpret_cast<float4*>(out + (size_t)qi * qd + (size_t)hq * HD + 16 * j + 4 * lg) =
            make_float4(v[0] / l, v[1] / l, v[2] / l, v[3] / l);
      }
    }
  }
}

// Prefill attention on f32 inputs (taken when a q, k or v value is beyond the fp16 pair's range):
// the reference's per-(position, head) loop (src/layers/attention.rs:364-415) with an online
// softmax. One wave per (query row i, head h): keys j in [j_min, i] (j_min = i - (window - 1)
// with a window) in chunks of 64, lane = key for the scores (dot * scale in f32), lane = head
// dims for P V. q and k carry RoPE; k and v rows are [M][n_kv * hd], KV head h / (n_heads / n_kv).
__global__ __launch_bounds__(64) void attn_prefill_f32_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                              const float* __restrict__ v, float* __restrict__ out,
                                                              int M, int n_heads, int n_kv, int hd, int window,
                                                              float scale) {
#pragma clang fp contract(off)
  constexpr int DPL = 8;  // head dims per lane (hd <= 512)
  __shared__ float qs[512];
  __shared__ float ps[64];
  const int i = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int kvh = h / (n_heads / n_kv);
  const size_t qd = (size_t)n_heads * hd, kvd = (size_t)n_kv * hd;
  for (int d = lane; d < hd; d += 64) qs[d] = q[(size_t)i * qd + (size_t)h * hd + d];
  __syncthreads();
  const int j0 = window > 0 ? max(0, i - (window - 1)) : 0;
  float m = -INFINITY, l = 0.f, o[DPL];
#pragma unroll
  for (int t = 0; t < DPL; ++t) o[t] = 0.f;
  for (int jb = j0; jb <= i; jb += 64) {
    const int j = jb + lane;
    float sc = -INFINITY;
    if (j <= i) {
      const float* kr = k + (size_t)j * kvd + (size_t)kvh * hd;
      float dot = 0.f;
      for (int d = 0; d < hd; ++d) dot += qs[d] * kr[d];
      sc = dot * scale;
    }
    const float cm = wave_max(sc);
    const float mn = fmaxf(m, cm);
    const float p = j <= i ? expf(sc - mn) : 0.f;
    const float corr = expf(m - mn);  // 0 on the first chunk (m = -inf)
    l = l * corr + wave_sum(p);
#pragma unroll
    for (int t = 0; t < DPL; ++t) o[t] *= corr;
    m = mn;
    ps[lane] = p;
    __syncthreads();
    const int nj = min(64, i + 1 - jb);
    for (int jj = 0; jj < nj; ++jj) {
      const float pj = ps[jj];
      const float* vr = v + (size_t)(jb + jj) * kvd + (size_t)kvh * hd;
#pragma unroll
      for (int t = 0; t < DPL; ++t) {
        const int d = lane + 64 * t;
        if (d < hd) o[t] += pj * vr[d];
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int t = 0; t < DPL; ++t) {
    const int d = lane + 64 * t;
    if (d < hd) out[(size_t)i * qd + (size_t)h * hd + d] = o[t] / l;
  }
}

void launch_attn_prefill_f32(const float* q, const float* k, const float* v, float* out, int M, int n_heads, int n_kv,
                             int head_dim, int window, float scale, hipStream_t st) {
  if (M <= 0) return;
  if (head_dim <= 0 || head_dim > 512 || n_kv <= 0 || n_heads % n_kv != 0)
    fail(ST_OP, "prefill attention (f32): head_dim <= 512 and whole GQA groups");
  hipLaunchKernelGGL(attn_prefill_f32_kernel, dim3(M, n_heads), dim3(64), 0, st, q, k, v, out, M, n_heads, n_kv,
                     head_dim, window, scale);
}

// Scratch halves the shared-K/V path needs: four planes of n_kv * HD * Mp.
size_t attn_prefill_scratch_halves(int M, int n_kv, int head_dim) {
  const size_t Mp = (size_t)((M + 63) / 64) * 64;
  return 4 * (size_t)n_kv * head_dim * Mp;
}

// The split K / V^T planes and attn_prefill_gqa_kernel: head_dim 64, 128 and (through
// kv_split_kernel only) 256.
static bool attn_planes_ok(int M, int n_heads, int n_kv, int head_dim, const void* scratch, size_t scratch_halves) {
  return scratch && M >= 1 && n_kv >= 1 && (head_dim == 64 || head_dim == 128 || head_dim == 256) &&
         n_heads % n_kv == 0 && scratch_halves >= attn_prefill_scratch_halves(M, n_kv, head_dim);
}

bool launch_attn_prefill_prep(float* q, const float* k, const float* v, int M, int n_heads, int n_kv, int head_dim,
                              const float* cs, int npairs, void* kc, void* vc, bool kv_f32, int ctx, int pos0,
                              void* scratch, size_t scratch_halves, int* ovf, hipStream_t st) {
  if (!attn_planes_ok(M, n_heads, n_kv, head_dim, scratch, scratch_halves) || head_dim > 128 || npairs < 0 ||
      2 * npairs > head_dim || !ovf)
    return false;
  if (pos0 < 0 || (size_t)pos0 + (size_t)M > (size_t)ctx) fail(ST_KVCACHE, "attention prep: the prompt does not fit the cache");
  const int Mp = ((M + 63) / 64) * 64;
  const size_t plane = (size_t)n_kv * head_dim * Mp;
  _Float16* s16 = static_cast<_Float16*>(scratch);
  _Float16 *kh = s16, *kl = s16 + plane, *vh = s16 + 2 * plane, *vl = s16 + 3 * plane;
  const dim3 grid(Mp / 64, (head_dim + 63) / 64, n_kv + n_heads);
  if (kv_f32)
    hipLaunchKernelGGL(attn_prep_kernel<float>, grid, dim3(256), 0, st, q, k, v, M, n_heads, n_kv, head_dim, Mp, cs,
                       npairs, (float*)kc, (float*)vc, ctx, pos0, kh, kl, vh, vl, ovf);
  else
    hipLaunchKernelGGL(attn_prep_kernel<__half>, grid, dim3(256), 0, st, q, k, v, M, n_heads, n_kv, head_dim, Mp, cs,
                       npairs, (__half*)kc, (__half*)vc, ctx, pos0, kh, kl, vh, vl, ovf);
  return true;
}

void launch_attn_prefill(const float* q, const float* k, const float* v, float* out, int M, int n_heads, int n_kv,
                         int head_dim, int window, float scale, hipStream_t st, void* scratch, size_t scratch_halves,
                         bool planes_ready, int* ovf) {
  const int G = n_heads / n_kv;
  if (!planes_ready && ovf) {
    // the kernels below split q, k and v into fp16 pairs themselves (or through kv_split_kernel)
    launch_range_flag(q, (size_t)M * n_heads * head_dim, ovf, st);
    launch_range_flag(k, (size_t)M * n_kv * head_dim, ovf, st);
    launch_range_flag(v, (size_t)M * n_kv * head_dim, ovf, st);
  }
  if (attn_planes_ok(M, n_heads, n_kv, head_dim, scratch, scratch_halves) && G >= 1) {
    const int Mp = ((M + 63) / 64) * 64;
    const size_t plane = (size_t)n_kv * head_dim * Mp;
    _Float16* s16 = static_cast<_Float16*>(scratch);
    _Float16 *kh = s16, *kl = s16 + plane, *vh = s16 + 2 * plane, *vl = s16 + 3 * plane;
    if (!planes_ready)
      hipLaunchKernelGGL(kv_split_kernel, dim3(Mp / 64, (head_dim + 63) / 64, n_kv), dim3(256), 0, st, k, v, M, n_kv,
                         head_dim, Mp, kh, kl, vh, vl);
    const int G4 = std::min(G, 4), HG = (G + 3) / 4;
    // eight waves of two query tiles each per staged block once the grid fills the machine twice
    // over, four waves of one tile below that
    const int qt8 = 32 * (8 / G4);
    const bool wide = (size_t)n_kv * HG * ((M + qt8 - 1) / qt8) >= 2 * (size_t)num_cus();
    const int QT = wide ? qt8 : 16 * (4 / G4);
    const dim3 grid(n_kv * HG, (M + QT - 1) / QT);
    if (head_dim == 256) {
      // 32-key blocks (the K and V^T planes of a block take 75 KB), four waves of one tile
      const int qt4 = 16 * (4 / G4);
      hipLaunchKernelGGL((attn_prefill_gqa_kernel<256, 1, 4, 32>), dim3(n_kv * HG, (M + qt4 - 1) / qt4), dim3(256), 0,
                         st, q, kh, kl, vh, vl, out, M, Mp, n_heads, n_kv, window, scale);
    } else if (head_dim == 128) {
      if (wide)
        hipLaunchKernelGGL((attn_prefill_gqa_kernel<128, 2, 8, 64>), grid, dim3(512), 0, st, q, kh, kl, vh, vl, out, M,
                           Mp, n_heads, n_kv, window, scale);
      else
        hipLaunchKernelGGL((attn_prefill_gqa_kernel<128, 1, 4, 64>), grid, dim3(256), 0, st, q, kh, kl, vh, vl, out, M,
                           Mp, n_heads, n_kv, window, scale);
    } else {
      if (wide)
        hipLaunchKernelGGL((attn_prefill_gqa_kernel<64, 2, 8, 64>), grid, dim3(512), 0, st, q, kh, kl, vh, vl, out, M,
                           Mp, n_heads, n_kv, window, scale);
      else
        hipLaunchKernelGGL((attn_prefill_gqa_kernel<64, 1, 4, 64>), grid, dim3(256), 0, st, q, kh, kl, vh, vl, out, M,
                           Mp, n_heads, n_kv, window, scale);
    }
    return;
  }
  dim3 grid(n_heads, (M + 63) / 64);
  switch (head_dim) {
#define IEK_AP(HD, KB)                                                                                          \
  hipLaunchKernelGGL((attn_prefill_mfma_kernel<HD, KB>), grid, dim3(256), 0, st, q, k, v, out, M, n_heads, n_kv, \
                     window, scale)
    case 64:
      IEK_AP(64, 64);
      break;
    case 128:
      IEK_AP(128, 64);
      break;
    case 256:
      IEK_AP(256, 32);
      break;
    case 512:
      IEK_AP(512, 32);
      break;
#undef IEK_AP
    default:
      fail(ST_OP, "prefill attention: head_dim must be 64, 128, 256 or 512");
  }
}

}  // namespace iek
