// Attention over an fp16 KV cache laid out per layer as [n_kv][ctx][head_dim].
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

template <int HD>
__global__ __launch_bounds__(256) void attn_decode_kernel(const float* __restrict__ q, const __half* __restrict__ kc,
                                                          const __half* __restrict__ vc, float* __restrict__ part,
                                                          float* __restrict__ out, int* __restrict__ counters,
                                                          int n_heads, int n_kv, int ctx, const int* pos_dev,
                                                          int window, float scale, int nsplit, int spc) {
  __shared__ __align__(16) char smem[AttnSmem<HD>::BYTES];
  // all arguments in one batch of scalar loads, ahead of the position they depend on
  asm volatile("" ::"s"(q), "s"(kc), "s"(vc), "s"(part), "s"(out), "s"(counters), "s"(n_heads), "s"(n_kv), "s"(ctx),
               "s"(pos_dev), "s"(window), "s"(scale), "s"(nsplit), "s"(spc));
  attn_chunk_f16<HD>(q, kc, vc, part, out, counters, n_heads, n_kv, ctx, *pos_dev + 1, window, scale, nsplit,
                     blockIdx.x, blockIdx.y, spc, smem);
}

// f32 KV cache variant (Gemma-4 sessions keep the reference's f32 cache: with q/k head norms
// and a score scale of 1 the softmax is sharp enough that fp16 keys/values move the logits by
// ~1e-2). Same grid, partials and merge as the fp16 kernel. The slice's K rows, then its V rows,
// are staged through one LDS buffer in pieces of up to 256 head dims with cooperative 16-byte
// loads (every load of a piece in flight at once); lane = key for the scores (two query heads
// per wave), then for P.V each lane owns DPP consecutive dims of the piece.
template <int HD>
__global__ __launch_bounds__(256) void attn_decode_f32_kernel(const float* __restrict__ q, const float* __restrict__ kc,
                                                              const float* __restrict__ vc, float* __restrict__ part,
                                                              float* __restrict__ out, int* __restrict__ counters,
                                                              int n_heads, int n_kv, int ctx, const int* pos_dev,
                                                              int window, float scale, int nsplit) {
  constexpr int PD = HD < 256 ? HD : 256;  // dims per staged piece
  constexpr int NP = HD / PD;
  // all arguments in one batch of scalar loads, ahead of the position they depend on
  asm volatile("" ::"s"(q), "s"(kc), "s"(vc), "s"(part), "s"(out), "s"(counters), "s"(n_heads), "s"(n_kv), "s"(ctx),
               "s"(pos_dev), "s"(window), "s"(scale), "s"(nsplit));
  constexpr int ROW = PD + 4;               // padded LDS row (floats)
  constexpr int DPP = PD / 64;              // dims per lane per piece in P.V
  constexpr int F4 = SPLIT * PD / 4 / 256;  // float4 per thread per piece
  const int G = n_heads / n_kv;
  // query heads split over HG workgroups per (KV head, slice) when the group has 8: each
  // workgroup stages the slice and runs one head per wave
  const int HG = G == 8 ? 2 : 1, GH = G / HG;
  const int kvh = blockIdx.x / HG, hg = blockIdx.x % HG, gb = hg * GH;
  const int sp = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int total = *pos_dev + 1;
  const int jmin = (window > 0 && total > window) ? total - window : 0;
  const int j0 = max(sp * SPLIT, jmin), j1 = min(total, (sp + 1) * SPLIT);
  const int nk = j1 - j0;
  if (nk <= 0) return;  // uniform across the workgroup
  __shared__ __align__(16) float qs[8][HD];
  __shared__ __align__(16) float kv[SPLIT][ROW];
  __shared__ float ps[8][SPLIT];
  const float* kb = kc + ((size_t)kvh * ctx + j0) * HD;
  const float* vb = vc + ((size_t)kvh * ctx + j0) * HD;
  // cooperative piece load: element e of the piece is row e / (PD/4), float4 column e % (PD/4)
  typedef float pf4_t __attribute__((ext_vector_type(4)));  // native vectors stay in registers
  auto stage_piece = [&](const float* base, int p) {
    pf4_t r[F4];
#pragma unroll
    for (int u = 0; u < F4; ++u) {
      const int e = tid + 256 * u, row = min(e / (PD / 4), nk - 1), c4 = e % (PD / 4);
      r[u] = *reinterpret_cast<const pf4_t*>(base + (size_t)row * HD + p * PD + 4 * c4);
    }
    __syncthreads();  // the previous piece's readers are done
#pragma unroll
    for (int u = 0; u < F4; ++u) {
      const int e = tid + 256 * u, row = e / (PD / 4), c4 = e % (PD / 4);
      *reinterpret_cast<pf4_t*>(&kv[row][4 * c4]) = r[u];
    }
    __syncthreads();
  };
  for (int i = tid; i < GH * HD; i += 256) qs[i / HD][i % HD] = q[(size_t)(kvh * G + gb) * HD + i];
  float sc[2] = {0.f, 0.f};
  for (int p = 0; p < NP; ++p) {
    stage_piece(kb, p);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int g = wave + 4 * t;
      if (g < GH) {
        float acc = 0.f;
#pragma unroll 8
        for (int d = 0; d < PD; d += 4) {
          const float4 k4 = *reinterpret_cast<const float4*>(&kv[lane][d]);
          const float4 q4 = *reinterpret_cast<const float4*>(&qs[g][p * PD + d]);
          acc += q4.x * k4.x + q4.y * k4.y + q4.z * k4.z + q4.w * k4.w;
        }
        sc[t] += acc;
      }
    }
  }
  const bool valid = lane < nk;
  float m[2], l[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int g = wave + 4 * t;
    if (g < GH) {
      const float s = valid ? sc[t] * scale : -INFINITY;
      m[t] = wave_max(s);
      const float pr = valid ? expf(s - m[t]) : 0.f;
      l[t] = wave_sum(pr);
      ps[g][lane] = pr;
    }
  }
  float o[2][NP][DPP];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int e = 0; e < DPP; ++e) o[t][p][e] = 0.f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    stage_piece(vb, p);  // its first barrier also publishes ps
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int g = wave + 4 * t;
      if (g < GH) {
#pragma unroll 8
        for (int j = 0; j < SPLIT; ++j) {
          const float pj = ps[g][j];
#pragma unroll
          for (int e = 0; e < DPP; ++e) o[t][p][e] += pj * kv[j][DPP * lane + e];
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int g = wave + 4 * t;
    if (g < GH) {
      float* pr = part + ((size_t)(kvh * G + gb + g) * nsplit + sp) * (HD + 2);
      if (lane == 0) {
        pr[0] = m[t];
        pr[1] = l[t];
      }
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int e = 0; e < DPP; ++e) pr[2 + p * PD + DPP * lane + e] = o[t][p][e];
    }
  }
  __shared__ int last;
  __shared__ float wsl[4 * 256];
  merge_if_last<HD>(part, out, counters, kvh, G, nsplit, jmin / SPLIT, (total + SPLIT - 1) / SPLIT, wave, &last, wsl,
                    gb, GH, kvh * HG + hg);
}

template <int HD>
static void attn_decode_hd(dim3 grid, hipStream_t st, const float* q, const void* kc, const void* vc, bool kv_f32,
                           float* out, float* part, int* counters, int n_heads, int n_kv, int ctx, const int* pos_dev,
                           int window, float scale, int nsplit) {
  if (kv_f32) {
    const int hgroups = n_heads / n_kv == 8 ? 2 : 1;  // the kernel's query-head split
    hipLaunchKernelGGL(attn_decode_f32_kernel<HD>, dim3(grid.x * hgroups, grid.y), dim3(256), 0, st, q,
                       (const float*)kc, (const float*)vc, part, out, counters, n_heads, n_kv, ctx, pos_dev, window,
                       scale, nsplit);
  } else {
    // fp16 cache: chunks of spc slices; one partial slot per chunk
    static int target = -1;
    if (target < 0) {
      const char* e = getenv("IEK_ATTN_CHUNKS");
      target = e ? std::max(1, atoi(e)) : 32;
    }
    const int spc = attn_slices_per_chunk(nsplit * SPLIT, window, target);
    const int nchunk = (nsplit + spc - 1) / spc;
    hipLaunchKernelGGL(attn_decode_kernel<HD>, dim3(grid.x, nchunk), dim3(256), 0, st, q, (const __half*)kc,
                       (const __half*)vc, part, out, counters, n_heads, n_kv, ctx, pos_dev, window, scale, nchunk,
                       spc);
  }
}

void launch_attn_decode(const float* q, const void* kc, const void* vc, bool kv_f32, float* out, float* part,
                        int* counters, int n_heads, int n_kv, int head_dim, int ctx, const int* pos_dev, int window,
                        float scale, int max_len, hipStream_t st) {
  const int nsplit = (max_len + SPLIT - 1) / SPLIT;
  dim3 grid(n_kv, nsplit);
  if (n_kv <= 0 || n_heads % n_kv != 0 || n_heads / n_kv > 8)
    fail(ST_OP, "attention: GQA group must divide the heads and be at most 8");
  switch (head_dim) {
#define IEK_AD(HD)                                                                                               \
  attn_decode_hd<HD>(grid, st, q, kc, vc, kv_f32, out, part, counters, n_heads, n_kv, ctx, pos_dev, window, scale, \
                     nsplit)
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

void launch_attn_prefill(const float* q, const float* k, const float* v, float* out, int M, int n_heads, int n_kv,
                         int head_dim, int window, float scale, hipStream_t st) {
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
