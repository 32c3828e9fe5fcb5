// Decode attention device code over a per-layer KV cache [n_kv][ctx][head_dim] (f32 or fp16
// elements), used by the decode attention kernels (attention.hip).
// src/layers/attention.rs:462-655 (decode_attention_layer): split-K flash-decode over 64-key
// slices, GQA groups sharing one K/V stream, (max, sum, o[]) partials merged per query head.
#pragma once
#include "common.cuh"
#include "../iek_internal.h"

namespace iek {

constexpr int SPLIT = 64;

// One 256-thread workgroup per (KV head, 64-key slice): the four waves load the slice's K and V
// rows (fp16) into LDS together in one burst of clamped, unconditional 16-byte loads, then wave w
// takes query heads w and w+4 of the GQA group. Lane j scores key j against its head (K row from
// LDS, q broadcast from LDS), the wave forms the slice softmax, and for P.V lane l owns head dims
// [DPL*l, DPL*l + DPL). Slices publish (max, sum, o[]) partials; the last workgroup of each KV
// head to finish merges its query heads (counted with an agent-scope acq_rel atomic per KV head).
// Merge of the live slice partials of query head h by one wave: global (max, sum) over slices,
// then each lane folds its head dims of every slice with the rescaled weights. One round trip
// fetches lane s's (max, sum) pair together with the first batch of B o rows; further batches
// follow only for more than B live slots.
template <int HD, bool COH = false, int B = (HD >= 512 ? 4 : 2048 / HD)>
IEK_DEV void merge_head(const float* __restrict__ part, float* __restrict__ out, int h, int nsplit, int s0, int nlive,
                        float* wsl) {
  constexpr int DPL = HD / 64;
  const int lane = threadIdx.x & 63;
  const int ns = min(nlive - s0, 256);
  const float* pr = part + ((size_t)h * nsplit + s0) * (HD + 2);
  const int sl = min(lane, ns - 1);
  const float m_l = ld_f<COH>(pr + (size_t)sl * (HD + 2));
  const float l_l = ld_f<COH>(pr + (size_t)sl * (HD + 2) + 1);
  float v[B][DPL];
  auto load_rows = [&](int b0) {
    // clamped, unconditional loads: the batch's rows are in flight together
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const size_t row = (size_t)min(b0 + u, ns - 1) * (HD + 2) + 2 + DPL * lane;
#pragma unroll
      for (int t = 0; t < DPL; ++t) v[u][t] = ld_f<COH>(pr + row + t);
    }
  };
  load_rows(0);
  float M = lane < ns ? m_l : -INFINITY;
  for (int s = 64 + lane; s < ns; s += 64) M = fmaxf(M, ld_f<COH>(pr + (size_t)s * (HD + 2)));
  M = wave_max(M);
  float L = 0.f;
  if (lane < ns) {
    const float w = expf(m_l - M);
    L = l_l * w;
    wsl[lane] = w;
  }
  for (int s = 64 + lane; s < ns; s += 64) {
    const float w = expf(ld_f<COH>(pr + (size_t)s * (HD + 2)) - M);
    L += ld_f<COH>(pr + (size_t)s * (HD + 2) + 1) * w;
    wsl[s] = w;
  }
  L = wave_sum(L);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float acc[DPL];
#pragma unroll
  for (int t = 0; t < DPL; ++t) acc[t] = 0.f;
  for (int b0 = 0; b0 < ns; b0 += B) {
    if (b0 > 0) load_rows(b0);
#pragma unroll
    for (int u = 0; u < B; ++u) {
      if (b0 + u < ns) {
        const float w = wsl[b0 + u];
#pragma unroll
        for (int t = 0; t < DPL; ++t) acc[t] += v[u][t] * w;
      }
    }
  }
  // slices beyond the 256 staged weights (contexts over 16K keys) use direct weights
  for (int s = 256; s < nlive - s0; ++s) {
    const float w = expf(ld_f<COH>(pr + (size_t)s * (HD + 2)) - M);
#pragma unroll
    for (int t = 0; t < DPL; ++t) acc[t] += ld_f<COH>(pr + (size_t)s * (HD + 2) + 2 + DPL * lane + t) * w;
  }
#pragma unroll
  for (int t = 0; t < DPL; ++t) st_f<COH>(out + (size_t)h * HD + DPL * lane + t, acc[t] / L);
}

// The last workgroup of a KV head to finish merges the group's heads. Release: the workgroup
// barrier orders every wave's partial stores before thread 0's agent-scope acq_rel add (which
// writes back this XCD's L2); the last arrival's acquire side invalidates its L2 before the
// partials are read. The counter is reset for the next launch.
// s0 .. nlive-1 are the live partial slots of the KV head. WIDE: up to twice the batch when that
// fetches the live slots in one round trip (many-slot merges).
template <int HD, bool COH = false, bool WIDE = false>
// The last workgroup to arrive on counters[cidx] merges query heads [gb, gb + gn) of KV head kvh
// (G query heads per KV head).
IEK_DEV void merge_if_last(const float* __restrict__ part, float* __restrict__ out, int* __restrict__ counters,
                           int kvh, int G, int nsplit, int s0, int nlive, int wave, int* last_s, float* wsl,
                           int gb = 0, int gn = -1, int cidx = -1) {
  if (gn < 0) gn = G;
  if (cidx < 0) cidx = kvh;
  int& last = *last_s;
  // every wave's partial stores complete before thread 0's release (the workgroup barrier alone
  // does not wait for global stores on this target)
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    // COH: the partials went out with coherent stores and were waited for above, so a relaxed
    // count (no L2 write-back / invalidate) orders them
    const int old = COH ? __hip_atomic_fetch_add(&counters[cidx], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                        : __hip_atomic_fetch_add(&counters[cidx], 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    last = old == nlive - s0 - 1;
    if (last) __hip_atomic_store(&counters[cidx], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last) return;
  if (!COH) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  constexpr int B1 = HD >= 512 ? 4 : 2048 / HD;  // 32 floats per lane
  const bool wide = WIDE && nlive - s0 > B1 && nlive - s0 <= 2 * B1;
  for (int g = gb + wave; g < gb + gn; g += 4) {
    if (WIDE && wide)
      merge_head<HD, COH, 2 * B1>(part, out, kvh * G + g, nsplit, s0, nlive, wsl + 256 * wave);
    else
      merge_head<HD, COH, B1>(part, out, kvh * G + g, nsplit, s0, nlive, wsl + 256 * wave);
  }
}

// LDS of one slice item: K rows (padded), V rows (HD <= 256), the group's q, the wave's
// probabilities, the merge weights and the last-arrival flag; K, V and the probabilities once per
// slice stream (SETS).
template <int HD, int SETS = 1, typename T = __half>
struct AttnSmem {
  static constexpr int ES = (int)sizeof(T);
  static constexpr int KROW = HD + 16 / ES;  // padded K row: 16 bytes
  static constexpr bool VL = HD <= 256;
  static constexpr size_t KS1 = (size_t)SPLIT * KROW * ES, VS1 = VL ? (size_t)SPLIT * HD * ES : 16;
  static constexpr size_t KS = SETS * KS1, VS = SETS * VS1, QS = 8 * (size_t)HD * 4, PS = 4 * SETS * SPLIT * 4,
                          WS = 4 * 256 * 4;
  static constexpr size_t BYTES = KS + VS + QS + PS + WS + 16;
  T* ks;
  T* vs;
  float* qs;
  float* ps;
  float* wsl;
  int* last;
  IEK_DEV explicit AttnSmem(char* base) {
    ks = reinterpret_cast<T*>(base);
    vs = reinterpret_cast<T*>(base + KS);
    qs = reinterpret_cast<float*>(base + KS + VS);
    ps = reinterpret_cast<float*>(base + KS + VS + QS);
    wsl = reinterpret_cast<float*>(base + KS + VS + QS + PS);
    last = reinterpret_cast<int*>(base + KS + VS + QS + PS + WS);
  }
};

// Cache elements as floats: N consecutive values of an f32 or fp16 cache row.
template <int N>
IEK_DEV void kv_load(const float* p, float* f) {
  static_assert(N % 2 == 0 || N == 1, "count");
  if constexpr (N == 1) {
    f[0] = *p;
  } else if constexpr (N == 2) {
    const float2 a = *reinterpret_cast<const float2*>(p);
    f[0] = a.x;
    f[1] = a.y;
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      const float4 a = *reinterpret_cast<const float4*>(p + i);
      f[i] = a.x;
      f[i + 1] = a.y;
      f[i + 2] = a.z;
      f[i + 3] = a.w;
    }
  }
}
template <int N>
IEK_DEV void kv_load(const __half* p, float* f) {
  if constexpr (N == 1) {
    f[0] = __half2float(*p);
  } else if constexpr (N == 2) {
    const float2 a = __half22float2(*reinterpret_cast<const __half2*>(p));
    f[0] = a.x;
    f[1] = a.y;
  } else if constexpr (N == 4) {
    const uint2 raw = *reinterpret_cast<const uint2*>(p);
    const __half2* h2 = reinterpret_cast<const __half2*>(&raw);
    const float2 a0 = __half22float2(h2[0]), a1 = __half22float2(h2[1]);
    f[0] = a0.x;
    f[1] = a0.y;
    f[2] = a1.x;
    f[3] = a1.y;
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 8) {
      const uint4 raw = *reinterpret_cast<const uint4*>(p + i);
      const __half2* h2 = reinterpret_cast<const __half2*>(&raw);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float2 a = __half22float2(h2[d]);
        f[i + 2 * d] = a.x;
        f[i + 2 * d + 1] = a.y;
      }
    }
  }
}

// One (KV head, head group, chunk) item of the decode attention over an f32 or fp16 cache (T), by
// one 256-thread workgroup: the chunk is `spc` consecutive 64-key slices. Each slice's K and V
// rows are loaded in one burst of clamped, unconditional 16-byte loads and staged in LDS; the
// loads of slice i+1 are in flight while slice i is computed. At head dim 512 the K slice fills
// the LDS, so V goes out once the K rows are staged and is staged in the same buffer after the
// scores. The GQA group's G query heads split into HG head groups of G / HG (one workgroup each,
// all streaming the same K / V); wave w takes heads w and w+4 of its group: lane = key for the
// scores, lane = head dims [DPL*l, DPL*l + DPL) for P.V, with a running (max, sum, o) across the
// chunk's slices. The chunk publishes its (max, sum, o[]) partials in slot `cp`; the last chunk
// of the (KV head, head group) to finish merges the group's heads (counter kvh * HG + hg).
// `total` = keys in the cache including this step's; chunks past the live range return at once
// (uniformly).
// SETS = 2 (512 threads): two slice streams, threads [256 s, 256 s + 256) taking the
// chunk's slices s, s + SETS, ... with their own LDS buffers and running (max, sum, o); streams
// 1.. hand their state to stream 0 through LDS at the end, and stream 0 publishes the partial. A
// chunk that is its KV head's only one (nslot = 1) writes the output itself (o / sum) instead.
template <int HD, bool COH = false, bool EARLY = false, int SETS = 1, typename T = __half>
IEK_DEV void attn_chunk(const float* __restrict__ q, const T* __restrict__ kc, const T* __restrict__ vc,
                        float* __restrict__ part, float* __restrict__ out, int* __restrict__ counters, int n_heads,
                        int n_kv, int ctx, const int* pos_dev, int total_in, int window, float scale, int nslot,
                        int kvh, int cp, int spc, char* smem, int hg = 0, int HG = 1) {
  constexpr int DPL = HD / 64;                          // head dims per lane in the PV phase
  constexpr int EPV = 16 / (int)sizeof(T);              // elements per 16-byte load
  constexpr int KROW = AttnSmem<HD, SETS, T>::KROW;     // padded K row: 16-byte reads of different rows spread banks
  constexpr int U4 = SPLIT * HD / EPV;                  // 16-byte loads per K (or V) slice
  // V is staged in LDS up to head_dim 256; at 512 the K slice, q and V would not fit together, so
  // the P.V phase reads V rows straight from memory (each row one coalesced 1 KB wave load).
  constexpr bool VL = HD <= 256;
  static_assert(HD == 64 || HD == 128 || HD == 256 || HD == 512, "head_dim");
  static_assert(SETS == 1 || SETS == 2, "slice streams");
  const int tid = threadIdx.x & 255, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int set = SETS == 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x >> 8);
  const int G = n_heads / n_kv, GH = G / HG, gb = hg * GH;  // the group's heads: gb .. gb + GH - 1
  const int CK = SPLIT * spc;
  const AttnSmem<HD, SETS, T> S(smem);
  auto ks = reinterpret_cast<T(*)[KROW]>(S.ks + (size_t)set * SPLIT * KROW);
  auto vs = reinterpret_cast<T(*)[VL ? HD : 8]>(S.vs + (VL ? (size_t)set * SPLIT * HD : 0));
  auto qs = reinterpret_cast<float(*)[HD]>(S.qs);
  auto ps = reinterpret_cast<float(*)[SPLIT]>(S.ps + (size_t)set * 4 * SPLIT);
  const T* kh = kc + (size_t)kvh * ctx * HD;
  const T* vh = vc + (size_t)kvh * ctx * HD;
  // native vectors (a HIP uint4 array captured by the lambda would not be promoted to registers)
  typedef uint32_t kv4_t __attribute__((ext_vector_type(4)));
  kv4_t kr[U4 / 256], vr[VL ? U4 / 256 : 1];
  // rows [j0, j0 + nk) of the cache; rows past nk repeat row j0 + nk - 1 (nk <= 0: row j0 + nk - 1,
  // within the cache for j0 + nk <= ctx)
  auto issue_rows = [&](int j0, int nk) {
#pragma unroll
    for (int u = 0; u < U4 / 256; ++u) {
      const int i = tid + 256 * u, row = j0 + min(i / (HD / EPV), nk - 1), c8 = i % (HD / EPV);
      kr[u] = *reinterpret_cast<const kv4_t*>(kh + (size_t)row * HD + EPV * c8);
      if constexpr (VL) vr[u] = *reinterpret_cast<const kv4_t*>(vh + (size_t)row * HD + EPV * c8);
    }
  };
  // head dim 512: the V rows of a slice into the K registers (after the K rows are staged)
  auto issue_v_rows = [&](int j0, int nk) {
#pragma unroll
    for (int u = 0; u < U4 / 256; ++u) {
      const int i = tid + 256 * u, row = j0 + min(i / (HD / EPV), nk - 1), c8 = i % (HD / EPV);
      kr[u] = *reinterpret_cast<const kv4_t*>(vh + (size_t)row * HD + EPV * c8);
    }
  };
  // EARLY (no window): the chunk's first slice does not depend on the position, so its rows (all
  // 64, within the cache) go out with q before the position load returns; rows past the live keys
  // get score -inf by a select and are skipped by P.V, so whatever they hold never reaches o.
  // q first (a fixed number of clamped loads per thread, G <= 8), so the wait for it leaves the
  // K / V loads in flight
  constexpr int QU = (8 * HD + 255) / 256;
  float qv[QU];
#pragma unroll
  for (int u = 0; u < QU; ++u) qv[u] = ld_f<COH>(q + (size_t)(kvh * G + gb) * HD + min(tid + 256 * u, GH * HD - 1));
  if constexpr (EARLY) issue_rows(cp * CK + SPLIT * set, min(SPLIT, ctx - cp * CK - SPLIT * set));
  typedef __attribute__((address_space(4))) const int* ConstInt;  // a scalar load
  const int total = pos_dev ? *(ConstInt)pos_dev + 1 : total_in;
  const int jmin = (window > 0 && total > window) ? total - window : 0;
  const int c0 = max(cp * CK, jmin), c1 = min(total, (cp + 1) * CK);
  if (c1 <= c0) return;  // uniform across the workgroup
#pragma unroll
  for (int u = 0; u < QU; ++u) {
    const int i = tid + 256 * u;
    if (i < GH * HD) qs[i / HD][i % HD] = qv[u];
  }
  const int sb0 = c0 / SPLIT, sb1 = (c1 + SPLIT - 1) / SPLIT;
  auto issue = [&](int sb) {
    const int j0 = max(sb * SPLIT, c0);
    issue_rows(j0, min((sb + 1) * SPLIT, c1) - j0);
  };
  if constexpr (!EARLY) issue(sb0 + set);
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f}, o_run[2][DPL];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int d = 0; d < DPL; ++d) o_run[t][d] = 0.f;
  for (int pb = sb0; pb < sb1; pb += SETS) {
    const int sb = pb + set;  // this stream's slice (none past sb1: the stream idles this round)
    const int j0 = max(sb * SPLIT, c0), nk = min((sb + 1) * SPLIT, c1) - j0;
    __syncthreads();  // the previous slice's LDS reads are done
#pragma unroll
    for (int u = 0; u < U4 / 256; ++u) {
      const int i = tid + 256 * u, row = i / (HD / EPV), c8 = i % (HD / EPV);
      *reinterpret_cast<kv4_t*>(&ks[row][EPV * c8]) = kr[u];
      if constexpr (VL) *reinterpret_cast<kv4_t*>(&vs[row][EPV * c8]) = vr[u];
    }
    __syncthreads();
    if constexpr (!VL) {
      // head dim 512: this slice's V rows go out while the scores run, then replace K in LDS
      issue_v_rows(j0, nk);
      const bool valid = lane < nk;
      float pv[2] = {0.f, 0.f}, cv[2] = {1.f, 1.f};
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int g = wave + 4 * t;
        if (g >= GH) break;
        float sc = 0.f;
#pragma unroll 8
        for (int c = 0; c < HD / 8; ++c) {
          float k8[8];
          kv_load<8>(&ks[lane][8 * c], k8);
          const float4 qa = *reinterpret_cast<const float4*>(&qs[g][8 * c]);
          const float4 qb = *reinterpret_cast<const float4*>(&qs[g][8 * c + 4]);
          sc += qa.x * k8[0] + qa.y * k8[1] + qa.z * k8[2] + qa.w * k8[3] + qb.x * k8[4] + qb.y * k8[5] +
                qb.z * k8[6] + qb.w * k8[7];
        }
        const float s = valid ? sc * scale : -INFINITY;
        const float m_new = fmaxf(m_run[t], wave_max(s));
        cv[t] = m_run[t] == -INFINITY ? 1.f : expf(m_run[t] - m_new);
        pv[t] = valid ? expf(s - m_new) : 0.f;
        l_run[t] = l_run[t] * cv[t] + wave_sum(pv[t]);
        m_run[t] = m_new;
      }
      __syncthreads();  // every wave's K reads are done
#pragma unroll
      for (int u = 0; u < U4 / 256; ++u) {
        const int i = tid + 256 * u, row = i / (HD / EPV), c8 = i % (HD / EPV);
        *reinterpret_cast<kv4_t*>(&ks[row][EPV * c8]) = kr[u];
      }
      __syncthreads();
      if (sb + SETS < sb1) issue(sb + SETS);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int g = wave + 4 * t;
        if (g >= GH) break;
        ps[wave][lane] = pv[t];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float o[DPL];
#pragma unroll
        for (int d = 0; d < DPL; ++d) o[d] = o_run[t][d] * cv[t];
#pragma unroll 8
        for (int j = 0; j < nk; ++j) {
          const float pj = ps[wave][j];
          float vv[DPL];
          kv_load<DPL>(&ks[j][DPL * lane], vv);
#pragma unroll
          for (int d = 0; d < DPL; ++d) o[d] += pj * vv[d];
        }
#pragma unroll
        for (int d = 0; d < DPL; ++d) o_run[t][d] = o[d];
        __builtin_amdgcn_wave_barrier();  // ps[wave] is rewritten by the next head
      }
      continue;
    }
    if (sb + SETS < sb1) issue(sb + SETS);
    if (SETS > 1 && sb >= sb1) continue;
    const bool valid = lane < nk;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int g = wave + 4 * t;
      if (g >= GH) break;
      // scores: lane = key
      float sc = 0.f;
#pragma unroll
      for (int c = 0; c < HD / 8; ++c) {
        float k8[8];
        kv_load<8>(&ks[lane][8 * c], k8);
        const float4 qa = *reinterpret_cast<const float4*>(&qs[g][8 * c]);
        const float4 qb = *reinterpret_cast<const float4*>(&qs[g][8 * c + 4]);
        sc += qa.x * k8[0] + qa.y * k8[1] + qa.z * k8[2] + qa.w * k8[3] + qb.x * k8[4] + qb.y * k8[5] +
              qb.z * k8[6] + qb.w * k8[7];
      }
      const float s = valid ? sc * scale : -INFINITY;
      const float m_new = fmaxf(m_run[t], wave_max(s));
      const float corr = m_run[t] == -INFINITY ? 1.f : expf(m_run[t] - m_new);
      const float p = valid ? expf(s - m_new) : 0.f;
      l_run[t] = l_run[t] * corr + wave_sum(p);
      m_run[t] = m_new;
      ps[wave][lane] = p;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // P.V over the slice's live keys only: lane owns dims DPL*lane .. +DPL-1. Rows past them may
      // hold anything (the cache is not cleared between conversations), so they are not read
      // here, not even with weight 0 (0 * inf is NaN).
      float o[DPL];
#pragma unroll
      for (int d = 0; d < DPL; ++d) o[d] = o_run[t][d] * corr;
#pragma unroll 8
      for (int j = 0; j < nk; ++j) {
        const float pj = ps[wave][j];
        float vv[DPL];
        kv_load<DPL>(&vs[j][DPL * lane], vv);
#pragma unroll
        for (int d = 0; d < DPL; ++d) o[d] += pj * vv[d];
      }
#pragma unroll
      for (int d = 0; d < DPL; ++d) o_run[t][d] = o[d];
      __builtin_amdgcn_wave_barrier();  // ps[wave] is rewritten by the next head or slice
    }
  }
  if constexpr (SETS > 1) {
    // streams 1..'s (max, sum, o) per head into the free K buffer of stream 0, folded in by stream 0
    float* hand = reinterpret_cast<float*>(S.ks);  // [SETS - 1][4 waves][2 heads][HD + 2]
    __syncthreads();
    if (set > 0) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (wave + 4 * t >= GH) break;
        float* hp = hand + (size_t)(8 * (set - 1) + 2 * wave + t) * (HD + 2);
        if (lane == 0) {
          hp[0] = m_run[t];
          hp[1] = l_run[t];
        }
#pragma unroll
        for (int d = 0; d < DPL; ++d) hp[2 + DPL * lane + d] = o_run[t][d];
      }
    }
    __syncthreads();
    if (set == 0) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (wave + 4 * t >= GH) break;
        for (int s1 = 1; s1 < SETS; ++s1) {
          const float* hp = hand + (size_t)(8 * (s1 - 1) + 2 * wave + t) * (HD + 2);
          const float m1 = hp[0], l1 = hp[1];
          // stream 0 always has a live key (c1 > c0), so m_new is finite
          const float m_new = fmaxf(m_run[t], m1);
          const float w0 = expf(m_run[t] - m_new), w1 = m1 == -INFINITY ? 0.f : expf(m1 - m_new);
          l_run[t] = l_run[t] * w0 + l1 * w1;
          m_run[t] = m_new;
#pragma unroll
          for (int d = 0; d < DPL; ++d) o_run[t][d] = o_run[t][d] * w0 + hp[2 + DPL * lane + d] * w1;
        }
      }
    }
  }
  if (nslot == 1) {
    // the KV head's only chunk: the output directly, as the merge of one partial would give it
    if (set == 0) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int g = wave + 4 * t;
        if (g >= GH) break;
#pragma unroll
        for (int d = 0; d < DPL; ++d)
          st_f<COH>(out + (size_t)(kvh * G + gb + g) * HD + DPL * lane + d, o_run[t][d] / l_run[t]);
      }
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int g = wave + 4 * t;
    if (g >= GH || set != 0) break;
    float* pr = part + ((size_t)(kvh * G + gb + g) * nslot + cp) * (HD + 2);
    if (lane == 0) {
      st_f<COH>(pr, m_run[t]);
      st_f<COH>(pr + 1, l_run[t]);
    }
#pragma unroll
    for (int d = 0; d < DPL; ++d) st_f<COH>(pr + 2 + DPL * lane + d, o_run[t][d]);
  }
  // stream 1's waves pass a wave index past the group: they take part in the arrival only
  merge_if_last<HD, COH, (SETS > 1)>(part, out, counters, kvh, G, nslot, jmin / CK, (total + CK - 1) / CK,
                                      set ? 8 : wave, S.last, S.wsl, gb, GH, kvh * HG + hg);
}

// Slices per chunk for a cache of `max_len` keys: one up to `target` slices per KV head, then
// enough that a KV head has at most ~`target` chunks (fewer workgroups, and fewer partials for
// the merge).
__host__ __device__ inline int attn_slices_per_chunk(int max_len, int window = 0, int target = 32) {
  int nsl = (max_len + SPLIT - 1) / SPLIT;
  // a window keeps only ~window / SPLIT + 1 slices live: size the chunks for those
  if (window > 0) nsl = min(nsl, (window + SPLIT - 1) / SPLIT + 1);
  return nsl <= target ? 1 : (nsl + target - 1) / target;
}

}  // namespace iek
