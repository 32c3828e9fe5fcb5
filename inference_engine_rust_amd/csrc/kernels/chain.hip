// Decode chain: a run of dependent decode matvec phases (e.g. O + residual -> RMSNorm + gate/up +
// SwiGLU -> down + residual -> RMSNorm + Q/K/V + RoPE + KV append) in one persistent launch, with
// the weights of the next phases streaming while a phase waits for its input.
//
// Why: the per-launch decode matvecs lose ~5 us per launch to dispatch, the first-byte latency of
// the weight stream and the tail, five times per layer. Weights never depend on activations, so a
// workgroup that keeps its next rows in flight across the wait for the previous phase's output
// turns that latency into streaming time.
//
// Workgroup = one control wave + NC consumer waves, one workgroup per CU.
//  * Consumer wave c owns items c, c + NC, ... of every phase (an item is one weight row, or one
//    4096-wide pass of a wider row). It copies each item's bytes from HBM straight into its own
//    LDS slots with global_load_lds_dwordx4 (no registers, no waits until the bytes are needed),
//    DSLOT items ahead, across phase boundaries, and touches the lines of the item DSLOT further
//    ahead so that its copy finds them in L2. Its only vector-memory operations are these copies,
//    so `s_waitcnt vmcnt` counts them exactly: every item is COPIES_PER_ITEM (four) copy
//    instructions, padded (five with the L2 touch), and the wait before computing an item is a
//    constant. The copies gather each lane's bytes into
//    lane-contiguous 16-byte columns, so the LDS reads are conflict-free.
//  * The control wave stages the phase input x into LDS (coherent copies: x was written by other
//    workgroups in this launch), in the register layout the consumers read (lane l's 64 values
//    as 16 float4 columns), with the RMSNorm sum of squares when the phase has a norm; it waits
//    for the consumers' partial dots, runs the epilogue (residual, SwiGLU, RoPE + f32 KV append,
//    logits + argmax), stores the outputs with coherent stores and arrives at the phase barrier.
//  * Phase barrier: two-level arrival counters (eight groups of workgroups, then one counter),
//    agent-scope relaxed atomics; every wait is bounded (err[1] iterations, read at launch, so that
//    a test can shorten it) and a timeout sets err[0] and ends the launch. The last workgroup to
//    leave resets the counters.
//
// Arithmetic per row (f32 activations throughout, as the reference's f32 dot, src/ops/
// matmul.rs:176-204, reassociated): Q4_K sub-block sums d*sc*sum(x*q) - dmin*m*sum(x) with the
// nibbles fed to v_fma_mix_f32 as exact f16 subnormals; regrouped Q6_K quarter sums
// d*sc*(sum x*(q+32) - 32*sum x). The row's partial sums are added in pass order.
#include "chain.h"
#include "mv_core.cuh"

namespace iek {

namespace {

// 12 consumers with 2 slots each measured 1.3% faster than 8 with 3 (the same LDS ring bytes):
// the ring fills early in a phase transition, so more waves reducing beat deeper slots
constexpr int NC = 12;                // consumer waves
constexpr int DSLOT = 2;              // LDS slots (items in flight) per consumer
constexpr bool L2PF = false;          // touch each item's lines DSLOT items before its copy
constexpr int NT = 64 * (1 + NC);     // threads per workgroup
constexpr int SLOT = 3584;            // bytes per slot: 3 x 1 KB columns + 16 + 2 columns of 16 B
constexpr int XF4 = 4 * 16 * 64;      // x staging: up to 4 passes x 16 float4 columns x 64 lanes
constexpr int MAXPART = 512;          // partial dots per workgroup and phase
// copy instructions per item (issue_item), plus the L2 touch when L2PF: the consumers' vmcnt waits
constexpr int COPIES_PER_ITEM = 4;
constexpr int VM_PER_ITEM = COPIES_PER_ITEM + (L2PF ? 1 : 0);

typedef const __attribute__((address_space(4))) ChainPhase* CPhase;

// No memory clobber: the copy's LDS side is ordered by the explicit waits around it (vm_wait
// before a slot is read, an lgkmcnt wait before a slot is refilled), and without the clobber the
// compiler keeps the phase fields in scalar registers across copies.
// The LDS offset is wave-uniform by construction; readfirstlane puts it in a scalar register even
// where the compiler cannot prove that.
IEK_DEV void dma16(uint32_t lds_off, const void* g) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(__builtin_amdgcn_readfirstlane(lds_off)),
               "v"(g));
}
// sc1: device-coherent (bypasses the non-coherent per-XCD L2 copy), for data other workgroups
// wrote in this launch
IEK_DEV void dma16_coh(uint32_t lds_off, const void* g) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off sc1" ::"s"(__builtin_amdgcn_readfirstlane(lds_off)),
               "v"(g)
               : "memory");
}
// 4-byte copy per lane into LDS, used to touch one 128-byte line per lane so a later copy of the
// item finds it in L2
IEK_DEV void dma4(uint32_t lds_off, const void* g) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" ::"s"(__builtin_amdgcn_readfirstlane(lds_off)),
               "v"(g));
}
template <int N>
IEK_DEV void vm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
IEK_DEV uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p; }
IEK_DEV int lds_ld(const int* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
IEK_DEV void lds_st(int* p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
IEK_DEV unsigned g_ld(const unsigned* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

IEK_DEV size_t row_bytes_of(int dt, int K) {
  return dt == DT_Q4K ? (size_t)(K / QK_K) * Q4K_BYTES : q6r_row_bytes((size_t)(K / QK_K));
}

// Pairs [u0, u1) of phase P owned by workgroup b of G.
IEK_DEV void unit_range(int units, int b, int G, int& u0, int& u1) {
  u0 = (units * b) / G;  // units * G < 2^31 (checked on the host)
  u1 = (units * (b + 1)) / G;
}
IEK_DEV int phase_items(const CPhase P, int b, int G) {
  int u0, u1;
  unit_range(P->units, b, G, u0, u1);
  return (u1 - u0) * 2 * P->npass;
}

// Wave-uniform view of one phase for this workgroup: where item i's weight row is.
struct PhaseView {
  const uint8_t *w0, *w1, *w2;  // separate fields: a dynamically indexed array would live in scratch
  size_t rb;  // row bytes
  int dt, K, lgp, n_items, u0, n0, n01, swiglu;
};

IEK_DEV PhaseView load_view(const CPhase P, int b, int G) {
  PhaseView v;
  int u0, u1;
  unit_range(P->units, b, G, u0, u1);
  v.w0 = P->seg[0].w;
  v.w1 = P->seg[1].w;
  v.w2 = P->seg[2].w;
  v.dt = P->dt;
  v.K = P->K;
  v.rb = row_bytes_of(v.dt, v.K);
  const int npass = P->npass;
  v.lgp = npass == 4 ? 2 : (npass == 2 ? 1 : 0);
  v.n_items = (u1 - u0) * 2 * npass;
  v.u0 = u0;
  v.n0 = P->seg[0].n;
  v.n01 = v.n0 + P->seg[1].n;
  v.swiglu = P->epi == CE_SWIGLU;
  return v;
}

// Item i = (pair, row of the pair, pass) -> weight row and pass.
IEK_DEV const uint8_t* view_row(const PhaseView& v, int i, int& pass) {
  pass = i & ((1 << v.lgp) - 1);
  const int q = i >> v.lgp, r = q & 1, u = v.u0 + (q >> 1);
  // the segment base by arithmetic: a select over the three pointer fields is turned into an
  // indexed load from a private copy of the struct (scratch memory, a vector load whose wait would
  // drain the copies in flight)
  const uintptr_t b0 = reinterpret_cast<uintptr_t>(v.w0), b1 = reinterpret_cast<uintptr_t>(v.w1),
                  b2 = reinterpret_cast<uintptr_t>(v.w2);
  if (v.swiglu) return reinterpret_cast<const uint8_t*>(b0 + (uintptr_t)r * (b1 - b0) + (size_t)u * v.rb);
  const int g = 2 * u + r;
  const uintptr_t in1 = g >= v.n0, in2 = g >= v.n01;
  const int row = g - (in2 ? v.n01 : (in1 ? v.n0 : 0));
  return reinterpret_cast<const uint8_t*>(b0 + in1 * (b1 - b0) + in2 * (b2 - b1) + (size_t)row * v.rb);
}

// COPIES_PER_ITEM (four) copy instructions per item, on every path (the wait counts rely on it):
// three 1 KB columns of quants and one column of scales.
IEK_DEV void issue_item(int dt, int K, const uint8_t* row, int pass, uint32_t slot, int lane) {
  const int nchunk = K / 64, ch = min(lane + 64 * pass, nchunk - 1);
  if (dt == DT_Q4K) {
    const uint8_t* blk = row + (size_t)(ch >> 2) * Q4K_BYTES;
    const int g = ch & 3;
    dma16(slot, blk + 16 + 32 * g);
    dma16(slot + 1024, blk + 32 + 32 * g);
    dma16(slot + 2048, blk);
    if (lane == 0) dma16(slot + 3072, blk);  // padding copy
  } else {
    const int nsb = K / QK_K, j = ch >> 2, k = ch & 3;
    const uint8_t* m = row + (size_t)j * 192 + 48 * k;
    dma16(slot, m);
    dma16(slot + 1024, m + 16);
    dma16(slot + 2048, m + 32);
    // scales of this pass's 16 superblocks (lanes 0-15), then their d (lanes 16-17)
    const size_t rb = q6r_row_bytes(nsb);
    if (lane < 18) {
      const size_t off = lane < 16 ? (size_t)nsb * 192 + 16 * (size_t)min(16 * pass + lane, nsb - 1)
                                   : min((size_t)nsb * 208 + 32 * (size_t)pass + 16 * (size_t)(lane - 16), rb - 16);
      dma16(slot + 3072, row + off);  // lane l lands at slot + 3072 + 16 l
    }
  }
}

// One copy instruction per item: lane l touches the item's l-th 128-byte line (Q4_K: 18 lines of
// one 2304-byte pass; regrouped Q6_K: 24 lines of quants, 2 of scales and 1 of d).
IEK_DEV void prefetch_item(int dt, int K, const uint8_t* row, int pass, uint32_t sink, int lane) {
  size_t off;
  bool on;
  if (dt == DT_Q4K) {
    const size_t pb = (size_t)min(64 * (pass + 1), K / 64) * (Q4K_BYTES / 4) - (size_t)64 * pass * (Q4K_BYTES / 4);
    off = (size_t)64 * pass * (Q4K_BYTES / 4) + 128 * (size_t)lane;
    on = 128 * (size_t)lane < pb;
  } else {
    const int nsb = K / QK_K, j0 = 16 * pass, nj = min(16, nsb - j0);
    if (lane < 24) {
      off = (size_t)j0 * 192 + 128 * (size_t)lane;
      on = 128 * lane < nj * 192;
    } else {
      off = lane < 26 ? (size_t)nsb * 192 + 16 * (size_t)j0 + 128 * (size_t)(lane - 24) : (size_t)nsb * 208 + 2 * (size_t)j0;
      on = lane < 27;
    }
  }
  if (lane == 0 || on) dma4(sink, row + (on ? off : 0));
}

// Q4_K item: lane's 64-value chunk (sub-blocks 2g, 2g+1 of superblock ch/4). x: the chunk's 64
// values, xsl / xsh their two 32-sums.
IEK_DEV float q4_item(const uint8_t* slot, int lane, int ch, const float (&x)[64], float xsl, float xsh) {
  const uint4 q0 = *reinterpret_cast<const uint4*>(slot + 16 * lane);
  const uint4 q1 = *reinterpret_cast<const uint4*>(slot + 1024 + 16 * lane);
  const uint4 hdr = *reinterpret_cast<const uint4*>(slot + 2048 + 16 * lane);
  const int g = ch & 3;
  const float d = half_bits_to_float(hdr.x), dmin = half_bits_to_float(hdr.x >> 16);
  float sc0, m0, sc1, m1;
  scale_min_k4_sel(2 * g, hdr.y, hdr.z, hdr.w, &sc0, &m0);
  scale_min_k4_sel(2 * g + 1, hdr.y, hdr.z, hdr.w, &sc1, &m1);
  const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
  float sl = 0.f, sh = 0.f, sl2 = 0.f, sh2 = 0.f;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    // low nibbles as f16 subnormals q * 2^-24; high nibbles left in place, q * 2^-20
    const uint32_t w = qw[t], w8 = w >> 8;
    const uint32_t t0 = w & 0x000F000Fu, t1 = w & 0x00F000F0u, t2 = w8 & 0x000F000Fu, t3 = w8 & 0x00F000F0u;
    sl = fmaf(x[4 * t + 0], h_lo(t0), sl);
    sl2 = fmaf(x[4 * t + 2], h_hi(t0), sl2);
    sh = fmaf(x[32 + 4 * t + 0], h_lo(t1), sh);
    sh2 = fmaf(x[32 + 4 * t + 2], h_hi(t1), sh2);
    sl = fmaf(x[4 * t + 1], h_lo(t2), sl);
    sl2 = fmaf(x[4 * t + 3], h_hi(t2), sl2);
    sh = fmaf(x[32 + 4 * t + 1], h_lo(t3), sh);
    sh2 = fmaf(x[32 + 4 * t + 3], h_hi(t3), sh2);
  }
  sl += sl2;
  sh += sh2;
  return (d * sc0 * 16777216.0f) * sl - (dmin * m0) * xsl + (d * sc1 * 1048576.0f) * sh - (dmin * m1) * xsh;
}

// Regrouped Q6_K item: lane chunk ch = (superblock j, k = 2h + j16): weights l = 16*j16..+15 of
// half h in its four quarters. x[16 qd + t] is the value of quarter qd, l = 16*j16 + t; xq[qd]
// the quarter sums.
IEK_DEV float q6_core(const uint4& qa, const uint4& qb, const uint4& qh, uint32_t scw, float d, const float (&x)[64],
                      const float (&xq)[4]) {
  const uint32_t A[4] = {qa.x, qa.y, qa.z, qa.w}, B[4] = {qb.x, qb.y, qb.z, qb.w}, H[4] = {qh.x, qh.y, qh.z, qh.w};
  float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t qq[4] = {(A[t] & 0x0F0F0F0Fu) | ((H[t] << 4) & 0x30303030u),
                            (B[t] & 0x0F0F0F0Fu) | ((H[t] << 2) & 0x30303030u),
                            ((A[t] >> 4) & 0x0F0F0F0Fu) | (H[t] & 0x30303030u),
                            ((B[t] >> 4) & 0x0F0F0F0Fu) | ((H[t] >> 2) & 0x30303030u)};
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const uint32_t e = qq[qd] & 0x00FF00FFu, o = (qq[qd] >> 8) & 0x00FF00FFu;
      s[qd] = fmaf(x[16 * qd + 4 * t + 0], h_lo(e), s[qd]);
      s[qd] = fmaf(x[16 * qd + 4 * t + 2], h_hi(e), s[qd]);
      s[qd] = fmaf(x[16 * qd + 4 * t + 1], h_lo(o), s[qd]);
      s[qd] = fmaf(x[16 * qd + 4 * t + 3], h_hi(o), s[qd]);
    }
  }
  float sum = 0.f;
#pragma unroll
  for (int qd = 0; qd < 4; ++qd)
    sum += (d * (float)(int8_t)((scw >> (8 * qd)) & 0xFF)) * (16777216.0f * s[qd] - 32.0f * xq[qd]);
  return sum;
}

IEK_DEV float q6_item(const uint8_t* slot, int lane, int ch, int pass, const float (&x)[64], const float (&xq)[4]) {
  const uint4 qa = *reinterpret_cast<const uint4*>(slot + 16 * lane);
  const uint4 qb = *reinterpret_cast<const uint4*>(slot + 1024 + 16 * lane);
  const uint4 qh = *reinterpret_cast<const uint4*>(slot + 2048 + 16 * lane);
  const int jl = (ch >> 2) - 16 * pass, k = ch & 3;
  const uint32_t scw = *reinterpret_cast<const uint32_t*>(slot + 3072 + 16 * jl + 4 * k);
  const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(slot + 3072 + 256 + 2 * jl));
  return q6_core(qa, qb, qh, scw, d, x, xq);
}

// Element offset of value e (0..63) of chunk ch in x (the register layout of each dtype).
IEK_DEV int x_elem(int dt, int ch, int e) {
  if (dt == DT_Q4K) return 64 * ch + e;
  const int j = ch >> 2, k = ch & 3;
  return j * QK_K + 128 * (k >> 1) + 16 * (k & 1) + 32 * (e >> 4) + (e & 15);
}

struct Smem {
  uint8_t ring[NC * DSLOT][SLOT];
  float4 xs[XF4];  // x columns [pass][16][lane]; the norm weight columns follow x's passes
  float part[MAXPART];
  uint32_t sink[NC][64];  // landing words of the L2 prefetch copies (never read)
  float rms;
  int rows_done, x_ready, norm_done, abort_;
  unsigned spin;  // bounded-wait limit of this launch (err[1], or 1 << 22 when it is zero)
};

IEK_DEV void set_abort(Smem& S, int* err, int code) {
  if ((threadIdx.x & 63) == 0) __hip_atomic_store(err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  lds_st(&S.abort_, 1);
}

// ---- control wave ------------------------------------------------------------------------------
IEK_DEV void control(const ChainArgs& a, Smem& S, int pos) {
  const int lane = threadIdx.x & 63, b = blockIdx.x, G = gridDim.x;
  const CPhase phases = (CPhase)a.phases;
  int seq_end = 0, nnorm = 0;
  for (int ph = 0; ph < a.nphase; ++ph) {
    const CPhase P = phases + ph;
    const int dt = P->dt, K = P->K, npass = P->npass, nchunk = K / 64;
    seq_end += phase_items(P, b, G);
    int u0, u1;
    unit_range(P->units, b, G, u0, u1);
    // Inputs that do not depend on the previous phase go out before its barrier: the norm weight
    // columns (the staging region is free: every consumer has its previous x in registers), and
    // the epilogue's residual pair or RoPE (cos, sin) for lane = pair (the residual rows of a
    // RESID phase are this workgroup's own rows, written by it earlier or by an earlier launch).
    if (P->norm_w) {
      for (int p = 0; p < npass; ++p) {
        const int ch = min(lane + 64 * p, nchunk - 1);
        for (int i4 = 0; i4 < 16; ++i4)
          dma16(lds_addr(&S.xs[((npass + p) * 16 + i4) * 64]), P->norm_w + x_elem(dt, ch, 4 * i4));
      }
    }
    float2 pre = make_float2(0.f, 0.f);
    if (lane < u1 - u0) {
      const int u = u0 + lane;
      if (P->epi == CE_RESID) {
        pre = make_float2(ld_coh(P->resid + 2 * u), ld_coh(P->resid + 2 * u + 1));
      } else if (P->epi == CE_QKV && P->role0 == 0) {
        const int n0 = P->seg[0].n, n1 = P->seg[1].n, g0 = 2 * u;
        const int row = g0 - (g0 >= n0 + n1 ? n0 + n1 : (g0 >= n0 ? n0 : 0));
        const int d = row % P->head_dim;
        if (d < 2 * P->npairs) pre = reinterpret_cast<const float2*>(P->rope_cs)[(size_t)pos * P->npairs + d / 2];
      }
    }
    if (P->wait_prev) {
      const unsigned* top = a.counters + ((ph - 1) * 9 + 8) * 64;
      unsigned it = 0;
      while (g_ld(top) < 8u) {
        __builtin_amdgcn_s_sleep(1);
        if (++it > S.spin) {
          set_abort(S, a.err, 1);
          break;
        }
      }
      if (lds_ld(&S.abort_)) {
        vm_wait<0>();  // the norm weight copies in flight land before the wave ends
        return;
      }
    }
    // ---- stage x (and the norm weight) in the consumers' register layout
    if (P->x_mode == CX_EMBED_Q4K) {
      // lane = chunk: dequantise row *tok of the Q4_K table (chunk = superblock ch/4, part ch%4),
      // element by element as the reference (quant_k_handler.rs:38-82, q == 0 -> product 0)
      typedef const __attribute__((address_space(4))) uint32_t* CU32;
      // the host checks the ids it is given; one the previous step produced is clamped to the
      // table (a flagged step's id is never used)
      const uint32_t tok = min(*(CU32)a.tok, (uint32_t)P->emb_rows - 1u);
      for (int p = 0; p < npass; ++p) {
        const int ch = min(lane + 64 * p, nchunk - 1);
        const uint8_t* blk = P->emb + ((size_t)tok * K + 64 * (size_t)ch) / QK_K * Q4K_BYTES;
        const float d = half_bits_to_float(load_u16(blk)), dmin = half_bits_to_float(load_u16(blk + 2));
        const uint4 hdr = *reinterpret_cast<const uint4*>(blk);
        float sc0, m0, sc1, m1;
        const int g = ch & 3;
        scale_min_k4_sel(2 * g, hdr.y, hdr.z, hdr.w, &sc0, &m0);
        scale_min_k4_sel(2 * g + 1, hdr.y, hdr.z, hdr.w, &sc1, &m1);
        const uint8_t* qs = blk + 16 + 32 * g;
        for (int i4 = 0; i4 < 16; ++i4) {
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int i = 4 * i4 + e;
            const uint32_t byte = qs[i & 31];
            v[e] = i < 32 ? q4k_value(d, dmin, sc0, m0, byte & 0xFu) : q4k_value(d, dmin, sc1, m1, byte >> 4);
          }
          const float4 f = make_float4(v[0], v[1], v[2], v[3]);
          S.xs[(p * 16 + i4) * 64 + lane] = f;
          if (b == 0 && lane + 64 * p < nchunk) *reinterpret_cast<float4*>(P->emb_out + 64 * ch + 4 * i4) = f;
        }
      }
    } else {
      for (int p = 0; p < npass; ++p) {
        const int ch = min(lane + 64 * p, nchunk - 1);
        for (int i4 = 0; i4 < 16; ++i4) dma16_coh(lds_addr(&S.xs[(p * 16 + i4) * 64]), P->x + x_elem(dt, ch, 4 * i4));
      }
    }
    vm_wait<0>();
    if (P->norm_w) {
      // rms = sqrt(sum(x^2) / K + eps) (src/ops/rmsnorm.rs:44-45), the sum over valid chunks
      float ss = 0.f;
      for (int p = 0; p < npass; ++p) {
        if (lane + 64 * p >= nchunk) continue;
        for (int i4 = 0; i4 < 16; ++i4) {
          const float4 v = S.xs[(p * 16 + i4) * 64 + lane];
          ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
        }
      }
      ss = wave_sum(ss);
      if (lane == 0) S.rms = rms_of(ss, K, P->eps);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane == 0) lds_st(&S.x_ready, ph);
    // ---- wait for the consumers' partial dots
    unsigned it = 0;
    while (lds_ld(&S.rows_done) < seq_end) {
      __builtin_amdgcn_s_sleep(1);
      if (++it > S.spin || lds_ld(&S.abort_)) {
        set_abort(S, a.err, 2);
        break;
      }
    }
    if (P->norm_w) {
      // every consumer has finished its share of the normalisation (also those without items here)
      ++nnorm;
      it = 0;
      while (lds_ld(&S.norm_done) < NC * nnorm) {
        __builtin_amdgcn_s_sleep(1);
        if (++it > S.spin || lds_ld(&S.abort_)) {
          set_abort(S, a.err, 5);
          break;
        }
      }
    }
    if (lds_ld(&S.abort_)) {
      vm_wait<0>();
      return;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    // ---- epilogue: lane = row pair
    unsigned long long run_key = 0;
    for (int lu = lane; lu < u1 - u0; lu += 64) {
      float v[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        float s = 0.f;
        for (int p = 0; p < npass; ++p) s += S.part[(lu * 2 + r) * npass + p];
        v[r] = s;
      }
      const int u = u0 + lu;
      if (P->epi == CE_SWIGLU) {
        st_coh(P->seg[0].out + u, silu_mul(v[0], v[1]));
        continue;
      }
      const int n0 = P->seg[0].n, n1 = P->seg[1].n;
      const int g0 = 2 * u, si = g0 >= n0 + n1 ? 2 : (g0 >= n0 ? 1 : 0);
      const int row = g0 - (si == 2 ? n0 + n1 : (si == 1 ? n0 : 0));
      float* out = si == 0 ? P->seg[0].out : (si == 1 ? P->seg[1].out : P->seg[2].out);
      const int s = P->epi == CE_QKV ? si + P->role0 : si;  // Q, K or V
      if (P->epi == CE_RESID) {
        const float2 r = lu == lane ? pre : make_float2(ld_coh(P->resid + row), ld_coh(P->resid + row + 1));
        st_coh(out + row, r.x + v[0]);
        st_coh(out + row + 1, r.y + v[1]);
      } else if (P->epi == CE_QKV) {
        const int hd = P->head_dim, d = row % hd;
        float o0 = v[0], o1 = v[1];
        if (s < 2 && d < 2 * P->npairs) {
          const float2 cs = lu == lane ? pre : reinterpret_cast<const float2*>(P->rope_cs)[(size_t)pos * P->npairs + d / 2];
          o0 = rope_rotate(v[0], v[1], cs.x, cs.y, true);
          o1 = rope_rotate(v[1], v[0], cs.x, cs.y, false);
        }
        if (s == 0) {
          st_coh(out + row, o0);
          st_coh(out + row + 1, o1);
        } else {
          float* c = s == 1 ? P->kc : P->vc;
          const size_t dst = ((size_t)(row / hd) * P->ctx + pos) * hd + d;
          const float2 f2 = make_float2(o0, o1);
          __hip_atomic_store(reinterpret_cast<unsigned long long*>(c + dst), __builtin_bit_cast(unsigned long long, f2),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      } else if (P->epi == CE_ARGMAX) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          float z = v[r];
          if (P->softcap > 0.f) z = soft_cap(z, P->softcap);
          out[row + r] = z;
          const unsigned long long key = argmax_key_dev(z, (uint32_t)(row + r));
          run_key = key > run_key ? key : run_key;
          if (!isfinite(z)) atomicOr(a.amax_flag, 1);
        }
      } else {
        st_coh(out + row, v[0]);
        st_coh(out + row + 1, v[1]);
      }
    }
    if (P->epi == CE_ARGMAX) {
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(run_key, off, WAVE);
        run_key = o > run_key ? o : run_key;
      }
      if (lane == 0 && run_key) atomicMax(a.amax_key, run_key);
    }
    // ---- arrive: stores complete, then the group counter; the group's last arrival bumps the top
    vm_wait<0>();
    if (lane == 0) {
      const unsigned grp = b & 7, members = (G - grp + 7) / 8;
      const unsigned old = __hip_atomic_fetch_add(a.counters + (ph * 9 + grp) * 64, 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
      if (old + 1 == members)
        __hip_atomic_fetch_add(a.counters + (ph * 9 + 8) * 64, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---- consumer waves ----------------------------------------------------------------------------
// A cursor over this consumer's items (c, c + NC, ... of each phase, phases in order), passed by
// value so that it stays in scalar registers.
struct Cursor {
  PhaseView v;
  int ph, i;
};

IEK_DEV Cursor cursor_first(CPhase phases, int b, int G, int c, int lph) {
  Cursor q;
  q.ph = 0;
  q.i = c;
  q.v = load_view(phases, b, G);
  while (q.ph < lph && q.i >= q.v.n_items) {
    ++q.ph;
    q.v = load_view(phases + q.ph, b, G);
  }
  return q;
}

// Next item; the cursor stops at the consumer's last item (lph, li).
IEK_DEV Cursor cursor_next(Cursor q, CPhase phases, int b, int G, int c, int lph, int li) {
  if (q.ph == lph && q.i == li) return q;
  q.i += NC;
  while (q.ph < lph && q.i >= q.v.n_items) {
    ++q.ph;
    q.v = load_view(phases + q.ph, b, G);
    q.i = c;
  }
  return q;
}

IEK_DEV void consumer(const ChainArgs& a, Smem& S, int c) {
  const int lane = threadIdx.x & 63, b = blockIdx.x, G = gridDim.x;
  const CPhase phases = (CPhase)a.phases;
  // The last item of this consumer: cursors stop there and repeat it, so the number of copy
  // instructions in flight stays constant (DSLOT items).
  int lph = -1, li = 0;
  for (int ph = 0; ph < a.nphase; ++ph) {
    const int n = phase_items(phases + ph, b, G);
    if (n > c) {
      lph = ph;
      li = c + NC * ((n - 1 - c) / NC);
    }
  }
  // copies land DSLOT items ahead of the compute; the L2 prefetch runs DSLOT items further ahead
  Cursor dq, pq;
  int nissued = 0;
  const uint32_t sink = lds_addr(&S.sink[c][0]);
#define IEK_CHAIN_ISSUE()                                                                                      \
  do {                                                                                                         \
    int pass_;                                                                                                 \
    const uint8_t* row_ = view_row(dq.v, dq.i, pass_);                                                         \
    issue_item(dq.v.dt, dq.v.K, row_, pass_, lds_addr(&S.ring[c * DSLOT + nissued % DSLOT][0]), lane);       \
    if constexpr (L2PF) {                                                                                      \
      row_ = view_row(pq.v, pq.i, pass_);                                                                      \
      prefetch_item(pq.v.dt, pq.v.K, row_, pass_, sink, lane);                                                 \
      pq = cursor_next(pq, phases, b, G, c, lph, li);                                                          \
    }                                                                                                          \
    ++nissued;                                                                                                 \
    dq = cursor_next(dq, phases, b, G, c, lph, li);                                                            \
  } while (0)
  if (lph >= 0) {
    dq = cursor_first(phases, b, G, c, lph);
    if constexpr (L2PF) {
      pq = dq;
      for (int k = 0; k < DSLOT; ++k) pq = cursor_next(pq, phases, b, G, c, lph, li);
    }
    for (int k = 0; k < DSLOT; ++k) IEK_CHAIN_ISSUE();
  }
  float x[64];
  float xs_a = 0.f, xs_b = 0.f, xq[4] = {0.f, 0.f, 0.f, 0.f};
  int k = 0, nnorm = 0;
  for (int ph = 0; ph < a.nphase; ++ph) {
    const PhaseView cv = load_view(phases + ph, b, G);
    const int npass = 1 << cv.lgp, nchunk = cv.K / 64;
    const bool mine = c < cv.n_items;
    const bool norm = phases[ph].norm_w != nullptr;
    if (!mine && !norm) continue;
    unsigned it = 0;
    while (lds_ld(&S.x_ready) < ph) {
      __builtin_amdgcn_s_sleep(1);
      if (++it > S.spin || lds_ld(&S.abort_)) {
        set_abort(S, a.err, 3);
        break;
      }
    }
    if (lds_ld(&S.abort_)) {
      vm_wait<0>();  // the copies in flight land before the wave ends
      return;
    }
    asm volatile("" ::: "memory");
    if (norm) {
      // y = (x * w) / rms with the reference's two roundings (rmsnorm.rs:46-47), computed once in
      // LDS: consumer c takes float4 columns c, c + NC, ...; then every consumer waits for all
      const float rms = S.rms;
      for (int j = c; j < 16 * npass; j += NC) {
        const float4 v = S.xs[j * 64 + lane], w = S.xs[(16 * npass + j) * 64 + lane];
        S.xs[j * 64 + lane] = make_float4(div_rn(mul_rn(v.x, w.x), rms), div_rn(mul_rn(v.y, w.y), rms),
                                          div_rn(mul_rn(v.z, w.z), rms), div_rn(mul_rn(v.w, w.w), rms));
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (lane == 0) __hip_atomic_fetch_add(&S.norm_done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      ++nnorm;
      it = 0;
      while (lds_ld(&S.norm_done) < NC * nnorm) {
        __builtin_amdgcn_s_sleep(1);
        if (++it > S.spin || lds_ld(&S.abort_)) {
          set_abort(S, a.err, 4);
          break;
        }
      }
      if (lds_ld(&S.abort_)) {
        vm_wait<0>();
        return;
      }
      asm volatile("" ::: "memory");
    }
    if (!mine) continue;
    const int p = c & (npass - 1);  // this consumer's pass in the phase (NC % npass == 0)
#pragma unroll
    for (int i4 = 0; i4 < 16; ++i4) {
      const float4 v = S.xs[(p * 16 + i4) * 64 + lane];
      x[4 * i4] = v.x;
      x[4 * i4 + 1] = v.y;
      x[4 * i4 + 2] = v.z;
      x[4 * i4 + 3] = v.w;
    }
    xs_a = xs_b = 0.f;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      xs_a += x[e];
      xs_b += x[32 + e];
    }
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      float s4 = 0.f;
#pragma unroll
      for (int t = 0; t < 16; ++t) s4 += x[16 * qd + t];
      xq[qd] = s4;
    }
    const int ch = lane + 64 * p;
    for (int i = c; i < cv.n_items; i += NC, ++k) {
      vm_wait<VM_PER_ITEM * (DSLOT - 1)>();  // this item's copies have landed
      const uint8_t* slot = &S.ring[c * DSLOT + k % DSLOT][0];
      float v = cv.dt == DT_Q4K ? q4_item(slot, lane, min(ch, nchunk - 1), x, xs_a, xs_b)
                                : q6_item(slot, lane, min(ch, nchunk - 1), p, x, xq);
      v = wave_sum(ch < nchunk ? v : 0.f);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot's reads are done before its refill
      IEK_CHAIN_ISSUE();
      if (lane == 0) {
        S.part[i & (MAXPART - 1)] = v;
        // LDS operations of one wave complete in order: the count follows the partial
        __hip_atomic_fetch_add(&S.rows_done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
  }
  vm_wait<0>();
#undef IEK_CHAIN_ISSUE
}

__global__ __launch_bounds__(NT) void chain_kernel(ChainArgs args) {
  __shared__ Smem S;
  (void)args;
  const ChainArgs& a = *(const ChainArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (tid == 0) {
    S.rows_done = 0;
    S.x_ready = -1;
    S.norm_done = 0;
    S.abort_ = 0;
    const unsigned lim = (unsigned)__hip_atomic_load(a.err + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    S.spin = lim ? lim : (1u << 22);  // ~0.1-0.2 s: each iteration sleeps ~64 clocks
  }
  __syncthreads();
  typedef const __attribute__((address_space(4))) int* CInt;
  const int pos = a.pos ? *(CInt)a.pos : 0;
  if (wave == 0) control(a, S, pos);
  else consumer(a, S, wave - 1);
  __syncthreads();
  // leave: the last workgroup publishes the argmax token, bumps the position and resets counters
  if (tid == 0) {
    unsigned* exitc = a.counters + CHAIN_MAX_PHASES * 9 * 64;
    const unsigned old = __hip_atomic_fetch_add(exitc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == gridDim.x - 1) {
      if (a.finish_argmax) {
        const unsigned long long key = __hip_atomic_load(a.amax_key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // every folded logit leaves a nonzero key; none (the launch gave its waits up before the LM
        // head) flags the step, and the published id stays a valid one for the next step's lookup
        const uint32_t idx = key ? 0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull) : 0u;
        a.out_tok[0] = idx;
        const int i = a.step ? *a.step : 0;
        a.flags[i] = key ? __hip_atomic_load(a.amax_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 1;
        if (a.step) {
          a.gen[i] = idx;
          *a.step = i + 1;
        }
        *a.amax_key = 0ull;
        *a.amax_flag = 0;
      }
      if (a.pos_inc) *a.pos_inc += 1;
      for (int w = 0; w <= CHAIN_MAX_PHASES * 9; ++w)
        __hip_atomic_store(a.counters + w * 64, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ==== Tiled chain (launch_chain2) ================================================================
// The same phases and epilogues as chain_kernel, with a different decomposition:
//  * A workgroup's rows of a phase form 16-row tiles; an item is one tile's 16 rows of one
//    superblock (256 columns): 16 x 144 bytes (Q4_K) or 16 x 210 (regrouped Q6_K). Lane l of a
//    consumer takes row l & 15 and the 64-value chunk l >> 4 of that superblock, so each lane's dot
//    is the chain's per-lane arithmetic (q4_item / q6_core) on its own row; the four chunk lanes of
//    a row are summed with two cross-lane adds per item (no full-wave reduction per row).
//  * Items go sb-major (every tile of superblock 0, then of 1, ...); consumer c takes a contiguous
//    range of them and keeps the x values of its current superblock in registers.
//  * Superblock sb of a phase's x is ready once the workgroups that write part of it (ChainPhase::
//    expect[sb] of them) have arrived on its counter, so there is no phase-wide barrier: the control
//    wave polls the counters (lane = superblock), stages each ready superblock into LDS with one
//    device-coherent copy and flags it; a consumer starts on a superblock as soon as it is flagged.
//  * A fused RMSNorm no longer sits on that path: the consumers dot the rows with x * w, the control
//    wave takes sum(x^2) once every superblock is staged, and the epilogue divides the dots by rms
//    (the reference's (x * w) / rms, reassociated).
constexpr int NC2 = 12;
constexpr int DSLOT2 = 2;
constexpr int NT2 = 64 * (1 + NC2);

struct Smem2 {
  uint8_t ring[NC2 * DSLOT2][SLOT];
  float4 xs[CHAIN2_XS_FLOATS / 4];  // x per superblock as [sb][i4][chunk] float4; a norm's w after x
  float part[CHAIN2_MAX_TILES][NC2][16];
  int xflag[CHAIN2_MAX_SB];  // superblock staged for phase (value - 1)
  // consumers finished with each phase: per phase, since a consumer without items in a run of
  // phases signals them all at once (a cumulative count would let it stand in for a late one)
  int done[CHAIN_MAX_PHASES];
  int abort_;
  unsigned spin;
};

IEK_DEV unsigned* cnt2(const ChainArgs& a, int ph, int sb) {
  return a.counters + (size_t)(ph * CHAIN2_MAX_SB + sb) * CHAIN2_CNT_STRIDE;
}

IEK_DEV void set_abort2(Smem2& S, int* err, int code) {
  if ((threadIdx.x & 63) == 0) __hip_atomic_store(err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  lds_st(&S.abort_, 1);
}

// Wave-uniform geometry of one phase for this workgroup.
struct View2 {
  const uint8_t *w0, *w1, *w2;
  size_t rb;
  int dt, nsb, u0, R, T, n_items, n0, n01, swiglu;
};

IEK_DEV View2 load_view2(const CPhase P, int b, int G) {
  View2 v;
  int u0, u1;
  unit_range(P->units, b, G, u0, u1);
  v.w0 = P->seg[0].w;
  v.w1 = P->seg[1].w;
  v.w2 = P->seg[2].w;
  v.dt = P->dt;
  v.nsb = P->K / QK_K;
  v.rb = row_bytes_of(v.dt, P->K);
  v.u0 = u0;
  v.R = 2 * (u1 - u0);
  v.T = (v.R + 15) / 16;
  v.n_items = v.T * v.nsb;
  v.n0 = P->seg[0].n;
  v.n01 = v.n0 + P->seg[1].n;
  v.swiglu = P->epi == CE_SWIGLU;
  return v;
}

// Weight row of this workgroup's local row l (0 <= l < R): pair u0 + l / 2, row l & 1 of the pair.
IEK_DEV const uint8_t* view2_row(const View2& v, int l) {
  const int u = v.u0 + (l >> 1), r = l & 1;
  const uintptr_t b0 = reinterpret_cast<uintptr_t>(v.w0), b1 = reinterpret_cast<uintptr_t>(v.w1),
                  b2 = reinterpret_cast<uintptr_t>(v.w2);
  if (v.swiglu) return reinterpret_cast<const uint8_t*>(b0 + (uintptr_t)r * (b1 - b0) + (size_t)u * v.rb);
  const int g = 2 * u + r;
  const uintptr_t in1 = g >= v.n0, in2 = g >= v.n01;
  const int row = g - (in2 ? v.n01 : (in1 ? v.n0 : 0));
  return reinterpret_cast<const uint8_t*>(b0 + in1 * (b1 - b0) + in2 * (b2 - b1) + (size_t)row * v.rb);
}

// Items go tile-major (every superblock of tile 0, then of tile 1, ...) and are dealt to the
// consumers round-robin, so that a workgroup's copies in flight cover whole rows (contiguous
// bytes) rather than one superblock of many rows.
IEK_DEV void item2_of(const View2& v, int i, int& sb, int& t) {
  t = i / v.nsb;
  sb = i - t * v.nsb;
}

// COPIES_PER_ITEM copy instructions for item i (the consumer waits rely on the count). Q4_K: lane
// (n, g) copies the 32 quant bytes of chunk g of row n's superblock and the row's header; regrouped
// Q6_K: the chunk's three 16-byte quant columns, then lanes 0-15 row n's 16 scale bytes of the
// superblock and lanes 16-31 the 16 bytes holding its d. Rows past R repeat row R - 1.
IEK_DEV void issue_item2(const View2& v, int i, uint32_t slot, int lane) {
  int sb, t;
  item2_of(v, i, sb, t);
  const int g = lane >> 4;
  const uint8_t* row = view2_row(v, min(16 * t + (lane & 15), v.R - 1));
  if (v.dt == DT_Q4K) {
    const uint8_t* blk = row + (size_t)sb * Q4K_BYTES;
    dma16(slot, blk + 16 + 32 * g);
    dma16(slot + 1024, blk + 32 + 32 * g);
    dma16(slot + 2048, blk);
    if (lane == 0) dma16(slot + 3072, blk);  // padding copy
  } else {
    const uint8_t* m = row + (size_t)sb * 192 + 48 * g;
    dma16(slot, m);
    dma16(slot + 1024, m + 16);
    dma16(slot + 2048, m + 32);
    if (lane < 32) {
      const uint8_t* rn = view2_row(v, min(16 * t + (lane & 15), v.R - 1));
      const size_t off = lane < 16 ? (size_t)v.nsb * 192 + 16 * (size_t)sb
                                   : (size_t)v.nsb * 208 + ((2 * (size_t)sb) & ~(size_t)15);
      dma16(slot + 3072, rn + off);  // lane l lands at slot + 3072 + 16 l
    }
  }
}

IEK_DEV float q6_item2(const uint8_t* slot, int lane, int sb, const float (&x)[64], const float (&xq)[4]) {
  const uint4 qa = *reinterpret_cast<const uint4*>(slot + 16 * lane);
  const uint4 qb = *reinterpret_cast<const uint4*>(slot + 1024 + 16 * lane);
  const uint4 qh = *reinterpret_cast<const uint4*>(slot + 2048 + 16 * lane);
  const int n = lane & 15, k = lane >> 4;
  const uint32_t scw = *reinterpret_cast<const uint32_t*>(slot + 3072 + 16 * n + 4 * k);
  const float d =
      half_bits_to_float(*reinterpret_cast<const uint16_t*>(slot + 3072 + 256 + 16 * n + ((2 * sb) & 15)));
  return q6_core(qa, qb, qh, scw, d, x, xq);
}

// Whether consumer c has an item in tile t (items c, c + NC2, ... of n, nsb per tile).
IEK_DEV bool covers2(int n, int nsb, int c, int t) {
  const int start = t * nsb, end = min(n, start + nsb);
  const int first = start + ((c - start) % NC2 + NC2) % NC2;
  return first < end;
}

// ---- control wave ------------------------------------------------------------------------------
IEK_DEV void control2(const ChainArgs& a, Smem2& S, int pos) {
  const int lane = threadIdx.x & 63, b = blockIdx.x, G = gridDim.x;
  const CPhase phases = (CPhase)a.phases;
  for (int ph = 0; ph < a.nphase; ++ph) {
    const CPhase P = phases + ph;
    const View2 v = load_view2(P, b, G);
    const int dt = P->dt, K = P->K, nsb = v.nsb;
    const int u0 = v.u0, npair = v.R / 2;
    // epilogue inputs that do not depend on this phase's x: the residual pair or RoPE (cos, sin)
    // for lane = pair
    float2 pre = make_float2(0.f, 0.f);
    if (lane < npair) {
      const int u = u0 + lane;
      if (P->epi == CE_RESID) {
        pre = make_float2(ld_coh(P->resid + 2 * u), ld_coh(P->resid + 2 * u + 1));
      } else if (P->epi == CE_QKV && P->role0 == 0) {
        const int n0 = P->seg[0].n, n1 = P->seg[1].n, g0 = 2 * u;
        const int row = g0 - (g0 >= n0 + n1 ? n0 + n1 : (g0 >= n0 ? n0 : 0));
        const int d = row % P->head_dim;
        if (d < 2 * P->npairs) pre = reinterpret_cast<const float2*>(P->rope_cs)[(size_t)pos * P->npairs + d / 2];
      }
    }
    // the norm weight: lane l of superblock sb's copy is (i4 = l >> 2, chunk l & 3)
    const int lc = lane & 3, li4 = lane >> 2;
    if (P->norm_w)
      for (int sb = 0; sb < nsb; ++sb)
        dma16(lds_addr(&S.xs[K / 4 + sb * 64]), P->norm_w + x_elem(dt, 4 * sb + lc, 4 * li4));
    // ---- stage x, superblock by superblock
    if (P->x_mode == CX_EMBED_Q4K) {
      // dequantise row *tok of the Q4_K table (quant_k_handler.rs:38-82, q == 0 -> product 0);
      // the host checks the ids it is given, and one the previous step produced is clamped
      typedef const __attribute__((address_space(4))) uint32_t* CU32;
      const uint32_t tok = min(*(CU32)a.tok, (uint32_t)P->emb_rows - 1u);
      for (int sb = 0; sb < nsb; ++sb) {
        const int ch = 4 * sb + lc;
        const uint8_t* blk = P->emb + ((size_t)tok * K + 64 * (size_t)ch) / QK_K * Q4K_BYTES;
        const float d = half_bits_to_float(load_u16(blk)), dmin = half_bits_to_float(load_u16(blk + 2));
        const uint4 hdr = *reinterpret_cast<const uint4*>(blk);
        float sc0, m0, sc1, m1;
        scale_min_k4_sel(2 * lc, hdr.y, hdr.z, hdr.w, &sc0, &m0);
        scale_min_k4_sel(2 * lc + 1, hdr.y, hdr.z, hdr.w, &sc1, &m1);
        const uint8_t* qs = blk + 16 + 32 * lc;
        float vv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * li4 + e;
          const uint32_t byte = qs[i & 31];
          vv[e] = i < 32 ? q4k_value(d, dmin, sc0, m0, byte & 0xFu) : q4k_value(d, dmin, sc1, m1, byte >> 4);
        }
        const float4 f = make_float4(vv[0], vv[1], vv[2], vv[3]);
        S.xs[sb * 64 + lane] = f;
        if (b == 0) *reinterpret_cast<float4*>(P->emb_out + 64 * ch + 4 * li4) = f;
      }
      vm_wait<0>();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      if (lane < nsb) lds_st(&S.xflag[lane], ph + 1);
    } else {
      // lane = superblock: poll its counter; every ready superblock is staged with one
      // device-coherent copy (x was written by other workgroups in this launch) and flagged
      bool staged = lane >= nsb;
      const unsigned need = lane < nsb ? (unsigned)P->expect[lane] : 0u;
      unsigned it = 0;
      while (true) {
        bool ready = false;
        if (!staged) ready = P->x_src < 0 || g_ld(cnt2(a, P->x_src, lane)) >= need;
        unsigned long long m = __ballot(ready);
        if (m) {
          unsigned long long mm = m;
          while (mm) {
            const int sb = __builtin_ctzll(mm);
            mm &= mm - 1;
            dma16_coh(lds_addr(&S.xs[sb * 64]), P->x + x_elem(dt, 4 * sb + lc, 4 * li4));
          }
          vm_wait<0>();
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
          if (ready) lds_st(&S.xflag[lane], ph + 1);
          staged = staged || ready;
        }
        if (__ballot(!staged) == 0ull) break;
        if (!m) {
          __builtin_amdgcn_s_sleep(1);
          if (++it > S.spin || lds_ld(&S.abort_)) {
            set_abort2(S, a.err, 1);
            break;
          }
        }
      }
      if (lds_ld(&S.abort_)) {
        vm_wait<0>();
        return;
      }
    }
    vm_wait<0>();  // the norm weight copies (the embedding path issues none after its wait)
    float rms = 1.f;
    if (P->norm_w) {
      // rms = sqrt(sum(x^2) / K + eps) (src/ops/rmsnorm.rs:44-45) over the staged superblocks
      float ss = 0.f;
      for (int sb = 0; sb < nsb; ++sb) {
        const float4 q = S.xs[sb * 64 + lane];
        ss += (q.x * q.x + q.y * q.y) + (q.z * q.z + q.w * q.w);
      }
      rms = rms_of(wave_sum(ss), K, P->eps);
    }
    // ---- wait for the consumers' partial dots
    unsigned it = 0;
    while (lds_ld(&S.done[ph]) < NC2) {
      __builtin_amdgcn_s_sleep(1);
      if (++it > S.spin || lds_ld(&S.abort_)) {
        set_abort2(S, a.err, 2);
        break;
      }
    }
    if (lds_ld(&S.abort_)) {
      vm_wait<0>();
      return;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    // ---- epilogue: lane = row pair; each row's dot is the sum of the consumers' tile partials
    unsigned long long run_key = 0;
    for (int lu = lane; lu < npair; lu += 64) {
      float vv[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int l = 2 * lu + r, t = l >> 4, n = l & 15;
        float s = 0.f;
        for (int c = 0; c < NC2; ++c)
          if (covers2(v.n_items, v.nsb, c, t)) s += S.part[t][c][n];
        vv[r] = P->norm_w ? s / rms : s;
      }
      const int u = u0 + lu;
      if (P->epi == CE_SWIGLU) {
        st_coh(P->seg[0].out + u, silu_mul(vv[0], vv[1]));
        continue;
      }
      const int n0 = P->seg[0].n, n1 = P->seg[1].n;
      const int g0 = 2 * u, si = g0 >= n0 + n1 ? 2 : (g0 >= n0 ? 1 : 0);
      const int row = g0 - (si == 2 ? n0 + n1 : (si == 1 ? n0 : 0));
      float* out = si == 0 ? P->seg[0].out : (si == 1 ? P->seg[1].out : P->seg[2].out);
      const int s = P->epi == CE_QKV ? si + P->role0 : si;  // Q, K or V
      if (P->epi == CE_RESID) {
        const float2 r = lu == lane ? pre : make_float2(ld_coh(P->resid + row), ld_coh(P->resid + row + 1));
        st_coh(out + row, r.x + vv[0]);
        st_coh(out + row + 1, r.y + vv[1]);
      } else if (P->epi == CE_QKV) {
        const int hd = P->head_dim, d = row % hd;
        float o0 = vv[0], o1 = vv[1];
        if (s < 2 && d < 2 * P->npairs) {
          const float2 cs = lu == lane ? pre : reinterpret_cast<const float2*>(P->rope_cs)[(size_t)pos * P->npairs + d / 2];
          o0 = rope_rotate(vv[0], vv[1], cs.x, cs.y, true);
          o1 = rope_rotate(vv[1], vv[0], cs.x, cs.y, false);
        }
        if (s == 0) {
          st_coh(out + row, o0);
          st_coh(out + row + 1, o1);
        } else {
          float* c = s == 1 ? P->kc : P->vc;
          const size_t dst = ((size_t)(row / hd) * P->ctx + pos) * hd + d;
          const float2 f2 = make_float2(o0, o1);
          __hip_atomic_store(reinterpret_cast<unsigned long long*>(c + dst), __builtin_bit_cast(unsigned long long, f2),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      } else if (P->epi == CE_ARGMAX) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          float z = vv[r];
          if (P->softcap > 0.f) z = soft_cap(z, P->softcap);
          out[row + r] = z;
          const unsigned long long key = argmax_key_dev(z, (uint32_t)(row + r));
          run_key = key > run_key ? key : run_key;
          if (!isfinite(z)) atomicOr(a.amax_flag, 1);
        }
      } else {
        st_coh(out + row, vv[0]);
        st_coh(out + row + 1, vv[1]);
      }
    }
    if (P->epi == CE_ARGMAX) {
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(run_key, off, WAVE);
        run_key = o > run_key ? o : run_key;
      }
      if (lane == 0 && run_key) atomicMax(a.amax_key, run_key);
    }
    // ---- arrive: the stores are complete, then one count on each superblock of the next
    // phases' x that this workgroup's outputs touch
    vm_wait<0>();
    if (P->arrive && npair > 0) {
      const int lo = P->epi == CE_SWIGLU ? u0 : 2 * u0, hi = P->epi == CE_SWIGLU ? u0 + npair : 2 * (u0 + npair);
      const int sb0 = lo / QK_K, sb1 = (hi - 1) / QK_K;
      if (lane <= sb1 - sb0)
        __hip_atomic_fetch_add(cnt2(a, ph, sb0 + lane), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---- consumer waves ----------------------------------------------------------------------------
struct Cursor2 {
  View2 v;
  int ph, i;
};

// The first item of phase ph or later (consumer c's items are c, c + NC2, ... of each phase).
IEK_DEV Cursor2 cursor2_at(CPhase phases, int nphase, int b, int G, int c, int ph) {
  Cursor2 q;
  q.ph = ph;
  q.i = c;
  while (true) {
    q.v = load_view2(phases + q.ph, b, G);
    if (c < q.v.n_items || q.ph == nphase - 1) return q;
    ++q.ph;
  }
}

// Next item; at the consumer's last item the cursor stays there (the same item's copies are
// issued again, keeping the number of copies in flight constant).
IEK_DEV Cursor2 cursor2_next(Cursor2 q, CPhase phases, int nphase, int b, int G, int c) {
  if (q.i + NC2 < q.v.n_items) {
    q.i += NC2;
    return q;
  }
  int ph = q.ph + 1;
  while (ph < nphase) {
    const View2 v = load_view2(phases + ph, b, G);
    if (c < v.n_items) {
      q.v = v;
      q.ph = ph;
      q.i = c;
      return q;
    }
    ++ph;
  }
  return q;
}

IEK_DEV void consumer2(const ChainArgs& a, Smem2& S, int c) {
  const int lane = threadIdx.x & 63, b = blockIdx.x, G = gridDim.x;
  const int g = lane >> 4;
  const CPhase phases = (CPhase)a.phases;
  const int nph = a.nphase;
  Cursor2 dq = cursor2_at(phases, nph, b, G, c, 0);
  const bool any = c < dq.v.n_items;
  int nissued = 0;
#define IEK_CHAIN2_ISSUE()                                                                                   \
  do {                                                                                                       \
    issue_item2(dq.v, dq.i, lds_addr(&S.ring[c * DSLOT2 + nissued % DSLOT2][0]), lane);                    \
    ++nissued;                                                                                               \
    dq = cursor2_next(dq, phases, nph, b, G, c);                                                             \
  } while (0)
  if (any)
    for (int k = 0; k < DSLOT2; ++k) IEK_CHAIN2_ISSUE();
  float x[64];
  float xs_a = 0.f, xs_b = 0.f, xq[4] = {0.f, 0.f, 0.f, 0.f};
  int k = 0;
  for (int ph = 0; ph < nph; ++ph) {
    const CPhase P = phases + ph;
    const View2 cv = load_view2(P, b, G);
    const bool norm = P->norm_w != nullptr;
    const int K4 = P->K / 4;
    int cur = -1;
    for (int i = c; i < cv.n_items; i += NC2, ++k) {
      int sb, t;
      item2_of(cv, i, sb, t);
      if (sb != cur) {
        unsigned it = 0;
        while (lds_ld(&S.xflag[sb]) != ph + 1) {
          __builtin_amdgcn_s_sleep(1);
          if (++it > S.spin || lds_ld(&S.abort_)) {
            set_abort2(S, a.err, 3);
            break;
          }
        }
        if (lds_ld(&S.abort_)) {
          vm_wait<0>();  // the copies in flight land before the wave ends
          return;
        }
        asm volatile("" ::: "memory");
#pragma unroll
        for (int i4 = 0; i4 < 16; ++i4) {
          float4 q = S.xs[sb * 64 + 4 * i4 + g];
          if (norm) {
            const float4 w = S.xs[K4 + sb * 64 + 4 * i4 + g];
            q = make_float4(mul_rn(q.x, w.x), mul_rn(q.y, w.y), mul_rn(q.z, w.z), mul_rn(q.w, w.w));
          }
          x[4 * i4] = q.x;
          x[4 * i4 + 1] = q.y;
          x[4 * i4 + 2] = q.z;
          x[4 * i4 + 3] = q.w;
        }
        xs_a = xs_b = 0.f;
#pragma unroll
        for (int e = 0; e < 32; ++e) {
          xs_a += x[e];
          xs_b += x[32 + e];
        }
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          float s4 = 0.f;
#pragma unroll
          for (int e = 0; e < 16; ++e) s4 += x[16 * qd + e];
          xq[qd] = s4;
        }
        cur = sb;
      }
      vm_wait<VM_PER_ITEM * (DSLOT2 - 1)>();  // this item's copies have landed
      const uint8_t* slot = &S.ring[c * DSLOT2 + k % DSLOT2][0];
      float vv = cv.dt == DT_Q4K ? q4_item(slot, lane, g, x, xs_a, xs_b) : q6_item2(slot, lane, sb, x, xq);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot's reads are done before its refill
      IEK_CHAIN2_ISSUE();
      vv += __shfl_xor(vv, 16, WAVE);
      vv += __shfl_xor(vv, 32, WAVE);
      if (lane < 16) {
        // this consumer's first item of a tile writes its partial, later ones add
        float* pp = &S.part[t][c][lane];
        *pp = i - NC2 < t * cv.nsb ? vv : *pp + vv;
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (lane == 0) __hip_atomic_fetch_add(&S.done[ph], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  vm_wait<0>();
#undef IEK_CHAIN2_ISSUE
}

__global__ __launch_bounds__(NT2) void chain2_kernel(ChainArgs args) {
  __shared__ Smem2 S;
  __shared__ int last;
  (void)args;
  const ChainArgs& a = *(const ChainArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (tid < CHAIN2_MAX_SB) S.xflag[tid] = 0;
  if (tid < CHAIN_MAX_PHASES) S.done[tid] = 0;
  if (tid == 0) {
    S.abort_ = 0;
    const unsigned lim = (unsigned)__hip_atomic_load(a.err + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    S.spin = lim ? lim : (1u << 22);  // ~0.1-0.2 s: each iteration sleeps ~64 clocks
  }
  __syncthreads();
  typedef const __attribute__((address_space(4))) int* CInt;
  const int pos = a.pos ? *(CInt)a.pos : 0;
  if (wave == 0) control2(a, S, pos);
  else consumer2(a, S, wave - 1);
  __syncthreads();
  // leave: the last workgroup publishes the argmax token, bumps the position and clears the counters
  if (tid == 0) {
    unsigned* exitc = a.counters + (size_t)CHAIN_MAX_PHASES * CHAIN2_MAX_SB * CHAIN2_CNT_STRIDE;
    const unsigned old = __hip_atomic_fetch_add(exitc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old == gridDim.x - 1;
  }
  __syncthreads();
  if (!last) return;
  if (tid == 0) {
    if (a.finish_argmax) {
      const unsigned long long key = __hip_atomic_load(a.amax_key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // every folded logit leaves a nonzero key; none (the launch gave its waits up before the LM
      // head) flags the step, and the published id stays a valid one for the next step's lookup
      const uint32_t idx = key ? 0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull) : 0u;
      a.out_tok[0] = idx;
      const int i = a.step ? *a.step : 0;
      a.flags[i] = key ? __hip_atomic_load(a.amax_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 1;
      if (a.step) {
        a.gen[i] = idx;
        *a.step = i + 1;
      }
      *a.amax_key = 0ull;
      *a.amax_flag = 0;
    }
    if (a.pos_inc) *a.pos_inc += 1;
  }
  for (int w = tid; w <= CHAIN_MAX_PHASES * CHAIN2_MAX_SB; w += NT2)
    __hip_atomic_store(a.counters + (size_t)w * CHAIN2_CNT_STRIDE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

size_t chain_row_bytes(int dt, int K) {
  return dt == DT_Q4K ? (size_t)(K / QK_K) * Q4K_BYTES : q6r_row_bytes((size_t)(K / QK_K));
}

bool chain_phase_ok(int dt, int K, bool norm) {
  if (dt != DT_Q4K && dt != DT_Q6K_R) return false;
  if (K % QK_K != 0 || K <= 0) return false;
  const int npass = (K + 4095) / 4096;
  // a consumer's pass is c & (npass - 1): npass must be a power of two that divides NC
  if (npass > 4 || (npass & (npass - 1)) != 0 || NC % npass != 0) return false;
  if (norm && 2 * npass > 4) return false;  // x and norm weight columns share the staging region
  return true;
}

void launch_chain(const ChainArgs& a, hipStream_t st) {
  if (a.nphase < 1 || a.nphase > CHAIN_MAX_PHASES) fail(ST_OP, "chain: 1..6 phases");
  // one workgroup per CU: the workgroups wait on each other, so all of them must be resident
  static int ok = -1;
  if (ok < 0) {
    int per_cu = 0;
    ok = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, chain_kernel, NT, 0) == hipSuccess && per_cu >= 1;
  }
  if (!ok) fail(ST_OP, "chain: the kernel does not fit on a compute unit");
  hipLaunchKernelGGL(chain_kernel, dim3(num_cus()), dim3(NT), 0, st, a);
}

}  // namespace iek

namespace iek {

bool chain2_phase_ok(int dt, int K, bool norm, int rows_per_wg) {
  if (dt != DT_Q4K && dt != DT_Q6K_R) return false;
  if (K <= 0 || K % QK_K != 0 || K / QK_K > CHAIN2_MAX_SB) return false;
  if ((norm ? 2 * K : K) > CHAIN2_XS_FLOATS) return false;
  return rows_per_wg <= 16 * CHAIN2_MAX_TILES;
}

void launch_chain2(const ChainArgs& a, hipStream_t st) {
  if (a.nphase < 1 || a.nphase > CHAIN_MAX_PHASES) fail(ST_OP, "chain: 1..6 phases");
  // one workgroup per CU: the workgroups wait on each other, so all of them must be resident
  static int ok = -1;
  if (ok < 0) {
    int per_cu = 0;
    ok = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, chain2_kernel, NT2, 0) == hipSuccess && per_cu >= 1;
  }
  if (!ok) fail(ST_OP, "chain: the kernel does not fit on a compute unit");
  hipLaunchKernelGGL(chain2_kernel, dim3(num_cus()), dim3(NT2), 0, st, a);
}

}  // namespace iek
