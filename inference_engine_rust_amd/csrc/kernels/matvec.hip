// Decode matvec kernels and launchers: the streaming kernel (mv_stream), the generic fallback for
// any dtype and K, and the one-time regrouping of Q6_K / Q8_0 weights. Their device code is in
// mv_core.cuh (the decode chain, chain.hip, shares its dequantisation helpers).
#include <type_traits>

#include "mv_core.cuh"

namespace iek {

// One thread per (row, superblock, lane chunk): regroup a Q6_K tensor [K, N] (K % 256 == 0) into
// the DT_Q6K_R layout above. Runs once at model load.
__global__ void repack_q6k_kernel(const uint8_t* __restrict__ src, int nsb, int N, uint8_t* __restrict__ dst) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)N * nsb * 4) return;
  const int k = (int)(i & 3), j = (int)((i >> 2) % nsb);
  const size_t n = (i >> 2) / nsb;
  const uint8_t* blk = src + (n * nsb + j) * Q6K_BYTES;
  uint8_t* row = dst + n * q6r_row_bytes(nsb);
  const int h = k >> 1, j16 = k & 1;
  uint8_t* m = row + (size_t)j * 192 + 48 * k;
  for (int t = 0; t < 16; ++t) {
    m[t] = blk[64 * h + 16 * j16 + t];
    m[16 + t] = blk[64 * h + 32 + 16 * j16 + t];
    m[32 + t] = blk[128 + 32 * h + 16 * j16 + t];
  }
  uint8_t* sc = row + (size_t)nsb * 192 + 16 * j + 4 * k;
  for (int qd = 0; qd < 4; ++qd) sc[qd] = blk[192 + 8 * h + j16 + 2 * qd];
  if (k == 0) {
    uint8_t* d = row + (size_t)nsb * 208 + 2 * j;
    d[0] = blk[208];
    d[1] = blk[209];
  }
}

void launch_repack_q6k(const void* src, int K, int N, void* dst, hipStream_t st) {
  if (K % QK_K != 0) fail(ST_OP, "repack_q6k: K must be a multiple of 256");
  const int nsb = K / QK_K;
  IEK_HIP(hipMemsetAsync(dst, 0, (size_t)N * q6r_row_bytes(nsb), st));
  const size_t threads = (size_t)N * nsb * 4;
  hipLaunchKernelGGL(repack_q6k_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                     (const uint8_t*)src, nsb, N, (uint8_t*)dst);
}

// One thread per (row, block): regroup a Q8_0 tensor [K, N] (K % 32 == 0) into DT_Q8_0_R.
__global__ void repack_q80_kernel(const uint8_t* __restrict__ src, int nb, int N, uint8_t* __restrict__ dst) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)N * nb) return;
  const int b = (int)(i % nb);
  const size_t n = i / nb;
  const uint8_t* blk = src + i * Q8_0_BYTES;
  uint8_t* row = dst + n * q8r_row_bytes(nb);
  for (int t = 0; t < 32; ++t) row[32 * b + t] = blk[2 + t];
  row[(size_t)32 * nb + 2 * b] = blk[0];
  row[(size_t)32 * nb + 2 * b + 1] = blk[1];
}

void launch_repack_q80(const void* src, int K, int N, void* dst, hipStream_t st) {
  if (K % Q8_0_ELEMS != 0) fail(ST_OP, "repack_q80: K must be a multiple of 32");
  const int nb = K / Q8_0_ELEMS;
  IEK_HIP(hipMemsetAsync(dst, 0, (size_t)N * q8r_row_bytes(nb), st));
  const size_t threads = (size_t)N * nb;
  hipLaunchKernelGGL(repack_q80_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                     (const uint8_t*)src, nb, N, (uint8_t*)dst);
}

// The body reads the arguments in place from the kernarg segment (a reference to the by-value
// parameter would make a private copy, and the segment-selecting reads would keep it in scratch).
template <class Tr, int R, bool DUAL, bool MULTI, int NT, int XS = 0>
__global__ __launch_bounds__(NT) void mv_stream(MvArgs args) {
  extern __shared__ __align__(16) float lds[];
  (void)args;
  const MvArgs& a = *(const MvArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  // Every argument the prologue branches on or addresses with, loaded in one batch: read lazily,
  // each branch would wait for its own scalar load before issuing the next.
  asm volatile("" ::"s"(a.epi), "s"(a.nseg), "s"(a.K), "s"(a.seg_start[1]), "s"(a.seg_start[2]),
               "s"(a.seg_start[3]), "s"(a.n[0]), "s"(a.x), "s"(a.norm_w), "s"(a.resid), "s"(a.w[0]), "s"(a.w[1]),
               "s"(a.w[2]), "s"(a.pos), "s"(a.rope_cs), "s"(a.npairs), "s"(gridDim.x));
  // a scalar load: its wait is on the scalar counter, not behind vector loads
  typedef __attribute__((address_space(4))) const int* ConstInt;
  const int pos = a.epi == EPI_QKV ? *(ConstInt)a.pos : 0;
  mv_body<Tr, R, DUAL, MULTI, NT, XS>(a, lds, pos);
  if (a.pos_inc && blockIdx.x == 0 && threadIdx.x == 0) *a.pos_inc += 1;
}

// ---- generic path: any dtype, any K (blocks may straddle rows when K % block != 0) ----------
__global__ __launch_bounds__(256) void mv_generic(MvArgs a, int dt) {
  extern __shared__ __align__(16) float lds[];
  const Lds L = lds_layout(a, lds);
  const float* xs = L.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.x * 4 + wave;
  const int pos = a.epi == EPI_QKV ? *a.pos : 0;
  stage(a, L, pos);
  const int total = a.seg_start[a.nseg];
  unsigned long long run_key = 0;
  if (row < total) {  // no early return: argmax_flush below has a workgroup barrier
    const int s = seg_of(a, row);
    const int n = row - a.seg_start[s];
    const bool dual = a.epi == EPI_SWIGLU || a.epi == EPI_GEGLU;
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
    epilogue<1>(a, L, s, n, acc, accu, lane, pos, run_key);
  }
  if (a.epi == EPI_ARGMAX) argmax_flush(a, run_key);
  if (a.pos_inc && blockIdx.x == 0 && threadIdx.x == 0) *a.pos_inc += 1;
}

// ---------------------------------------------------------------------------------------------
int num_cus() {
  static int n = 0;
  if (n == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
  }
  return n;
}

// Workgroups per CU of the streaming matvec (counted in 256-thread workgroups' worth of waves):
// 3 measured best for the f32-staged traits at the C2 decode shapes (2: 430, 3: 445, 4: 445 tok/s).
constexpr int kMvPerCu = 3;

// Persistent grid: at most the workgroups that are resident at once, so no second wave of
// workgroups forms a tail; every wave then strides over the row groups. MULTI when some wave has
// more than one step.
template <class Tr, bool DUAL, int NT, int XS = 0>
static void launch_stream_x(const MvArgs& a, int groups, hipStream_t st) {
  constexpr int NW = NT / 64;
  const size_t lds = lds_bytes(a);
  if (lds > 160 * 1024) fail(ST_OP, "matvec: K too large for the LDS-staged input");
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, mv_stream<Tr, 2, DUAL, true, NT, XS>, NT, lds) !=
          hipSuccess ||
      per_cu <= 0)
    per_cu = 1;
  per_cu = std::min(per_cu, std::max(1, kMvPerCu * 256 / NT));
  const int blocks = std::max(1, std::min((groups + NW - 1) / NW, num_cus() * per_cu));
  const int waves = NW * blocks;
  const int nchunk = (a.K / QK_K) * Tr::CHUNKS, npass = (nchunk + WAVE - 1) / WAVE;
  const int max_steps = ((groups + waves - 1) / waves) * npass;
  if (max_steps > 1)
    hipLaunchKernelGGL((mv_stream<Tr, 2, DUAL, true, NT, XS>), dim3(blocks), dim3(NT), lds, st, a);
  else
    hipLaunchKernelGGL((mv_stream<Tr, 2, DUAL, false, NT, XS>), dim3(blocks), dim3(NT), lds, st, a);
}

// x staging: split (issued ahead of the weight loads) when x and its companions are
// float4-aligned, thread t owning float4 slots t + NT s of x for s < XS; 512-thread workgroups
// (one per CU worth of waves, x staged once per CU) for inputs over 8192 elements.
template <class Tr, bool DUAL>
static void launch_stream(const MvArgs& a, int groups, hipStream_t st) {
  auto al = [](const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (a.K % 4 == 0 && al(a.x) && al(a.norm_w) && al(a.pre_t) && al(a.pre_w) && al(a.pre_out)) {
    if (a.K <= 2048) return launch_stream_x<Tr, DUAL, 256, 2>(a, groups, st);
    if (a.K <= 4096) return launch_stream_x<Tr, DUAL, 256, 4>(a, groups, st);
    if (a.K <= 8192) return launch_stream_x<Tr, DUAL, 256, 8>(a, groups, st);
    if (a.K <= 16384) return launch_stream_x<Tr, DUAL, 512, 8>(a, groups, st);
  }
  launch_stream_x<Tr, DUAL, 256>(a, groups, st);
}

// Segment starts of a launch's row space; a gate/up pair streams over the gate rows with the up
// weight riding along as w[1].
void mv_finalize(MvArgs& a) {
  int total = 0;
  for (int i = 0; i < a.nseg; ++i) {
    a.seg_start[i] = total;
    total += a.n[i];
  }
  a.seg_start[a.nseg] = total;
  if (a.epi == EPI_SWIGLU || a.epi == EPI_GEGLU) {
    a.seg_start[1] = a.n[0];
    a.nseg = 1;
  }
}

void launch_mv(int dt, MvArgs a, hipStream_t st) {
  mv_finalize(a);
  const bool dual = a.epi == EPI_SWIGLU || a.epi == EPI_GEGLU;
  const int total = a.seg_start[a.nseg];
  bool fast = (dt == DT_Q4K || dt == DT_Q6K || dt == DT_Q6K_R || dt == DT_Q8_0_R) && a.K % QK_K == 0 &&
              (reinterpret_cast<uintptr_t>(a.x) % 16) == 0;
  for (int i = 0; i < (dual ? 2 : a.nseg); ++i) fast = fast && (reinterpret_cast<uintptr_t>(a.w[i]) % 16) == 0;
  // Two rows per wave: more rows per wave spill the prefetch registers.
  const int R = 2;
  for (int i = 0; i < a.nseg; ++i) fast = fast && a.n[i] % R == 0;
  if (fast) {
    const int groups = total / R;
#define IEK_L(TR) (dual ? launch_stream<TR, true>(a, groups, st) : launch_stream<TR, false>(a, groups, st))
    if (dt == DT_Q6K_R) IEK_L(Q6RTr);
    else if (dt == DT_Q8_0_R) IEK_L(Q8RTr);
    else if (dt == DT_Q4K) IEK_L(Q4Tr);
    else IEK_L(Q6Tr);
#undef IEK_L
    return;
  }
  const size_t lds_f = lds_bytes(a);
  if (lds_f > 160 * 1024) fail(ST_OP, "matvec: K too large for the LDS-staged input");
  if (a.epi == EPI_QKV) fail(ST_OP, "matvec: fused Q/K/V epilogue needs the aligned K-quant path");
  if (dt == DT_Q6K_R || dt == DT_Q8_0_R)
    fail(ST_OP, "matvec: a regrouped weight layout needs K % 256 == 0 and aligned inputs");
  hipLaunchKernelGGL(mv_generic, dim3((total + 3) / 4), dim3(256), lds_f, st, a, dt);
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
