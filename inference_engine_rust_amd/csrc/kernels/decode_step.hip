// Persistent decode step (Mistral/Llama family, fused path): every layer of one decode token in
// one launch (src/layers/block.rs:50-89 per layer, src/engine/runtime.rs:37-61 over layers).
//
// The per-launch path pays a fixed cost per kernel (launch, first-byte latency of the weight
// stream, tail) five times per layer. Here one grid of resident workgroups runs the phases
//   QKV matvec (+RMSNorm, RoPE, fp16 KV append) | attention slices (+merge) | O matvec (+residual)
//   | gate/up matvec (+RMSNorm, SwiGLU) | down matvec (+residual)
// back to back, separated by grid barriers. Before each barrier a wave issues the weight loads of
// its first step of the next phase (weights never depend on activations), so the barrier wait
// overlaps the head of the next weight stream instead of adding to it.
//
// Phase code is the same device code as the per-launch kernels (mv_core.cuh, attn_core.cuh) with
// the same row-to-wave mapping rules, so every output element is computed with the same
// arithmetic in the same order.
//
// Barrier (grid_sync below): two-level arrival counting and coherent accesses for the data that
// crosses workgroups, so no L2 write-back or invalidate is needed. The grid is exactly the number
// of workgroups resident at once, so every workgroup is running; each wait is still bounded and a
// timeout sets an error flag and ends the launch instead of hanging. The last workgroup to leave
// resets the counters.
#include <cstring>

#include "attn_core.cuh"
#include "mv_core.cuh"

namespace iek {

struct StepLayer {
  MvArgs qkv, o, dual, down;  // finalized launch arguments (segments filled in)
  const __half* kc;
  const __half* vc;
  float* q;    // this layer's rotated q (written by the QKV phase)
  float* att;  // attention output (input of the O phase)
  int window;
};

struct StepArgs {
  const StepLayer* layers;
  int n_layers, n_heads, n_kv, ctx, nsplit;
  float scale;
  float* part;
  int* counters;
  const int* pos;
  int* pos_inc;
  unsigned* bar;  // barrier counters (step_bar_words() words): zero at launch, zero again after it
  int* err;       // 1 when a barrier wait ran out
  unsigned long long* trace;  // optional: workgroup 0's clock (100 MHz) at every phase end / barrier exit
};

constexpr unsigned STEP_SPIN_LIMIT = 1u << 20;
// Barrier counter words (each on its own 256-byte line): global arrivals, exits, 8 group counters.
constexpr int BAR_STRIDE = 64, BAR_GLOBAL = 0, BAR_EXIT = BAR_STRIDE, BAR_GROUP = 2 * BAR_STRIDE;
constexpr int BAR_WORDS = 10 * BAR_STRIDE;

// Grid barrier with the next phase's weight prefetch in flight across it, in two levels: the
// workgroups of one group (blockIdx % 8, which is also the XCD the dispatcher places them on)
// count on their own counter, and the last arrival of a group bumps the global counter that every
// workgroup polls. One counter for all workgroups serialises every arrival on one address
// (measured ~9 us per barrier at 512 workgroups, against ~3 us in two levels).
// No cache maintenance: every piece of data one workgroup writes and another reads in this launch
// goes through coherent (agent-scope, L2-bypassing) loads and stores, so each wave only waits for
// its own stores to complete before its workgroup arrives. Waves 1-3 issue their prefetch before
// the workgroup barrier; wave 0 after thread 0 has arrived, then thread 0 polls.
template <class F>
IEK_DEV bool grid_sync(unsigned* bar, unsigned phase, int* err, int* ok_s, F&& prefetch) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  __builtin_amdgcn_s_waitcnt(0);
  if (wave != 0) prefetch();
  __syncthreads();
  if (wave == 0) {
    if (threadIdx.x == 0) {
      const unsigned g = blockIdx.x & 7, members = (gridDim.x - g + 7) / 8;
      const unsigned old = __hip_atomic_fetch_add(bar + BAR_GROUP + BAR_STRIDE * g, 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
      if (old + 1 == phase * members)
        __hip_atomic_fetch_add(bar + BAR_GLOBAL, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("" ::: "memory");
    prefetch();
    asm volatile("" ::: "memory");
    if (threadIdx.x == 0) {
      const unsigned target = phase * 8u;
      unsigned it = 0;
      int good = 1;
      while (__hip_atomic_load(bar + BAR_GLOBAL, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
        __builtin_amdgcn_s_sleep(1);
        if (++it > STEP_SPIN_LIMIT) {
          good = 0;
          break;
        }
      }
      if (!good) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *ok_s = good;
    }
  }
  __syncthreads();
  return *ok_s != 0;
}

struct NoPrefetch {
  IEK_DEV void operator()() const {}
};

// Records workgroup 0's real-time clock into the optional trace (a profiling aid: per-phase
// durations of the step as seen by one workgroup).
IEK_DEV void step_mark(unsigned long long* trace, int& k) {
  if (trace && blockIdx.x == 0 && threadIdx.x == 0) trace[k] = __builtin_amdgcn_s_memrealtime();
  ++k;
}

template <int HD>
__global__ __launch_bounds__(256, 2) void decode_step_kernel(StepArgs args) {
  extern __shared__ __align__(16) float lds[];
  __shared__ int ok_s;
  (void)args;
  const StepArgs& S = *(const StepArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  // The per-layer arguments are read through the constant address space so that every read is a
  // scalar load: a vector load would share the counter of the weight stream and its wait would
  // drain the prefetch.
  typedef __attribute__((address_space(4))) const StepLayer* ConstLayers;
  const ConstLayers layers = (ConstLayers)S.layers;
  const int pos = __builtin_amdgcn_readfirstlane(*S.pos);
  const unsigned nwg = gridDim.x;
  unsigned phase = 0;
  int mk = 0;
  step_mark(S.trace, mk);
  typename Q4I8Tr::template Buf<2> pq;
  typename Q4I8Tr::template Buf<4> pd;
  typename Q6RTr::template Buf<2> pw;
  mv_prefetch<Q4I8Tr, 2, false>(((const StepLayer*)&layers[0])->qkv, pq);
  for (int l = 0; l < S.n_layers; ++l) {
    const StepLayer& L = *(const StepLayer*)&layers[l];
    mv_body<Q4I8Tr, 2, false, true>(L.qkv, lds, pos, pq, true);
    step_mark(S.trace, mk);
    if (!grid_sync(S.bar, ++phase, S.err, &ok_s, NoPrefetch{})) return;
    step_mark(S.trace, mk);
    const int spc = attn_slices_per_chunk(S.nsplit * SPLIT, L.window), nchunk = (S.nsplit + spc - 1) / spc;
    const int items = S.n_kv * nchunk;
    for (int it = blockIdx.x; it < items; it += nwg) {
      attn_chunk_f16<HD, true>(L.q, L.kc, L.vc, S.part, L.att, S.counters, S.n_heads, S.n_kv, S.ctx, nullptr, pos + 1,
                               L.window, S.scale, nchunk, it % S.n_kv, it / S.n_kv, spc, reinterpret_cast<char*>(lds));
      __syncthreads();
    }
    step_mark(S.trace, mk);
    if (!grid_sync(S.bar, ++phase, S.err, &ok_s, [&] { mv_prefetch<Q4I8Tr, 2, false>(L.o, pq); })) return;
    step_mark(S.trace, mk);
    mv_body<Q4I8Tr, 2, false, true>(L.o, lds, pos, pq, true);
    step_mark(S.trace, mk);
    if (!grid_sync(S.bar, ++phase, S.err, &ok_s, [&] { mv_prefetch<Q4I8Tr, 2, true>(L.dual, pd); })) return;
    step_mark(S.trace, mk);
    mv_body<Q4I8Tr, 2, true, true>(L.dual, lds, pos, pd, true);
    step_mark(S.trace, mk);
    if (!grid_sync(S.bar, ++phase, S.err, &ok_s, [&] { mv_prefetch<Q6RTr, 2, false>(L.down, pw); })) return;
    step_mark(S.trace, mk);
    mv_body<Q6RTr, 2, false, true>(L.down, lds, pos, pw, true);
    step_mark(S.trace, mk);
    if (l + 1 < S.n_layers) {
      const StepLayer& N = *(const StepLayer*)&layers[l + 1];
      if (!grid_sync(S.bar, ++phase, S.err, &ok_s, [&] { mv_prefetch<Q4I8Tr, 2, false>(N.qkv, pq); })) return;
    }
    step_mark(S.trace, mk);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    if (blockIdx.x == 0 && S.pos_inc) *S.pos_inc += 1;
    const unsigned old = __hip_atomic_fetch_add(S.bar + BAR_EXIT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == nwg - 1)
      for (int w = 0; w < BAR_WORDS; w += BAR_STRIDE)
        __hip_atomic_store(S.bar + w, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---- host side --------------------------------------------------------------------------------

static int step_cus() {
  static int n = 0;
  if (n == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
  }
  return n;
}

template <int HD>
static void step_launch(const StepArgs& a, size_t lds, hipStream_t st) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_step_kernel<HD>, 256, lds) != hipSuccess ||
      per_cu <= 0)
    fail(ST_OP, "decode step: the kernel does not fit on a compute unit");
  per_cu = std::min(per_cu, 2);
  hipLaunchKernelGGL(decode_step_kernel<HD>, dim3(step_cus() * per_cu), dim3(256), lds, st, a);
}

void launch_decode_step(const void* layers, int n_layers, int n_heads, int n_kv, int head_dim, int ctx, float scale,
                        float* part, int* counters, const int* pos, int* pos_inc, unsigned* bar, int* err,
                        size_t lds_bytes, unsigned long long* trace, hipStream_t st) {
  StepArgs a{};
  a.trace = trace;
  a.layers = static_cast<const StepLayer*>(layers);
  a.n_layers = n_layers;
  a.n_heads = n_heads;
  a.n_kv = n_kv;
  a.ctx = ctx;
  a.nsplit = (ctx + SPLIT - 1) / SPLIT;
  a.scale = scale;
  a.part = part;
  a.counters = counters;
  a.pos = pos;
  a.pos_inc = pos_inc;
  a.bar = bar;
  a.err = err;
  if (n_kv <= 0 || n_heads % n_kv != 0 || n_heads / n_kv > 8)
    fail(ST_OP, "decode step: GQA group must divide the heads and be at most 8");
  switch (head_dim) {
    case 64: {
      const size_t l = std::max(lds_bytes, AttnSmem<64>::BYTES);
      step_launch<64>(a, l, st);
      break;
    }
    case 128: {
      const size_t l = std::max(lds_bytes, AttnSmem<128>::BYTES);
      step_launch<128>(a, l, st);
      break;
    }
    default:
      fail(ST_OP, "decode step: head_dim must be 64 or 128");
  }
}

size_t step_layer_bytes() { return sizeof(StepLayer); }
int step_bar_words() { return BAR_WORDS; }

// Host image of one StepLayer (the caller copies an array of these to the device).
void step_layer_pack(void* dst, const MvArgs& qkv, const MvArgs& o, const MvArgs& dual, const MvArgs& down,
                     const __half* kc, const __half* vc, float* q, float* att, int window) {
  StepLayer L;
  L.qkv = qkv;
  L.o = o;
  L.dual = dual;
  L.down = down;
  L.kc = kc;
  L.vc = vc;
  L.q = q;
  L.att = att;
  L.window = window;
  std::memcpy(dst, &L, sizeof(L));
}

}  // namespace iek
