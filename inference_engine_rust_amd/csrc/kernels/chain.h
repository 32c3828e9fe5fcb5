// Launch description of the decode chain kernel (kernels/chain.hip): a run of dependent decode
// matvec phases in one persistent launch. Shared by the kernel and the host engine.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace iek {

enum ChainEpi : int {
  CE_STORE = 0,   // out[seg][row] = dot
  CE_RESID = 1,   // out[row] = resid[row] + dot (one segment)
  CE_SWIGLU = 2,  // seg 0 = gate, seg 1 = up: out[row] = silu(gate.x) * (up.x) into seg[0].out
  CE_QKV = 3,     // segments q, k, v: RoPE on q and k pairs, q -> seg[0].out, k / v -> the f32 cache at pos
  CE_ARGMAX = 4,  // logits -> seg[0].out (optional soft cap), packed (value, first index) key maximum
};

enum ChainX : int {
  CX_F32 = 0,        // x is an f32 vector in device memory
  CX_EMBED_Q4K = 1,  // x is row *tok of a Q4_K embedding table, dequantised in the prologue
};

struct ChainSeg {
  const uint8_t* w;  // weight rows: native Q4_K blocks or the regrouped Q6_K layout
  float* out;
  int n;  // rows
  int pad;
};

// One phase: every row of its segments dotted with the phase input x. Rows go in pairs (a RoPE
// pair, a gate/up pair, or two consecutive rows); the pairs are split evenly over the workgroups.
struct ChainPhase {
  ChainSeg seg[3];
  int nseg, dt, K, npass;  // dt: DT_Q4K or DT_Q6K_R (all segments); npass = ceil(K / 4096)
  int epi, units, x_mode, wait_prev;  // units = row pairs; wait_prev: x is the previous phase's output
  const float* x;
  const float* norm_w;  // fused RMSNorm of x, or null
  float eps;
  int emb_rows;  // CX_EMBED_Q4K: rows of the embedding table
  const float* resid;  // CE_RESID
  // CE_QKV
  const float* rope_cs;  // [ctx][npairs][2]
  int npairs, head_dim, ctx;
  int role0;  // role of seg[0]: 0 = Q (segments Q, K, V), 2 = V (a V-only phase, when V's dtype differs)
  float* kc;  // f32 KV cache [n_kv][ctx][head_dim]
  float* vc;
  // CX_EMBED_Q4K
  const uint8_t* emb;
  float* emb_out;  // workgroup 0 also writes the dequantised row here
  // CE_ARGMAX
  float softcap;  // <= 0: none
  int pad2;
  // Tiled chain (launch_chain2): the phase whose output is this phase's x (-1: x was written
  // before the launch), whether a later phase reads this phase's output (its workgroups then
  // arrive on the per-superblock counters), and per superblock of x the number of workgroups that
  // write part of it (the arrivals that make it ready).
  int x_src, arrive;
  int expect[64];
};

constexpr int CHAIN_MAX_PHASES = 6;
// counter words: per phase 8 group counters + 1 global, then the exit counter; 64 words apart
constexpr int CHAIN_COUNTER_WORDS = (CHAIN_MAX_PHASES * 9 + 1) * 64;

struct ChainArgs {
  const ChainPhase* phases;  // device array
  int nphase;
  int finish_argmax;  // the last workgroup publishes the argmax token (CE_ARGMAX present)
  const int* pos;
  const uint32_t* tok;   // token of CX_EMBED_Q4K
  unsigned* counters;    // CHAIN_COUNTER_WORDS, zero at launch; zero again when the launch ends
  int* err;              // [0]: set when a bounded wait runs out (the launch then ends early);
                         // [1]: the bounded waits' iteration limit (0: the default, ~0.1-0.2 s)
  int* pos_inc;          // when set, the last workgroup adds 1 at the end
  // CE_ARGMAX and its finish (as launch_argmax_finish)
  unsigned long long* amax_key;
  int* amax_flag;
  uint32_t* out_tok;
  uint32_t* gen;
  int* flags;
  int* step;
};

// Whether the chain kernel takes a phase of this dtype and width (host check).
bool chain_phase_ok(int dt, int K, bool norm);
void launch_chain(const ChainArgs& a, hipStream_t st);
size_t chain_row_bytes(int dt, int K);

// Tiled chain (the same phases, ChainArgs and epilogues): each workgroup's rows of a phase are
// 16-row tiles, a consumer's items are (tile, superblock) pairs, and each superblock of x becomes
// ready on its own counter (ChainPhase::x_src / arrive / expect). Counter words: per phase and
// superblock one word, CHAIN2_CNT_STRIDE words apart, then the exit counter.
constexpr int CHAIN2_MAX_SB = 64;     // superblocks of x per phase (K <= 16384)
constexpr int CHAIN2_MAX_TILES = 8;   // 16-row tiles per workgroup and phase
constexpr int CHAIN2_CNT_STRIDE = 16;
constexpr int CHAIN2_COUNTER_WORDS = (CHAIN_MAX_PHASES * CHAIN2_MAX_SB + 1) * CHAIN2_CNT_STRIDE;
// The x staging region holds K floats (K + K with a fused norm's weights).
constexpr int CHAIN2_XS_FLOATS = 14336;
bool chain2_phase_ok(int dt, int K, bool norm, int rows_per_wg);
void launch_chain2(const ChainArgs& a, hipStream_t st);

}  // namespace iek
