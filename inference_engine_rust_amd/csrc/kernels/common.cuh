// Device helpers shared by the CDNA4 (gfx950) kernels: wave64 reductions, block dequant
// primitives matching the reference's arithmetic, and the ggml block geometry.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../iek_internal.h"

#define IEK_DEV __device__ __forceinline__

namespace iek {

constexpr int WAVE = 64;
constexpr int QK_K = 256;
constexpr int Q4K_BYTES = 144;
constexpr int Q6K_BYTES = 210;
constexpr int Q8_0_ELEMS = 32;
constexpr int Q8_0_BYTES = 34;
// Largest magnitude an fp16 (hi, lo) pair of an f32 holds (the largest finite fp16): prefill GEMM
// and attention inputs beyond it are flagged and the prefill runs on f32 activations instead.
constexpr float F16_PAIR_MAX = 65504.f;

// IEEE half bits -> f32. Exact for every non-NaN input (subnormals included), which is what the
// reference's hand-rolled f16_to_f32 computes (src/ops/quant/utils.rs:2-32).
IEK_DEV float half_bits_to_float(uint32_t bits16) {
  return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xFFFFu)));
}

// Cross-lane steps on DPP (register-to-register, no LDS round trip). update_dpp returns `old` in
// the rows the row mask leaves out.
template <int CTRL, int ROW_MASK = 0xF>
IEK_DEV float dpp_f(float old, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                                               CTRL, ROW_MASK, 0xF, false));
}
constexpr int DPP_XOR1 = 0xB1;         // quad_perm [1, 0, 3, 2]
constexpr int DPP_XOR2 = 0x4E;         // quad_perm [2, 3, 0, 1]
constexpr int DPP_HALF_MIRROR = 0x141;  // lane i <- 7 - i within each 8
constexpr int DPP_MIRROR = 0x140;       // lane i <- 15 - i within each 16
constexpr int DPP_BCAST15 = 0x142;      // lane 15 of row r -> row r + 1
constexpr int DPP_BCAST31 = 0x143;      // lane 31 -> rows 2 and 3

// Sum / max over each 16-lane row, the result in every lane of the row.
IEK_DEV float row16_sum(float v) {
  v += dpp_f<DPP_XOR1>(0.f, v);
  v += dpp_f<DPP_XOR2>(0.f, v);
  v += dpp_f<DPP_HALF_MIRROR>(0.f, v);
  return v + dpp_f<DPP_MIRROR>(0.f, v);
}
IEK_DEV float row16_max(float v) {
  v = fmaxf(v, dpp_f<DPP_XOR1>(-INFINITY, v));
  v = fmaxf(v, dpp_f<DPP_XOR2>(-INFINITY, v));
  v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(-INFINITY, v));
  return fmaxf(v, dpp_f<DPP_MIRROR>(-INFINITY, v));
}

// Sum / max over the wave, the result in every lane: the 16-lane rows, then rows 0+1 into row 1
// and (0+1)+(2+3) into row 3, whose last lane is broadcast.
IEK_DEV float wave_sum(float v) {
  v = row16_sum(v);
  v += dpp_f<DPP_BCAST15, 0xA>(0.f, v);
  v += dpp_f<DPP_BCAST31, 0xC>(0.f, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

IEK_DEV float wave_max(float v) {
  v = row16_max(v);
  v = fmaxf(v, dpp_f<DPP_BCAST15, 0xA>(-INFINITY, v));
  v = fmaxf(v, dpp_f<DPP_BCAST31, 0xC>(-INFINITY, v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Loads and stores coherent across the XCDs' L2 caches without cache maintenance (agent-scope
// relaxed atomics: sc1 accesses). Used for data that one workgroup writes and another reads within
// the same launch (the decode chain's phases, the decode attention's partials under its COH
// flag); elsewhere kernel boundaries order the data and plain accesses suffice.
IEK_DEV float ld_coh(const float* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
IEK_DEV float4 ld_coh4(const float4* p) {
  const unsigned long long* q = reinterpret_cast<const unsigned long long*>(p);
  const unsigned long long a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned long long b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float4(__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)), __uint_as_float((uint32_t)b),
                     __uint_as_float((uint32_t)(b >> 32)));
}
IEK_DEV void st_coh(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
IEK_DEV void st_coh_h(__half* p, __half v) {
  __hip_atomic_store(reinterpret_cast<unsigned short*>(p), __half_as_ushort(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
template <bool COH>
IEK_DEV float ld_f(const float* p) {
  if constexpr (COH) return ld_coh(p);
  else return *p;
}
template <bool COH>
IEK_DEV float4 ld_f4(const float4* p) {
  if constexpr (COH) return ld_coh4(p);
  else return *p;
}
template <bool COH>
IEK_DEV void st_f(float* p, float v) {
  if constexpr (COH) st_coh(p, v);
  else *p = v;
}
template <bool COH>
IEK_DEV void st_h(__half* p, __half v) {
  if constexpr (COH) st_coh_h(p, v);
  else *p = v;
}

// gelu_tanh (src/ops/gelu.rs:5-11): 0.5 x (1 + tanh(k (x + 0.044715 x^3))) with
// k = FRAC_2_SQRT_PI * FRAC_1_SQRT_2 rounded to f32, each step rounded separately.
IEK_DEV float gelu_tanh_dev(float x) {
#pragma clang fp contract(off)
  const float k = 1.12837916709551257390f * 0.707106781186547524401f;
  float x3 = x * x * x;
  return 0.5f * x * (1.0f + tanhf(k * (x + 0.044715f * x3)));
}

IEK_DEV uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xFFu; }

// get_scale_min_k4 over the 12 packed scale bytes held as three dwords
// (src/ops/quant/quant_k_handler.rs:138-155).
IEK_DEV void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2, float* sc, float* m) {
  if (j < 4) {
    *sc = (float)(byte_of(s0, j) & 63u);
    *m = (float)(byte_of(s1, j) & 63u);
  } else {
    uint32_t lo = byte_of(s2, j - 4);
    *sc = (float)((lo & 0xFu) | ((byte_of(s0, j - 4) >> 6) << 4));
    *m = (float)((lo >> 4) | ((byte_of(s1, j - 4) >> 6) << 4));
  }
}

// One dequantised element of a Q4_K block: (d*sc)*q - dmin*m with the reference's q == 0 -> 0
// convention (quant_k_handler.rs:6-8, :38-82). Every product is exact in f32 (at most 21
// significant bits), so the single f32 rounding of the subtraction equals the reference's
// f64-then-f32 result.
IEK_DEV float q4k_value(float d, float dmin, float sc, float m, uint32_t q) {
#pragma clang fp contract(off)
  float ds = d * sc;
  float dq = q == 0 ? 0.0f : ds * (float)q;
  return dq - dmin * m;
}

// Unaligned little-endian u16 from a byte pointer (Q6_K / Q8_0 blocks are only 2-byte aligned).
IEK_DEV uint32_t load_u16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

// Single element `o` (0..255) of a Q4_K block.
IEK_DEV float q4k_elem(const uint8_t* blk, int o) {
  float d = half_bits_to_float(load_u16(blk)), dmin = half_bits_to_float(load_u16(blk + 2));
  const uint8_t* s = blk + 4;
  int g = o >> 6, r = o & 63, is = 2 * g + (r >= 32 ? 1 : 0), l = r & 31;
  uint32_t byte = blk[16 + 32 * g + l];
  uint32_t q = r < 32 ? (byte & 0xFu) : (byte >> 4);
  float sc, m;
  if (is < 4) {
    sc = (float)(s[is] & 63);
    m = (float)(s[is + 4] & 63);
  } else {
    sc = (float)((s[is + 4] & 0xF) | ((s[is - 4] >> 6) << 4));
    m = (float)((s[is + 4] >> 4) | ((s[is] >> 6) << 4));
  }
  return q4k_value(d, dmin, sc, m, q);
}

// Single element of a Q6_K block (quant_k_handler.rs:85-135): y = (d*s)*q, int8 s, q in [-32,31].
IEK_DEV float q6k_elem(const uint8_t* blk, int o) {
  float d = half_bits_to_float(load_u16(blk + 208));
  int h = o >> 7, r = o & 127, quarter = r >> 5, l = r & 31;
  uint32_t qlb = blk[64 * h + l + ((quarter & 1) ? 32 : 0)];
  uint32_t nib = quarter < 2 ? (qlb & 0xFu) : (qlb >> 4);
  uint32_t hb = (blk[128 + 32 * h + l] >> (2 * quarter)) & 3u;
  int q = (int)(nib | (hb << 4)) - 32;
  float s = (float)(int8_t)blk[192 + 8 * h + (l >> 4) + 2 * quarter];
  float ds = d * s;
  return q == 0 ? 0.0f : ds * (float)q;
}

// Single element of a Q8_0 block (quant_k_handler.rs:21-35).
IEK_DEV float q80_elem(const uint8_t* blk, int o) {
  float d = half_bits_to_float(load_u16(blk));
  return d * (float)(int8_t)blk[2 + o];
}

// Element at flat index `f` of a tensor stored as consecutive blocks of type `dt`.
IEK_DEV float flat_elem(int dt, const uint8_t* base, size_t f) {
  switch (dt) {
    case DT_Q4K: return q4k_elem(base + (f / QK_K) * Q4K_BYTES, (int)(f % QK_K));
    case DT_Q6K: return q6k_elem(base + (f / QK_K) * Q6K_BYTES, (int)(f % QK_K));
    case DT_Q8_0: return q80_elem(base + (f / Q8_0_ELEMS) * Q8_0_BYTES, (int)(f % Q8_0_ELEMS));
    default: return reinterpret_cast<const float*>(base)[f];
  }
}

}  // namespace iek
