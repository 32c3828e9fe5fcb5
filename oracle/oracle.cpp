// TEST INFRASTRUCTURE ONLY — CPU oracle for parity tests and the CPU baseline timing.
// Restates the reference's CPU path function by function; each function cites the reference
// file:line it follows (paths relative to the reference repository root).
// Never linked by the product library. See oracle_core.h for the arithmetic rules.
#include <immintrin.h>
#include "oracle_core.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <thread>

namespace orc {

static thread_local std::string g_last_error;

[[noreturn]] static void fail(int code, const std::string& m) { throw Error{code, m}; }

// ---------------------------------------------------------------------------------------------
// Thread helpers. parallel_for splits [0, n) dynamically across `threads` workers
// (Rayon-like work distribution; results never depend on the split).
// ---------------------------------------------------------------------------------------------
static void parallel_for(size_t n, int threads, const std::function<void(size_t)>& body) {
  if (n == 0) return;
  if (threads <= 1 || n == 1) {
    for (size_t i = 0; i < n; ++i) body(i);
    return;
  }
  std::atomic<size_t> next{0};
  std::atomic<bool> failed{false};
  Error first{0, ""};
  auto worker = [&]() {
    for (;;) {
      size_t i = next.fetch_add(1);
      if (i >= n || failed.load()) return;
      try {
        body(i);
      } catch (const Error& e) {
        bool expected = false;
        if (failed.compare_exchange_strong(expected, true)) first = e;
        return;
      }
    }
  };
  int t = (int)std::min<size_t>((size_t)threads, n);
  std::vector<std::thread> pool;
  for (int i = 1; i < t; ++i) pool.emplace_back(worker);
  worker();
  for (auto& th : pool) th.join();
  if (failed.load()) throw first;
}

// ---------------------------------------------------------------------------------------------
// Quant primitives — src/ops/quant/utils.rs:2-32, src/ops/quant/quant_k_handler.rs
// ---------------------------------------------------------------------------------------------

// f16_to_f32 (src/ops/quant/utils.rs:2-32): hand-rolled IEEE half decode; any NaN -> canonical NaN.
float f16_to_f32(uint16_t bits) {
  uint16_t sign = (bits >> 15) & 1, exponent = (bits >> 10) & 0x1F, mantissa = bits & 0x3FF;
  if (exponent == 0) {
    if (mantissa == 0) return sign == 0 ? 0.0f : -0.0f;
    // (mantissa as f32) / 1024.0 * 2^-14 — two exact f32 steps.
    float value = ((float)mantissa / 1024.0f) * 6.103515625e-05f;
    return sign == 0 ? value : -value;
  } else if (exponent == 0x1F) {
    if (mantissa == 0) return sign == 0 ? INFINITY : -INFINITY;
    return NAN;
  }
  int e = (int)exponent - 15;
  float mant = 1.0f + (float)mantissa / 1024.0f;
  float value = mant * ldexpf(1.0f, e);  // 2.0_f32.powi(exp) is exact for |exp| <= 15
  return sign == 0 ? value : -value;
}

// scale_times_quant_f64 (quant_k_handler.rs:6-8): 0 * inf = 0 convention.
static inline double scale_times_quant(double scale, double q) { return q == 0.0 ? 0.0 : scale * q; }

// extract_scale_min_k4 (quant_k_handler.rs:138-155)
void extract_scale_min_k4(size_t j, const uint8_t* scales, uint8_t* sc, uint8_t* m) {
  if (j < 4) {
    *sc = scales[j] & 0x3F;
    *m = scales[j + 4] & 0x3F;
  } else {
    uint8_t low = scales[j + 4];
    uint8_t scale_low = low & 0x0F, min_low = (low >> 4) & 0x0F;
    uint8_t scale_high = (scales[j - 4] >> 6) & 0x03, min_high = (scales[j] >> 6) & 0x03;
    *sc = (uint8_t)(scale_low | (scale_high << 4));
    *m = (uint8_t)(min_low | (min_high << 4));
  }
}

static const size_t QK = 256, Q4K_BYTES = 144, Q6K_BYTES = 210, Q8_0_ELEMS = 32, Q8_0_BYTES = 34;

// dequantize_q8_0_block (quant_k_handler.rs:21-35): f32 `d * (i8)q`.
void dequant_q8_0(const uint8_t* b, float* out) {
  float d = f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
  for (size_t i = 0; i < 32; ++i) out[i] = d * (float)(int8_t)b[2 + i];
}

// dequantize_q4k_block (quant_k_handler.rs:38-82): f64 `(d*sc)*q - dmin*m`, one f32 rounding.
void dequant_q4k(const uint8_t* b, float* out) {
  double d = (double)f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
  double dmin = (double)f16_to_f32((uint16_t)(b[2] | (b[3] << 8)));
  const uint8_t* scales = b + 4;
  const uint8_t* q = b + 16;
  size_t y = 0, qp = 0;
  for (int is = 0; is < 8; is += 2) {
    uint8_t sc0, m0, sc1, m1;
    extract_scale_min_k4((size_t)is, scales, &sc0, &m0);
    extract_scale_min_k4((size_t)is + 1, scales, &sc1, &m1);
    for (size_t l = 0; l < 32; ++l) {
      double v = (double)(q[qp + l] & 0xF);
      double dq = scale_times_quant(d * (double)sc0, v);
      double mq = dmin * (double)m0;
      out[y + l] = (float)(dq - mq);
    }
    for (size_t l = 0; l < 32; ++l) {
      double v = (double)((q[qp + l] >> 4) & 0x0F);
      double dq = scale_times_quant(d * (double)sc1, v);
      double mq = dmin * (double)m1;
      out[y + 32 + l] = (float)(dq - mq);
    }
    y += 64;
    qp += 32;
  }
}

// dequantize_q6k_block (quant_k_handler.rs:85-135): int8 scales, q in [-32, 31].
void dequant_q6k(const uint8_t* b, float* out) {
  const uint8_t* ql = b;
  const uint8_t* qh = b + 128;
  const uint8_t* scales = b + 192;
  double d = (double)f16_to_f32((uint16_t)(b[208] | (b[209] << 8)));
  for (size_t half = 0; half < 2; ++half) {
    size_t yb = half * 128, lo = half * 64, ho = half * 32, so = half * 8;
    const uint8_t* s = scales + so;
    for (size_t l = 0; l < 32; ++l) {
      size_t is = l / 16;
      int q1 = ((ql[lo + l] & 0xF) | ((qh[ho + l] & 3) << 4)) - 32;
      int q2 = ((ql[lo + l + 32] & 0xF) | (((qh[ho + l] >> 2) & 3) << 4)) - 32;
      int q3 = ((ql[lo + l] >> 4) | (((qh[ho + l] >> 4) & 3) << 4)) - 32;
      int q4 = ((ql[lo + l + 32] >> 4) | (((qh[ho + l] >> 6) & 3) << 4)) - 32;
      double s0 = (double)(int8_t)s[is], s2 = (double)(int8_t)s[is + 2];
      double s4 = (double)(int8_t)s[is + 4], s6 = (double)(int8_t)s[is + 6];
      out[yb + l] = (float)scale_times_quant(d * s0, (double)q1);
      out[yb + l + 32] = (float)scale_times_quant(d * s2, (double)q2);
      out[yb + l + 64] = (float)scale_times_quant(d * s4, (double)q3);
      out[yb + l + 96] = (float)scale_times_quant(d * s6, (double)q4);
    }
  }
}

static inline size_t block_elems(int t) { return t == T_Q8_0 ? Q8_0_ELEMS : QK; }
static inline size_t block_bytes(int t) {
  return t == T_Q4K ? Q4K_BYTES : t == T_Q6K ? Q6K_BYTES : Q8_0_BYTES;
}
static inline void dequant_block(int t, const uint8_t* b, float* out) {
  if (t == T_Q4K) dequant_q4k(b, out);
  else if (t == T_Q6K) dequant_q6k(b, out);
  else dequant_q8_0(b, out);
}

// Expected raw byte length of a tensor (src/model_loader/tensor_loader.rs:69-88).
static size_t expected_byte_len(int t, size_t nelem) {
  if (t == T_F32) return nelem * 4;
  size_t be = block_elems(t);
  return ((nelem + be - 1) / be) * block_bytes(t);
}

// ---------------------------------------------------------------------------------------------
// matmul (src/ops/matmul.rs:18-415)
// out[row, col] = sum_kk a[row, kk] * W(kk, col), W(kk, col) at flat kk + col*K (ggml layout),
// sequential f32 `acc += a * w` in kk order, zero activations skipped.
// ---------------------------------------------------------------------------------------------
static const size_t PARALLEL_MATMUL_MIN_OPS = 64 * 1024;  // matmul.rs:16

// Reference row kernel for quantised W (matmul.rs:176-204): one cached decoded block.
static void q_row_kernel(int t, const float* a, size_t k, const uint8_t* w, size_t n, float* out_row,
                         size_t col0, size_t col1) {
  size_t be = block_elems(t), bb = block_bytes(t);
  float decoded[256];
  size_t cur = (size_t)-1;
  for (size_t col = col0; col < col1; ++col) {
    float acc = 0.0f;
    for (size_t kk = 0; kk < k; ++kk) {
      float av = a[kk];
      if (av == 0.0f) continue;
      size_t wi = kk + col * k;
      size_t bi = wi / be;
      if (bi != cur) {
        dequant_block(t, w + bi * bb, decoded);
        cur = bi;
      }
      acc += av * decoded[wi % be];
    }
    out_row[col] = acc;
  }
  (void)n;
}

static void f32_row_kernel(const float* a, size_t k, const float* w, float* out_row, size_t col0,
                           size_t col1) {
  for (size_t col = col0; col < col1; ++col) {
    float acc = 0.0f;
    for (size_t kk = 0; kk < k; ++kk) acc += a[kk] * w[kk + col * k];
    out_row[col] = acc;
  }
}

// Register-blocked GEMM over a k-major weight copy Wt[kk*N + col]. Each output element is still
// `acc += a*w` in kk order with separate multiply and add, so every element is bit-identical to
// the reference's scalar loop. Skipping a == 0 is only observable for non-finite weights; the
// caller routes those to the exact skip loop. One work item is one NR-column panel of W over every
// row of `a`: the panel (k x NR floats) comes from memory once and is reused from cache by each
// MR-row block.
static void gemm_kmajor(const float* a, size_t m, size_t k, const float* wt, size_t n, float* out,
                        int threads, bool reassoc = false) {
  if (reassoc) {
    // two halves of K, each summed in order, added at the end
    const size_t kh = k / 2;
    std::vector<float> a0(m * kh), a1(m * (k - kh)), o1(m * n);
    for (size_t i = 0; i < m; ++i) {
      memcpy(&a0[i * kh], a + i * k, kh * 4);
      memcpy(&a1[i * (k - kh)], a + i * k + kh, (k - kh) * 4);
    }
    gemm_kmajor(a0.data(), m, kh, wt, n, out, threads);
    gemm_kmajor(a1.data(), m, k - kh, wt + kh * n, n, o1.data(), threads);
    for (size_t i = 0; i < m * n; ++i) out[i] = out[i] + o1[i];
    return;
  }
  constexpr size_t MR = 6, NR = 16;
  const size_t nblocks = (n + NR - 1) / NR;
  parallel_for(nblocks, threads, [&](size_t nb) {
    const size_t n0 = nb * NR, nr = std::min(NR, n - n0);
    for (size_t m0 = 0; m0 < m; m0 += MR) {
      const size_t mr = std::min(MR, m - m0);
      float acc[MR][NR];
      for (size_t i = 0; i < MR; ++i)
        for (size_t j = 0; j < NR; ++j) acc[i][j] = 0.0f;
      if (mr == MR && nr == NR) {
        // 8-wide vectors across columns (GCC vector extension): lane j is column n0 + j, still a
        // separate multiply and add per element in kk order
        typedef float v8 __attribute__((vector_size(32)));
        v8 va[MR][2];
        for (size_t i = 0; i < MR; ++i) va[i][0] = va[i][1] = v8{};
        for (size_t kk = 0; kk < k; ++kk) {
          v8 w0, w1;
          memcpy(&w0, wt + kk * n + n0, 32);
          memcpy(&w1, wt + kk * n + n0 + 8, 32);
          for (size_t i = 0; i < MR; ++i) {
            const float av = a[(m0 + i) * k + kk];
            const v8 b = {av, av, av, av, av, av, av, av};
            const v8 p0 = b * w0, p1 = b * w1;
            va[i][0] = va[i][0] + p0;
            va[i][1] = va[i][1] + p1;
          }
        }
        for (size_t i = 0; i < MR; ++i) {
          memcpy(&acc[i][0], &va[i][0], 32);
          memcpy(&acc[i][8], &va[i][1], 32);
        }
      } else {
        for (size_t kk = 0; kk < k; ++kk) {
          const float* wr = wt + kk * n + n0;
          for (size_t i = 0; i < mr; ++i) {
            const float av = a[(m0 + i) * k + kk];
            for (size_t j = 0; j < nr; ++j) {
              float p = av * wr[j];
              acc[i][j] = acc[i][j] + p;
            }
          }
        }
      }
      for (size_t i = 0; i < mr; ++i)
        for (size_t j = 0; j < nr; ++j) out[(m0 + i) * n + n0 + j] = acc[i][j];
    }
  });
}

// Validation follows matmul.rs:18-50 and the per-type checks (:129-173).
void matmul(const float* a, size_t m, size_t k, const Tensor& w, float* out, size_t out_m,
            size_t out_n, int mode, int threads) {
  if (w.dims.size() != 2) fail(E_MATMUL, "expects 2D tensors for input, weight, and output");
  if (k != w.dims[0]) fail(E_MATMUL, "inner dim mismatch");
  size_t n = w.dims[1];
  if (out_m * out_n != m * n) fail(E_MATMUL, "output dims incompatible with matmul result");
  if (out_m != m || out_n != n) fail(E_MATMUL, "output dimensions do not match M×N of matmul");
  int t = w.dtype;
  if (t != T_F32) {
    size_t need = expected_byte_len(t, k * n);
    if (w.buf.size() < need) fail(E_MATMUL, "weight buffer is smaller than expected");
  }
  if (mode == PAIR || mode == F16) {
    if (m > 1) {
      std::vector<float> r(m * k);
      for (size_t i = 0; i < m * k; ++i) {
        // f16 round to nearest even (F16C), as the device's conversion
        const float h = _cvtsh_ss(_cvtss_sh(a[i], _MM_FROUND_TO_NEAREST_INT));
        r[i] = mode == F16 ? h : h + _cvtsh_ss(_cvtss_sh(a[i] - h, _MM_FROUND_TO_NEAREST_INT));
      }
      matmul(r.data(), m, k, w, out, out_m, out_n, REASSOC, threads);
      return;
    }
    mode = REASSOC;
  }
  if (mode == I8X2_ROW || mode == I8X2_B32 || mode == I8X3_ROW) {
    if (m > 1) {
      const size_t blk = mode == I8X2_B32 ? 32 : k;
      const int planes = mode == I8X3_ROW ? 3 : 2;
      std::vector<float> r(m * k);
      for (size_t row = 0; row < m; ++row)
        for (size_t b0 = 0; b0 < k; b0 += blk) {
          const size_t b1 = std::min(k, b0 + blk);
          const float* x = a + row * k;
          double mx = 0.0;
          for (size_t i = b0; i < b1; ++i) mx = std::max(mx, std::fabs((double)x[i]));
          for (size_t i = b0; i < b1; ++i) {
            double sc = mx / 127.0, rem = x[i], y = 0.0;
            for (int pl = 0; pl < planes && sc > 0.0; ++pl) {
              const double q = std::max(-127.0, std::min(127.0, std::nearbyint(rem / sc)));
              y += q * sc;
              rem -= q * sc;
              sc /= 254.0;
            }
            r[row * k + i] = (float)y;
          }
        }
      matmul(r.data(), m, k, w, out, out_m, out_n, REASSOC, threads);
      return;
    }
    mode = REASSOC;
  }
  size_t ops = m * n * k;
  if (mode == BASELINE) {
    // Reference decomposition: Rayon over output rows iff ops >= 64Ki (matmul.rs:206-216).
    int thr = ops >= PARALLEL_MATMUL_MIN_OPS ? threads : 1;
    parallel_for(m, thr, [&](size_t row) {
      if (t == T_F32) f32_row_kernel(a + row * k, k, w.f32(), out + row * n, 0, n);
      else q_row_kernel(t, a + row * k, k, w.buf.data(), n, out + row * n, 0, n);
    });
    return;
  }
  // PARITY mode (REASSOC: the k-major GEMM in two halves of K).
  if (m <= 4 && mode != REASSOC) {
    const size_t CH = 64;
    size_t chunks = (n + CH - 1) / CH;
    parallel_for(m * chunks, threads, [&](size_t idx) {
      size_t row = idx / chunks, c = idx % chunks;
      size_t c0 = c * CH, c1 = std::min(n, c0 + CH);
      if (t == T_F32) f32_row_kernel(a + row * k, k, w.f32(), out + row * n, c0, c1);
      else q_row_kernel(t, a + row * k, k, w.buf.data(), n, out + row * n, c0, c1);
    });
    return;
  }
  // Decode W once into a k-major copy.
  std::vector<float> wt(k * n);
  std::atomic<bool> nonfinite{false};
  if (t == T_F32) {
    const float* wf = w.f32();
    parallel_for(n, threads, [&](size_t col) {
      for (size_t kk = 0; kk < k; ++kk) {
        float v = wf[kk + col * k];
        if (!std::isfinite(v)) nonfinite = true;
        wt[kk * n + col] = v;
      }
    });
  } else if (k % block_elems(t) == 0) {
    // every column starts on a block: decode 16 columns' blocks at a time straight into the
    // k-major copy (rows of 16 contiguous floats)
    const size_t be = block_elems(t), bb = block_bytes(t), kb_n = k / be;
    parallel_for((n + 15) / 16, threads, [&](size_t g) {
      const size_t c0 = g * 16, nc = std::min<size_t>(16, n - c0);
      float dec[16][256];
      for (size_t kb = 0; kb < kb_n; ++kb) {
        for (size_t c = 0; c < nc; ++c) dequant_block(t, w.buf.data() + ((c0 + c) * kb_n + kb) * bb, dec[c]);
        for (size_t e = 0; e < be; ++e) {
          float* dst = &wt[(kb * be + e) * n + c0];
          for (size_t c = 0; c < nc; ++c) {
            const float v = dec[c][e];
            if (!std::isfinite(v)) nonfinite = true;
            dst[c] = v;
          }
        }
      }
    });
  } else {
    size_t be = block_elems(t), bb = block_bytes(t);
    size_t nblk = (k * n + be - 1) / be;
    std::vector<float> flat(nblk * be);
    parallel_for((nblk + 63) / 64, threads, [&](size_t c) {
      for (size_t bi = c * 64; bi < std::min(nblk, c * 64 + 64); ++bi)
        dequant_block(t, w.buf.data() + bi * bb, flat.data() + bi * be);
    });
    parallel_for(n, threads, [&](size_t col) {
      for (size_t kk = 0; kk < k; ++kk) {
        float v = flat[kk + col * k];
        if (!std::isfinite(v)) nonfinite = true;
        wt[kk * n + col] = v;
      }
    });
  }
  if (nonfinite.load()) {
    parallel_for(m, threads, [&](size_t row) {
      if (t == T_F32) f32_row_kernel(a + row * k, k, w.f32(), out + row * n, 0, n);
      else q_row_kernel(t, a + row * k, k, w.buf.data(), n, out + row * n, 0, n);
    });
    return;
  }
  gemm_kmajor(a, m, k, wt.data(), n, out, threads, mode == REASSOC);
}

// ---------------------------------------------------------------------------------------------
// Small ops (src/ops/*.rs)
// ---------------------------------------------------------------------------------------------

// rmsnorm (src/ops/rmsnorm.rs:25-50): s = sum x*x sequential; rms = sqrt(s/dim + eps); y = x*w/rms.
void rmsnorm(const float* in, const float* w, size_t dim, float eps, float* out) {
  float ss = 0.0f;
  for (size_t i = 0; i < dim; ++i) ss += in[i] * in[i];
  float mean = ss / (float)dim;
  float rms = sqrtf(mean + eps);
  for (size_t i = 0; i < dim; ++i) out[i] = in[i] * w[i] / rms;
}

// rmsnorm_inplace_no_scale (src/ops/rmsnorm.rs:8-23)
void rmsnorm_no_scale(float* x, size_t dim, float eps) {
  if (dim == 0) return;
  float ss = 0.0f;
  for (size_t i = 0; i < dim; ++i) ss += x[i] * x[i];
  float rms = sqrtf(ss / (float)dim + eps);
  if (rms > 0.0f)
    for (size_t i = 0; i < dim; ++i) x[i] /= rms;
}

// rope (src/ops/rope.rs:11-59): adjacent pairs, theta *= base^(-2/n_rot) running product.
void rope(float* v, size_t len, float base, uint32_t pos, uint32_t head_dim, uint32_t rotary_dim,
          const float* ff, size_t ff_len) {
  if (rotary_dim > head_dim) fail(E_OP, "RoPE rotary_dim > head_dim");
  size_t end = std::min((size_t)rotary_dim, len);
  if (end % 2 != 0) fail(E_OP, "RoPE rotary span must be even");
  size_t num_pairs = end / 2;
  if (ff && ff_len < num_pairs) fail(E_OP, "RoPE freq_factors len < num_pairs");
  float n_rot = (float)rotary_dim;
  float theta_scale = powf(base, -2.0f / n_rot);
  float theta = (float)pos;
  for (size_t k = 0; k < num_pairs; ++k) {
    float f = 1.0f;
    if (ff && k < ff_len && ff[k] != 0.0f) f = ff[k];
    float angle = theta / f;
    size_t p = 2 * k;
    float t0 = v[p], t1 = v[p + 1];
    float c = cosf(angle), s = sinf(angle);
    v[p] = t0 * c - t1 * s;
    v[p + 1] = t0 * s + t1 * c;
    theta *= theta_scale;
  }
}

// softmax (src/ops/softmax.rs:3-28): recomputes exp in the output pass.
void softmax(const float* in, float* out, size_t n) {
  if (n == 0) fail(E_OP, "softmax: empty input");
  float mx = in[0];
  for (size_t i = 0; i < n; ++i)
    if (in[i] > mx) mx = in[i];
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) sum += expf(in[i] - mx);
  for (size_t i = 0; i < n; ++i) out[i] = expf(in[i] - mx) / sum;
}

// sigmoid + swiglu (src/ops/swiglu.rs:3-36): y = (g * sigmoid(g)) * u.
static inline float sigmoid1(float x) {
  if (x >= 0.0f) {
    float z = expf(-x);
    return 1.0f / (1.0f + z);
  }
  float z = expf(x);
  return z / (1.0f + z);
}
void swiglu(const float* g, const float* u, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    float s = sigmoid1(g[i]);
    out[i] = g[i] * s * u[i];
  }
}

// gelu_tanh (src/ops/gelu.rs:5-11): SQRT_2_OVER_PI = FRAC_2_SQRT_PI * FRAC_1_SQRT_2 in f32.
static const float SQRT_2_OVER_PI = 1.12837916709551257390f * 0.707106781186547524401f;
float gelu_tanh(float x) {
  float x3 = x * x * x;
  return 0.5f * x * (1.0f + tanhf(SQRT_2_OVER_PI * (x + 0.044715f * x3)));
}

// residual_add (src/ops/residual_add.rs:3-12)
void residual_add(const float* a, const float* b, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

// sample_temperature (src/engine/sampling.rs:54-79) for the uniform draw r the reference takes
// from rng.gen_range(0.0..1.0): -1 = EmptyLogits, -3 = InvalidTemperature; else the first index
// whose cumulative f32 probability exceeds r, or the last index.
long sample_temperature(const float* l, size_t n, float temperature, float r) {
  if (n == 0) return -1;
  if (!std::isfinite(temperature) || temperature <= 0.0f) return -3;
  std::vector<float> scaled(n), probs(n);
  for (size_t i = 0; i < n; ++i) scaled[i] = l[i] / temperature;
  softmax(scaled.data(), probs.data(), n);
  float cum = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    cum += probs[i];
    if (r < cum || i + 1 == n) return (long)i;
  }
  return (long)(n - 1);
}

// argmax_index / sample_greedy (src/engine/sampling.rs:25-49):
// -1 = EmptyLogits, -2 = InvalidLogits (any non-finite); first index wins ties.
long argmax(const float* l, size_t n) {
  if (n == 0) return -1;
  for (size_t i = 0; i < n; ++i)
    if (!std::isfinite(l[i])) return -2;
  size_t best = 0;
  float bv = l[0];
  for (size_t i = 1; i < n; ++i)
    if (l[i] > bv) {
      bv = l[i];
      best = i;
    }
  return (long)best;
}

// unpack_llama_gguf_qk_row (src/layers/attention.rs:149-172)
void unpack_qk_row(float* row, size_t n_groups, size_t head_dim) {
  size_t half = head_dim / 2;
  std::vector<float> tmp(row, row + n_groups * head_dim);
  for (size_t g = 0; g < n_groups; ++g) {
    size_t base = g * head_dim;
    for (size_t h = 0; h < half; ++h)
      for (size_t b = 0; b < 2; ++b) row[base + b * half + h] = tmp[base + h * 2 + b];
  }
}

// ---------------------------------------------------------------------------------------------
// GGUF reader (src/model_loader/{file_loader,parser,reader,tensor_loader}.rs)
// ---------------------------------------------------------------------------------------------
struct Reader {
  FILE* f;
  uint64_t pos = 0;
  void read(void* dst, size_t n) {
    if (n && fread(dst, 1, n, f) != n) fail(E_IO, "failed to fill whole buffer");
    pos += n;
  }
  template <class T>
  T get() {
    T v;
    read(&v, sizeof(T));
    return v;
  }
  std::string str() {
    uint64_t len = get<uint64_t>();
    std::string s(len, '\0');
    read(&s[0], len);
    return s;
  }
};

static GVal read_value(Reader& r, uint32_t type);

static uint32_t check_type(uint32_t code) {
  if (code > 12) fail(E_GGUF, "unknown value type code " + std::to_string(code));
  return code;
}

// reader.rs:94-114 (bool must be 0 or 1), :130-157 (arrays).
static GVal read_value(Reader& r, uint32_t type) {
  GVal v;
  v.type = (int)type;
  switch (type) {
    case G_U8: v.u = r.get<uint8_t>(); break;
    case G_I8: v.i = r.get<int8_t>(); break;
    case G_U16: v.u = r.get<uint16_t>(); break;
    case G_I16: v.i = r.get<int16_t>(); break;
    case G_U32: v.u = r.get<uint32_t>(); break;
    case G_I32: v.i = r.get<int32_t>(); break;
    case G_F32: v.f32 = r.get<float>(); v.f = v.f32; break;
    case G_BOOL: {
      uint8_t b = r.get<uint8_t>();
      if (b > 1) fail(E_GGUF, "invalid GGUF bool byte (expected 0 or 1, got " + std::to_string(b) + ")");
      v.b = b == 1;
      break;
    }
    case G_STR: v.s = r.str(); break;
    case G_ARR: {
      uint32_t et = check_type(r.get<uint32_t>());
      uint64_t len = r.get<uint64_t>();
      v.arr.reserve(len);
      for (uint64_t i = 0; i < len; ++i) v.arr.push_back(read_value(r, et));
      break;
    }
    case G_U64: v.u = r.get<uint64_t>(); break;
    case G_I64: v.i = r.get<int64_t>(); break;
    case G_F64: v.f = r.get<double>(); break;
    default: fail(E_GGUF, "unknown value type code");
  }
  return v;
}

// GgmlType -> TensorType (src/model_loader/tensor.rs:86-97); BF16 (30) widened at load.
static int ggml_to_ttype(uint32_t id) {
  switch (id) {
    case 0: return T_F32;
    case 12: return T_Q4K;
    case 14: return T_Q6K;
    case 8: return T_Q8_0;
  }
  fail(E_TENSOR, "unsupported GGML type for inference: " + std::to_string(id));
}

// read_file (file_loader.rs:26-65) + tensor_data_section_offset (:11-22).
static void read_gguf_meta(const std::string& path, GGUF& g) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) fail(E_IO, "cannot open " + path);
  Reader r{f};
  try {
    char magic[4];
    r.read(magic, 4);  // magic is read, not validated (file_loader.rs:31)
    g.version = r.get<uint32_t>();
    uint64_t nt = r.get<uint64_t>(), nkv = r.get<uint64_t>();
    for (uint64_t i = 0; i < nkv; ++i) {
      std::string key = r.str();
      uint32_t ty = check_type(r.get<uint32_t>());
      g.kv[key] = read_value(r, ty);
    }
    for (uint64_t i = 0; i < nt; ++i) {
      TensorInfo ti;
      ti.name = r.str();
      uint32_t nd = r.get<uint32_t>();
      for (uint32_t d = 0; d < nd; ++d) ti.dims.push_back((size_t)r.get<uint64_t>());
      ti.type_id = r.get<uint32_t>();
      ti.offset = r.get<uint64_t>();
      g.infos.push_back(ti);
    }
    uint64_t align = 32;
    const GVal* a = g.meta("general.alignment");
    if (a && a->type == G_U32 && a->u > 0 && (a->u & (a->u - 1)) == 0) align = a->u;
    g.data_offset = (r.pos + align - 1) & ~(align - 1);
  } catch (...) {
    fclose(f);
    throw;
  }
  fclose(f);
}

// load_tensor (tensor_loader.rs:27-67): raw block bytes; BF16 -> F32.
static void load_tensors(const std::string& path, GGUF& g, const std::vector<std::string>& names) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) fail(E_IO, "cannot open " + path);
  std::vector<size_t> idx;
  for (auto& n : names) {
    if (g.tensors.count(n)) continue;
    bool found = false;
    for (size_t i = 0; i < g.infos.size(); ++i)
      if (g.infos[i].name == n) {
        if (std::find(idx.begin(), idx.end(), i) == idx.end()) idx.push_back(i);
        found = true;
        break;
      }
    if (!found) {
      fclose(f);
      fail(E_MODEL, "tensor '" + n + "' not found in model metadata");
    }
  }
  std::sort(idx.begin(), idx.end(), [&](size_t x, size_t y) { return g.infos[x].offset < g.infos[y].offset; });
  try {
    for (size_t i : idx) {
      const TensorInfo& ti = g.infos[i];
      size_t nelem = 1;
      for (size_t d : ti.dims) nelem *= d;
      uint64_t abs = g.data_offset + ti.offset;
      if (fseeko(f, (off_t)abs, SEEK_SET) != 0) fail(E_GGUF, "seek failed");
      Tensor t;
      t.dims = ti.dims;
      if (ti.type_id == 30) {  // BF16 -> F32 (tensor_loader.rs:11-16, :39-54)
        std::vector<uint16_t> raw(nelem);
        if (nelem && fread(raw.data(), 2, nelem, f) != nelem) fail(E_IO, "failed to fill whole buffer");
        t.dtype = T_F32;
        t.buf.resize(nelem * 4);
        for (size_t e = 0; e < nelem; ++e) {
          uint32_t bits = (uint32_t)raw[e] << 16;
          memcpy(&t.buf[e * 4], &bits, 4);
        }
      } else {
        if (ti.type_id > 40 || ti.type_id == 4 || ti.type_id == 5 || (ti.type_id > 30 && ti.type_id < 34) ||
            (ti.type_id > 35 && ti.type_id < 39))
          fail(E_GGUF, "unknown GGML type id: " + std::to_string(ti.type_id));
        t.dtype = ggml_to_ttype(ti.type_id);
        size_t bl = expected_byte_len(t.dtype, nelem);
        t.buf.resize(bl);
        if (bl && fread(t.buf.data(), 1, bl, f) != bl) fail(E_IO, "failed to fill whole buffer");
      }
      g.tensors[ti.name] = std::move(t);
    }
  } catch (...) {
    fclose(f);
    throw;
  }
  fclose(f);
}

// ---------------------------------------------------------------------------------------------
// ModelConfig::from_gguf (src/model_config.rs:143-306) and helpers (:631-730)
// ---------------------------------------------------------------------------------------------
static bool usize_from(const GVal& v, size_t* out) {
  switch (v.type) {
    case G_U8: case G_U16: case G_U32: case G_U64: *out = (size_t)v.u; return true;
    case G_I8: case G_I16: case G_I32: case G_I64:
      if (v.i < 0) return false;
      *out = (size_t)v.i;
      return true;
  }
  return false;
}
static bool get_usize_opt(const GGUF& g, const std::string& k, size_t* out) {
  const GVal* v = g.meta(k);
  if (!v) return false;
  if (v->type == G_ARR) {
    if (v->arr.empty()) return false;
    return usize_from(v->arr[0], out);
  }
  return usize_from(*v, out);
}
static size_t get_usize_alt(const GGUF& g, const std::vector<std::string>& keys) {
  size_t v;
  for (auto& k : keys)
    if (get_usize_opt(g, k, &v)) return v;
  fail(E_MODEL, "missing integer metadata; tried keys " + keys[0]);
}
static bool get_f32_opt(const GGUF& g, const std::string& k, float* out) {
  const GVal* v = g.meta(k);
  if (!v) return false;
  if (v->type == G_F32) { *out = v->f32; return true; }
  if (v->type == G_F64) { *out = (float)v->f; return true; }
  return false;
}
static std::string get_string(const GGUF& g, const std::string& k) {
  const GVal* v = g.meta(k);
  return (v && v->type == G_STR) ? v->s : std::string();
}
// get_u32 (model_config.rs:711-723): an integer of any width whose value fits u32, else `dflt`.
static uint32_t get_u32_or(const GGUF& g, const std::string& k, uint32_t dflt) {
  const GVal* v = g.meta(k);
  if (!v) return dflt;
  switch (v->type) {
    case G_U8: case G_U16: case G_U32: case G_U64:
      return v->u <= 0xFFFFFFFFull ? (uint32_t)v->u : dflt;
    case G_I8: case G_I16: case G_I32: case G_I64:
      return (v->i >= 0 && v->i <= 0xFFFFFFFFll) ? (uint32_t)v->i : dflt;
  }
  return dflt;
}
static std::string lower(std::string s) {
  for (auto& c : s) c = (char)tolower((unsigned char)c);
  return s;
}

// detect_model_family (model_config.rs:461-482)
static int detect_family(const GGUF& g) {
  std::string arch = lower(get_string(g, "general.architecture"));
  std::string name = lower(get_string(g, "general.name"));
  if (arch.find("gemma4") != std::string::npos || arch.find("gemma-4") != std::string::npos ||
      name.find("gemma-4") != std::string::npos || name.find("gemma4") != std::string::npos)
    return GEMMA4;
  if (g.meta("gemma4.attention.sliding_window_pattern")) return GEMMA4;
  return MISTRAL_LLAMA;
}

static const TensorInfo* find_info(const GGUF& g, const std::string& n) {
  for (auto& t : g.infos)
    if (t.name == n) return &t;
  return nullptr;
}

// tensor_weight_k_n (model_config.rs:446-459)
static void weight_k_n(const GGUF& g, const std::string& n, size_t* k, size_t* nn) {
  const TensorInfo* t = find_info(g, n);
  if (!t) fail(E_MODEL, "missing tensor metadata '" + n + "'");
  if (t->dims.size() < 2) fail(E_MODEL, "tensor '" + n + "': expected 2 dimensions");
  *k = t->dims[0];
  *nn = t->dims[1];
}

static bool env_is(const char* name, bool* val) {
  const char* v = getenv(name);
  if (!v) return false;
  std::string s = lower(v);
  if (s == "1" || s == "true") { *val = true; return true; }
  if (s == "0" || s == "false") { *val = false; return true; }
  return false;
}

static ModelConfig config_from_gguf(const GGUF& g) {
  ModelConfig c;
  c.context_length = get_usize_alt(g, {"llama.context_length", "gemma4.context_length"});
  c.hidden_dim = get_usize_alt(g, {"llama.embedding_length", "gemma4.embedding_length"});
  c.n_layers = get_usize_alt(g, {"llama.block_count", "gemma4.block_count"});
  c.n_heads = get_usize_alt(g, {"llama.attention.head_count", "gemma4.attention.head_count"});
  size_t nkv;
  if (get_usize_opt(g, "llama.attention.head_count_kv", &nkv) ||
      get_usize_opt(g, "gemma4.attention.head_count_kv", &nkv))
    c.n_kv_heads = nkv;
  else
    c.n_kv_heads = c.n_heads;
  size_t ffn_meta = get_usize_alt(g, {"llama.feed_forward_length", "gemma4.feed_forward_length"});
  float th;
  if (get_f32_opt(g, "llama.rope.theta", &th) || get_f32_opt(g, "gemma4.rope.freq_base", &th))
    c.rope_theta = th;
  else
    c.rope_theta = 10000.0f;
  float eps;
  if (get_f32_opt(g, "llama.attention.layer_norm_rms_epsilon", &eps) ||
      get_f32_opt(g, "gemma4.attention.layer_norm_rms_epsilon", &eps))
    c.rms_norm_eps = eps;
  else
    fail(E_MODEL, "missing float metadata; tried keys [llama.attention.layer_norm_rms_epsilon, ...]");
  size_t vs;
  if (get_usize_opt(g, "llama.vocab_size", &vs) || get_usize_opt(g, "gemma4.vocab_size", &vs)) {
    c.vocab_size = vs;
  } else {
    const GVal* t = g.meta("tokenizer.ggml.tokens");
    if (!t) fail(E_MODEL, "missing metadata key 'tokenizer.ggml.tokens'");
    if (t->type != G_ARR) fail(E_MODEL, "metadata key 'tokenizer.ggml.tokens' is not an array");
    c.vocab_size = t->arr.size();
  }
  size_t hd;
  size_t kd;
  if (get_usize_opt(g, "gemma4.attention.key_length", &kd)) {
    if (kd * c.n_heads == c.hidden_dim) hd = kd;
    else if (c.hidden_dim % c.n_heads != 0) fail(E_MODEL, "hidden_dim not divisible by n_heads");
    else hd = c.hidden_dim / c.n_heads;
  } else if (c.hidden_dim % c.n_heads != 0) {
    fail(E_MODEL, "hidden_dim not divisible by n_heads");
  } else {
    hd = c.hidden_dim / c.n_heads;
  }
  if (c.n_heads % c.n_kv_heads != 0) fail(E_MODEL, "GQA requires n_heads divisible by n_kv_heads");
  c.family = detect_family(g);
  std::string nm = lower(get_string(g, "general.name"));
  bool mistral_style = nm.find("mistral") != std::string::npos || nm.find("gemma") != std::string::npos;
  bool val;
  if (env_is("INFERENCE_ENGINE_GGUF_QK_UNPACK", &val)) c.unpack_llama_gguf_qk = val;
  else {
    const char* no = getenv("INFERENCE_ENGINE_GGUF_NO_QK_UNPACK");
    std::string ns = no ? lower(no) : "";
    if (no && (ns == "1" || ns == "true")) c.unpack_llama_gguf_qk = false;
    else c.unpack_llama_gguf_qk = c.family == GEMMA4 ? false : !mistral_style;
  }
  // infer_layer_dims (model_config.rs:374-444)
  if (c.family == MISTRAL_LLAMA) {
    for (size_t i = 0; i < c.n_layers; ++i) c.layer_dims.push_back({c.n_heads * hd, c.n_kv_heads * hd, hd, ffn_meta});
  } else {
    for (size_t i = 0; i < c.n_layers; ++i) {
      std::string p = "blk." + std::to_string(i) + ".";
      size_t kq, qd, kk, kvd, kg, fd;
      weight_k_n(g, p + "attn_q.weight", &kq, &qd);
      weight_k_n(g, p + "attn_k.weight", &kk, &kvd);
      weight_k_n(g, p + "ffn_gate.weight", &kg, &fd);
      if (kq != c.hidden_dim || kk != c.hidden_dim || kg != c.hidden_dim)
        fail(E_MODEL, "layer " + std::to_string(i) + ": unexpected attn/FFN input dim");
      if (qd % c.n_heads != 0) fail(E_MODEL, "q out dim not divisible by n_heads");
      if (kvd % c.n_kv_heads != 0) fail(E_MODEL, "k out dim not divisible by n_kv_heads");
      size_t hq = qd / c.n_heads, hk = kvd / c.n_kv_heads;
      if (hq != hk) fail(E_MODEL, "Q head dim != KV head dim");
      c.layer_dims.push_back({qd, kvd, hq, fd});
    }
  }
  if (c.family == MISTRAL_LLAMA) {
    c.head_dim = hd;
    c.ffn_dim = ffn_meta;
  } else {
    if (c.layer_dims.empty()) fail(E_MODEL, "layer_dims empty");
    c.head_dim = 0;
    c.ffn_dim = 0;
    for (auto& d : c.layer_dims) {
      c.head_dim = std::max(c.head_dim, d.head_dim);
      c.ffn_dim = std::max(c.ffn_dim, d.ffn_dim);
    }
  }
  // build_layer_attention_specs (model_config.rs:484-513) / gemma4 (:515-629)
  if (c.layer_dims.size() != c.n_layers) fail(E_MODEL, "layer_attention: layer_dims len != n_layers");
  if (c.n_layers == 0) fail(E_MODEL, "layer_dims empty");
  size_t hd0 = c.layer_dims[0].head_dim;
  if (hd0 == 0 || hd0 % 2 != 0) fail(E_MODEL, "layer attention: head_dim must be positive and even");
  if (c.family == MISTRAL_LLAMA) {
    LayerAttentionSpec s;
    s.sliding_window = -1;
    s.rope_theta = c.rope_theta;
    s.rope_rotary_dim = hd0;
    c.layer_attention.assign(c.n_layers, s);
  } else {
    const GVal* pat = g.meta("gemma4.attention.sliding_window_pattern");
    if (!pat) fail(E_MODEL, "Gemma 4 GGUF missing gemma4.attention.sliding_window_pattern");
    if (pat->type != G_ARR) fail(E_MODEL, "gemma4.attention.sliding_window_pattern has wrong type");
    if (pat->arr.size() != c.n_layers) fail(E_MODEL, "sliding_window_pattern length != n_layers");
    std::vector<bool> swa;
    for (auto& it : pat->arr) {
      if (it.type == G_BOOL) swa.push_back(it.b);
      else if (it.type == G_U8 || it.type == G_U32) swa.push_back(it.u != 0);
      else if (it.type == G_I8 || it.type == G_I32) swa.push_back(it.i != 0);
      else fail(E_MODEL, "gemma4.attention.sliding_window_pattern must be bool[] (or integer 0/1)");
    }
    size_t window;
    if (!get_usize_opt(g, "gemma4.attention.sliding_window", &window) &&
        !get_usize_opt(g, "llama.attention.sliding_window", &window))
      fail(E_MODEL, "Gemma 4 GGUF missing sliding window size");
    if (window == 0) fail(E_MODEL, "Gemma 4 sliding window size must be > 0");
    size_t default_hd = c.layer_dims[0].head_dim;
    size_t rd_local, rd_global;
    if (!get_usize_opt(g, "gemma4.rope.dimension_count_swa", &rd_local) &&
        !get_usize_opt(g, "gemma4.attention.rotary_dim_local", &rd_local) &&
        !get_usize_opt(g, "llama.rope.dimension_count", &rd_local))
      rd_local = default_hd;
    if (!get_usize_opt(g, "gemma4.rope.dimension_count", &rd_global) &&
        !get_usize_opt(g, "gemma4.attention.rotary_dim_global", &rd_global))
      rd_global = rd_local;
    auto clamp_rot = [](size_t rd, size_t mx) {
      rd = std::min(rd, mx);
      if (rd == 0) rd = mx;
      if (rd % 2 != 0) rd -= 1;
      return rd;
    };
    float th_local, th_global;
    if (!get_f32_opt(g, "gemma4.rope.freq_base_swa", &th_local) && !get_f32_opt(g, "gemma4.rope.local_theta", &th_local))
      th_local = c.rope_theta;
    if (!get_f32_opt(g, "gemma4.rope.freq_base", &th_global) && !get_f32_opt(g, "gemma4.rope.global_theta", &th_global))
      th_global = c.rope_theta;
    for (size_t i = 0; i < c.n_layers; ++i) {
      LayerAttentionSpec s;
      s.rope_rotary_dim = clamp_rot(swa[i] ? rd_local : rd_global, c.layer_dims[i].head_dim);
      s.sliding_window = swa[i] ? (long)window : -1;
      s.rope_theta = swa[i] ? th_local : th_global;
      c.layer_attention.push_back(s);
    }
  }
  size_t ple = 0;
  if (c.family == GEMMA4) {
    if (!get_usize_opt(g, "gemma4.embedding_length_per_layer_input", &ple)) ple = 0;
  }
  c.embedding_length_per_layer = ple;
  c.token_embedding_scale = c.family == GEMMA4 ? sqrtf((float)c.hidden_dim) : 1.0f;
  if (ple > 0) {
    c.ple_combine_scale = 1.0f / sqrtf(2.0f);
    c.ple_model_proj_scale = 1.0f / sqrtf((float)c.hidden_dim);
  }
  // build_gemma4_kv_borrow_from (model_config.rs:332-372)
  c.kv_borrow_from.assign(c.n_layers, -1);
  if (c.family == GEMMA4) {
    size_t n_shared = 0;
    if (!get_usize_opt(g, "gemma4.attention.shared_kv_layers", &n_shared)) n_shared = 0;
    if (n_shared > 0) {
      if (n_shared > c.n_layers) fail(E_MODEL, "gemma4 attention.shared_kv_layers exceeds block_count");
      size_t first = c.n_layers - n_shared;
      if (first == 0) fail(E_MODEL, "gemma4: shared_kv_layers == block_count is unsupported");
      for (size_t li = first; li < c.n_layers; ++li) {
        bool want = c.layer_attention[li].sliding_window >= 0;
        long src = -1;
        for (size_t s = first; s-- > 0;)
          if ((c.layer_attention[s].sliding_window >= 0) == want) {
            src = (long)s;
            break;
          }
        if (src < 0) fail(E_MODEL, "Gemma 4: no KV-borrow source for layer");
        c.kv_borrow_from[li] = src;
      }
    }
  }
  float cap;
  if (get_f32_opt(g, "gemma4.final_logit_softcapping", &cap) && cap > 0.0f && std::isfinite(cap)) {
    c.has_softcap = true;
    c.softcap = cap;
  }
  // TokenizerPromptConfig::from_gguf (model_config.rs:35-50) with
  // defaults_for_tokenizer_model (:53-60): "llama" -> (add BOS, no EOS), otherwise neither
  const bool llama_vocab = get_string(g, "tokenizer.ggml.model") == "llama";
  c.add_bos_token = llama_vocab;
  c.add_eos_token = false;
  if (const GVal* v = g.meta("tokenizer.ggml.add_bos_token"); v && v->type == G_BOOL) c.add_bos_token = v->b;
  if (const GVal* v = g.meta("tokenizer.ggml.add_eos_token"); v && v->type == G_BOOL) c.add_eos_token = v->b;
  c.bos_token_id = get_u32_or(g, "tokenizer.ggml.bos_token_id", 1);
  c.eos_token_id = get_u32_or(g, "tokenizer.ggml.eos_token_id", 2);
  return c;
}

// ---------------------------------------------------------------------------------------------
// Weight name resolution (src/model_weights/names.rs:52-336)
// ---------------------------------------------------------------------------------------------
static bool has_info(const GGUF& g, const std::string& n) { return find_info(g, n) != nullptr; }
static std::string resolve(const GGUF& g, const std::vector<std::string>& cands) {
  for (auto& c : cands)
    if (has_info(g, c)) return c;
  fail(E_MODEL, "none of the candidate tensor names were found: " + cands[0]);
}
static std::string optional(const GGUF& g, const std::vector<std::string>& cands) {
  for (auto& c : cands)
    if (has_info(g, c)) return c;
  return "";
}

struct Names {
  std::string emb, out_norm, lm_head;
  struct L {
    std::string attn_norm, ffn_norm, attn_post, ffn_post, qn, kn, wq, wk, wv, wo, gate, up, down,
        ple_gate, ple_proj, ple_post, rope_freqs, out_scale;
  };
  std::vector<L> layers;
  std::string ple_tok, ple_mproj, ple_pnorm;
};

static Names resolve_names(const GGUF& g, const ModelConfig& c) {
  Names n;
  n.emb = resolve(g, {"token_embd.weight", "tok_embeddings.weight", "embeddings.weight"});
  n.out_norm = resolve(g, {"output_norm.weight", "norm.weight"});
  n.lm_head = optional(g, {"output.weight", "lm_head.weight"});
  if (n.lm_head.empty()) {
    if (has_info(g, "token_embd.weight")) n.lm_head = "token_embd.weight";
    else fail(E_MODEL, "LM head: none of output.weight, lm_head.weight, token_embd.weight (tied) found");
  }
  for (size_t i = 0; i < c.n_layers; ++i) {
    std::string p = "blk." + std::to_string(i) + ".";
    Names::L l;
    if (c.family == GEMMA4) {
      l.attn_post = resolve(g, {p + "post_attention_norm.weight"});
      l.ffn_post = resolve(g, {p + "post_ffw_norm.weight"});
      if (c.embedding_length_per_layer > 0) {
        l.ple_gate = resolve(g, {p + "inp_gate.weight"});
        l.ple_proj = resolve(g, {p + "proj.weight"});
        l.ple_post = resolve(g, {p + "post_norm.weight"});
      }
    }
    l.attn_norm = resolve(g, {p + "attn_norm.weight", p + "attention_norm.weight"});
    l.ffn_norm = resolve(g, {p + "ffn_norm.weight", p + "feed_forward_norm.weight"});
    l.wq = resolve(g, {p + "attn_q.weight", p + "wq.weight"});
    l.wk = resolve(g, {p + "attn_k.weight", p + "wk.weight"});
    l.wv = resolve(g, {p + "attn_v.weight", p + "wv.weight"});
    l.wo = resolve(g, {p + "attn_output.weight", p + "wo.weight"});
    l.gate = resolve(g, {p + "ffn_gate.weight", p + "w1.weight"});
    l.up = resolve(g, {p + "ffn_up.weight", p + "w3.weight"});
    l.down = resolve(g, {p + "ffn_down.weight", p + "w2.weight"});
    l.qn = optional(g, {p + "attn_q_norm.weight"});
    l.kn = optional(g, {p + "attn_k_norm.weight"});
    l.rope_freqs = optional(g, {p + "rope_freqs.weight", p + "rope_freqs"});
    l.out_scale = optional(g, {p + "layer_output_scale.weight"});
    n.layers.push_back(l);
  }
  if (c.family == GEMMA4 && c.embedding_length_per_layer > 0) {
    n.ple_tok = resolve(g, {"per_layer_token_embd.weight"});
    n.ple_mproj = resolve(g, {"per_layer_model_proj.weight"});
    n.ple_pnorm = resolve(g, {"per_layer_proj_norm.weight"});
  }
  return n;
}

// LoadedModel::load (src/loaded_model.rs:23-50)
Model* model_load(const std::string& path) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) fail(E_MODEL, "model file not found: " + path);
  fclose(f);
  std::unique_ptr<Model> m(new Model());
  read_gguf_meta(path, m->gguf);
  m->cfg = config_from_gguf(m->gguf);
  Names n = resolve_names(m->gguf, m->cfg);
  std::vector<std::string> all = {n.emb, n.out_norm, n.lm_head};
  for (auto& l : n.layers) {
    for (auto* s : {&l.attn_norm, &l.ffn_norm, &l.attn_post, &l.ffn_post, &l.qn, &l.kn, &l.wq, &l.wk, &l.wv,
                    &l.wo, &l.gate, &l.up, &l.down, &l.ple_gate, &l.ple_proj, &l.ple_post, &l.rope_freqs,
                    &l.out_scale})
      if (!s->empty()) all.push_back(*s);
  }
  for (auto* s : {&n.ple_tok, &n.ple_mproj, &n.ple_pnorm})
    if (!s->empty()) all.push_back(*s);
  load_tensors(path, m->gguf, all);
  auto get = [&](const std::string& s) -> const Tensor* {
    if (s.empty()) return nullptr;
    const Tensor* t = m->gguf.get(s);
    if (!t) fail(E_MODEL, "tensor '" + s + "' not found after loading");
    return t;
  };
  m->w.token_embd = get(n.emb);
  m->w.output_norm = get(n.out_norm);
  m->w.lm_head = get(n.lm_head);
  for (auto& l : n.layers) {
    LayerW lw;
    lw.attn_norm = get(l.attn_norm);
    lw.ffn_norm = get(l.ffn_norm);
    lw.attn_post_norm = get(l.attn_post);
    lw.ffn_post_norm = get(l.ffn_post);
    lw.attn_q_norm = get(l.qn);
    lw.attn_k_norm = get(l.kn);
    lw.wq = get(l.wq);
    lw.wk = get(l.wk);
    lw.wv = get(l.wv);
    lw.wo = get(l.wo);
    lw.w_gate = get(l.gate);
    lw.w_up = get(l.up);
    lw.w_down = get(l.down);
    lw.ple_inp_gate = get(l.ple_gate);
    lw.ple_proj = get(l.ple_proj);
    lw.ple_post_norm = get(l.ple_post);
    lw.rope_freqs = get(l.rope_freqs);
    lw.layer_output_scale = get(l.out_scale);
    m->w.layers.push_back(lw);
  }
  m->w.ple_token_embd = get(n.ple_tok);
  m->w.ple_model_proj = get(n.ple_mproj);
  m->w.ple_proj_norm = get(n.ple_pnorm);
  m->emb_name = n.emb;
  return m.release();
}

// ---------------------------------------------------------------------------------------------
// Embeddings (src/layers/embeddings.rs:95-210)
// ---------------------------------------------------------------------------------------------
static std::vector<float> lookup_rows(const Tensor& t, const uint32_t* ids, size_t n, size_t* hidden_out) {
  if (t.dims.size() != 2) fail(E_TENSOR, "expected 2D embedding tensor");
  size_t hidden, vocab;
  if (t.dims[0] < t.dims[1]) { hidden = t.dims[0]; vocab = t.dims[1]; }
  else { hidden = t.dims[1]; vocab = t.dims[0]; }
  for (size_t i = 0; i < n; ++i)
    if ((size_t)ids[i] >= vocab)
      fail(E_MODEL, "token ID " + std::to_string(ids[i]) + " out of vocabulary range [0, " + std::to_string(vocab) + ")");
  std::vector<float> out(n * hidden);
  for (size_t r = 0; r < n; ++r) {
    float* row = out.data() + r * hidden;
    if (t.dtype == T_F32) {
      for (size_t h = 0; h < hidden; ++h) {
        size_t idx = (size_t)ids[r] * hidden + h;
        if ((idx + 1) * 4 > t.buf.size()) fail(E_TENSOR, "F32 index out of bounds");
        row[h] = t.f32()[idx];
      }
    } else {
      size_t be = block_elems(t.dtype), bb = block_bytes(t.dtype);
      float dec[256];
      size_t cur = (size_t)-1;
      for (size_t h = 0; h < hidden; ++h) {
        size_t idx = (size_t)ids[r] * hidden + h;
        size_t bi = idx / be;
        if (bi != cur) {
          if ((bi + 1) * bb > t.buf.size()) fail(E_TENSOR, "embedding block out of bounds");
          dequant_block(t.dtype, t.buf.data() + bi * bb, dec);
          cur = bi;
        }
        row[h] = dec[idx % be];
      }
    }
  }
  *hidden_out = hidden;
  return out;
}

// compute_packed_per_layer_inputs (src/layers/gemma4_ple.rs:27-109)
static std::vector<float> ple_packed(const Model& m, const uint32_t* ids, size_t n, const std::vector<float>& emb,
                                     int mode, int thr) {
  const ModelConfig& c = m.cfg;
  size_t pd = c.embedding_length_per_layer, nl = c.n_layers, pack = nl * pd;
  std::vector<float> proj(n * pack);
  matmul(emb.data(), n, c.hidden_dim, *m.w.ple_model_proj, proj.data(), n, pack, mode, thr);
  for (auto& v : proj) v *= c.ple_model_proj_scale;
  float sqrt_ple = sqrtf((float)pd);
  const Tensor& nw = *m.w.ple_proj_norm;
  if (nw.f32_len() != pd) fail(E_MODEL, "per_layer_proj_norm len != ple_dim");
  std::vector<float> out(n * pack), normed(pd);
  for (size_t p = 0; p < n; ++p) {
    size_t hid;
    std::vector<float> tok = lookup_rows(*m.w.ple_token_embd, &ids[p], 1, &hid);
    if (tok.size() != pack) fail(E_MODEL, "per_layer_token_embd row width != n_layers*ple_dim");
    for (auto& v : tok) v *= sqrt_ple;
    size_t base = p * pack;
    for (size_t l = 0; l < nl; ++l) {
      size_t off = base + l * pd;
      rmsnorm(&proj[off], nw.f32(), pd, c.rms_norm_eps, normed.data());
      for (size_t i = 0; i < pd; ++i) out[off + i] = (normed[i] + tok[l * pd + i]) * c.ple_combine_scale;
    }
  }
  return out;
}

// prefill_from_tokens_loaded / prefill_state_for_single_token_loaded (src/engine/embed.rs:53-149)
static State embed_tokens(const Session& s, const uint32_t* ids, size_t n, bool check_ctx) {
  const Model& m = *s.model;
  const ModelConfig& c = m.cfg;
  if (check_ctx) {
    if (n == 0) fail(E_MODEL, "prefill: empty token list");
    if (n > c.context_length)
      fail(E_MODEL, "prefill: token length " + std::to_string(n) + " exceeds context length " + std::to_string(c.context_length));
  }
  State st;
  size_t hid;
  st.hidden = lookup_rows(*m.w.token_embd, ids, n, &hid);
  if (c.token_embedding_scale != 1.0f)
    for (auto& v : st.hidden) v *= c.token_embedding_scale;
  if (hid != c.hidden_dim) fail(E_MODEL, "ForwardState: embedding dim mismatch");
  st.seq_len = n;
  st.hidden_dim = c.hidden_dim;
  if (c.family == GEMMA4 && c.embedding_length_per_layer > 0) {
    st.ple_packed = ple_packed(m, ids, n, st.hidden, s.mode, s.threads);
    st.ple_n_layers = c.n_layers;
    st.ple_dim = c.embedding_length_per_layer;
  }
  return st;
}

// ---------------------------------------------------------------------------------------------
// Attention (src/layers/attention.rs)
// ---------------------------------------------------------------------------------------------
static void append_kv(KVCache& kv, const float* k, const float* v) {  // attention.rs:54-74
  if (kv.current_pos >= kv.max_seq_len) fail(E_KVCACHE, "KVCache is Full: max len is " + std::to_string(kv.max_seq_len) + ".");
  size_t e = kv.n_kv_heads * kv.head_dim;
  memcpy(&kv.k[kv.current_pos * e], k, e * 4);
  memcpy(&kv.v[kv.current_pos * e], v, e * 4);
  kv.current_pos++;
}
static const float* kslice(const KVCache& kv, size_t pos, size_t h) {  // attention.rs:77-92
  if (pos >= kv.current_pos) fail(E_KVCACHE, "KV cache position out of bounds");
  if (h >= kv.n_kv_heads) fail(E_KVCACHE, "KV head index out of bounds");
  return &kv.k[pos * kv.n_kv_heads * kv.head_dim + h * kv.head_dim];
}
static const float* vslice(const KVCache& kv, size_t pos, size_t h) {
  if (pos >= kv.current_pos) fail(E_KVCACHE, "KV cache position out of bounds");
  if (h >= kv.n_kv_heads) fail(E_KVCACHE, "KV head index out of bounds");
  return &kv.v[pos * kv.n_kv_heads * kv.head_dim + h * kv.head_dim];
}

// apply_optional_head_rmsnorm (attention.rs:424-455)
static void head_rmsnorm(float* row, size_t ng, size_t hd, const Tensor* norm, float eps) {
  if (!norm) return;
  if (norm->f32_len() != hd) fail(E_MODEL, "attn q/k norm weight len != head_dim");
  std::vector<float> tmp(hd);
  for (size_t g = 0; g < ng; ++g) {
    rmsnorm(row + g * hd, norm->f32(), hd, eps, tmp.data());
    memcpy(row + g * hd, tmp.data(), hd * 4);
  }
}

static const float* rope_ff(const LayerW& w, size_t* len) {
  if (w.rope_freqs && w.rope_freqs->dtype == T_F32 && w.rope_freqs->f32_len() > 0) {
    *len = w.rope_freqs->f32_len();
    return w.rope_freqs->f32();
  }
  *len = 0;
  return nullptr;
}

// The head loop of prefill_attention_layer (attention.rs:364-415): for every position p and
// query head h (KV head h / group), scores q.K[j] * scale for j in [j_min, p] (j_min = p - (w - 1)
// with a sliding window w >= 0; -inf below it), the reference softmax over p + 1 scores, then
// out[p][h] = sum_j w[j] V[j] in j order. krow / vrow give the K and V rows of (position, KV head).
template <class KRow, class VRow>
static void prefill_heads(const float* q, size_t seq, size_t n_heads, size_t n_kv, size_t hd, long sliding_window,
                          float scale, KRow krow, VRow vrow, float* out, int threads) {
  const size_t qd = n_heads * hd, group = n_heads / n_kv;
  // Keys transposed per KV head (kt[kvh][e][j], j padded to a multiple of 8) so that eight
  // scores are formed at once, lane by lane in the same e order as the scalar dot product.
  const size_t sp = (seq + 7) / 8 * 8;
  std::vector<float> kt(n_kv * hd * sp, 0.0f);
  parallel_for(n_kv, threads, [&](size_t kvh) {
    for (size_t j = 0; j < seq; ++j) {
      const float* kr = krow(j, kvh);
      for (size_t e = 0; e < hd; ++e) kt[(kvh * hd + e) * sp + j] = kr[e];
    }
  });
  typedef float v8 __attribute__((vector_size(32)));
  // one work item per query head, positions in order (each output row depends on its own
  // scores only, so the split does not change any value)
  parallel_for(n_heads, threads, [&](size_t h) {
    const size_t kvh = h / group;
    std::vector<float> sc(seq), wts(seq);
    for (size_t p = 0; p < seq; ++p) {
      size_t j_min = 0;
      if (sliding_window >= 0) {
        size_t wm1 = sliding_window > 0 ? (size_t)sliding_window - 1 : 0;
        j_min = p > wm1 ? p - wm1 : 0;
      }
      const float* qv = &q[p * qd + h * hd];
      for (size_t j = 0; j < j_min; ++j) sc[j] = -INFINITY;
      for (size_t j0 = j_min / 8 * 8; j0 <= p; j0 += 8) {
        v8 dot = {};
        for (size_t e = 0; e < hd; ++e) {
          v8 kk;
          memcpy(&kk, &kt[(kvh * hd + e) * sp + j0], 32);
          const float qe = qv[e];
          const v8 qb = {qe, qe, qe, qe, qe, qe, qe, qe};
          const v8 prod = qb * kk;
          dot = dot + prod;
        }
        for (size_t l = 0; l < 8; ++l) {
          const size_t j = j0 + l;
          if (j >= j_min && j <= p) sc[j] = dot[l] * scale;
        }
      }
      softmax(sc.data(), wts.data(), p + 1);
      float* o = &out[p * qd + h * hd];
      for (size_t j = j_min; j <= p; ++j) {
        const float wt = wts[j];
        const float* vv = vrow(j, kvh);
        for (size_t e = 0; e < hd; ++e) o[e] += wt * vv[e];
      }
    }
  });
}

// prefill_attention_layer (attention.rs:175-422); input = normed hidden [seq, hidden].
static std::vector<float> prefill_attention(Session& s, const float* input, size_t seq, size_t li) {
  const Model& m = *s.model;
  const ModelConfig& c = m.cfg;
  const LayerW& w = m.w.layers[li];
  const LayerDims& d = c.layer_dims[li];
  const LayerAttentionSpec& la = c.layer_attention[li];
  size_t qd = d.q_dim, kvd = d.kv_dim, hd = d.head_dim;
  if (qd != c.n_heads * hd) fail(E_MODEL, "prefill attention: q_dim != n_heads * head_dim");
  if (kvd != c.n_kv_heads * hd) fail(E_MODEL, "prefill attention: kv_dim != n_kv_heads * head_dim");
  KVCache& own = s.kv[li];
  if (own.n_kv_heads != c.n_kv_heads || own.head_dim != hd) fail(E_MODEL, "KVCache shape mismatch");
  long borrow = c.kv_borrow_from[li];
  if (borrow >= 0) {
    const KVCache& src = s.kv[(size_t)borrow];
    if (src.n_kv_heads != c.n_kv_heads || src.head_dim != hd) fail(E_MODEL, "borrow source KV shape mismatch");
    if (src.current_pos != seq) fail(E_MODEL, "prefill attention: borrow source cache len mismatch");
  }
  std::vector<float> q(seq * qd), k(seq * kvd, 0.0f), v(seq * kvd, 0.0f);
  matmul(input, seq, c.hidden_dim, *w.wq, q.data(), seq, qd, s.mode, s.threads);
  if (borrow < 0) {
    matmul(input, seq, c.hidden_dim, *w.wk, k.data(), seq, kvd, s.mode, s.threads);
    matmul(input, seq, c.hidden_dim, *w.wv, v.data(), seq, kvd, s.mode, s.threads);
  }
  if (c.unpack_llama_gguf_qk)
    for (size_t p = 0; p < seq; ++p) {
      unpack_qk_row(&q[p * qd], c.n_heads, hd);
      if (borrow < 0) unpack_qk_row(&k[p * kvd], c.n_kv_heads, hd);
    }
  for (size_t p = 0; p < seq; ++p) {
    head_rmsnorm(&q[p * qd], c.n_heads, hd, w.attn_q_norm, c.rms_norm_eps);
    if (borrow < 0) head_rmsnorm(&k[p * kvd], c.n_kv_heads, hd, w.attn_k_norm, c.rms_norm_eps);
  }
  if (borrow < 0 && c.family == GEMMA4)
    for (size_t p = 0; p < seq; ++p)
      for (size_t h = 0; h < c.n_kv_heads; ++h) rmsnorm_no_scale(&v[p * kvd + h * hd], hd, c.rms_norm_eps);
  size_t fl;
  const float* ff = rope_ff(w, &fl);
  for (size_t p = 0; p < seq; ++p) {
    for (size_t h = 0; h < c.n_heads; ++h)
      rope(&q[p * qd + h * hd], hd, la.rope_theta, (uint32_t)p, (uint32_t)hd, (uint32_t)la.rope_rotary_dim, ff, fl);
    if (borrow < 0)
      for (size_t h = 0; h < c.n_kv_heads; ++h)
        rope(&k[p * kvd + h * hd], hd, la.rope_theta, (uint32_t)p, (uint32_t)hd, (uint32_t)la.rope_rotary_dim, ff, fl);
  }
  if (borrow < 0)
    for (size_t p = 0; p < seq; ++p) append_kv(own, &k[p * kvd], &v[p * kvd]);
  std::vector<float> out(seq * qd, 0.0f);
  float scale = c.family == GEMMA4 ? 1.0f : 1.0f / sqrtf((float)hd);
  size_t src_idx = borrow >= 0 ? (size_t)borrow : li;
  auto krow = [&](size_t j, size_t kvh) -> const float* {
    return borrow >= 0 ? kslice(s.kv[src_idx], j, kvh) : &k[j * kvd + kvh * hd];
  };
  auto vrow = [&](size_t j, size_t kvh) -> const float* {
    return borrow >= 0 ? vslice(s.kv[src_idx], j, kvh) : &v[j * kvd + kvh * hd];
  };
  prefill_heads(q.data(), seq, c.n_heads, c.n_kv_heads, hd, la.sliding_window, scale, krow, vrow, out.data(),
                s.threads);
  std::vector<float> proj(seq * c.hidden_dim);
  matmul(out.data(), seq, qd, *w.wo, proj.data(), seq, c.hidden_dim, s.mode, s.threads);
  return proj;
}

// decode_attention_layer (attention.rs:462-655)
// The head loop of decode_attention_layer (attention.rs:608-650): per query head h (KV head
// h / group), scores q.K[j] * scale for j in [j_min, total) and -inf below j_min, the reference
// softmax over all `total` scores, then out[h] = sum_j w[j] V[j] accumulated in j order.
static void decode_heads(const float* q, const KVCache& src, size_t n_heads, size_t total, size_t j_min, float scale,
                         float* out, int threads) {
  const size_t hd = src.head_dim, group = n_heads / src.n_kv_heads;
  parallel_for(n_heads, threads, [&](size_t h) {
    size_t kvh = h / group;
    const float* qv = &q[h * hd];
    std::vector<float> sc(total, -INFINITY), wts(total, 0.0f);
    for (size_t j = j_min; j < total; ++j) {
      const float* kk = kslice(src, j, kvh);
      float dot = 0.0f;
      for (size_t e = 0; e < hd; ++e) dot += qv[e] * kk[e];
      sc[j] = dot * scale;
    }
    softmax(sc.data(), wts.data(), total);
    float* o = &out[h * hd];
    for (size_t j = j_min; j < total; ++j) {
      float wt = wts[j];
      const float* vv = vslice(src, j, kvh);
      for (size_t e = 0; e < hd; ++e) o[e] += wt * vv[e];
    }
  });
}

static std::vector<float> decode_attention(Session& s, const float* input, size_t li) {
  const Model& m = *s.model;
  const ModelConfig& c = m.cfg;
  const LayerW& w = m.w.layers[li];
  const LayerDims& d = c.layer_dims[li];
  const LayerAttentionSpec& la = c.layer_attention[li];
  size_t qd = d.q_dim, kvd = d.kv_dim, hd = d.head_dim;
  if (qd != c.n_heads * hd || kvd != c.n_kv_heads * hd) fail(E_MODEL, "decode attention: layer_dims inconsistent");
  KVCache& own = s.kv[li];
  if (own.n_kv_heads != c.n_kv_heads || own.head_dim != hd) fail(E_MODEL, "KVCache shape mismatch");
  long borrow = c.kv_borrow_from[li];
  uint32_t rope_pos;
  if (borrow >= 0) {
    size_t n = s.kv[(size_t)borrow].current_pos;
    if (n == 0) fail(E_MODEL, "decode attention: KV borrow source cache empty (rope_pos)");
    rope_pos = (uint32_t)(n - 1);
  } else {
    rope_pos = (uint32_t)own.current_pos;
  }
  std::vector<float> q(qd), k(kvd, 0.0f), v(kvd, 0.0f);
  matmul(input, 1, c.hidden_dim, *w.wq, q.data(), 1, qd, s.mode, s.threads);
  if (borrow < 0) {
    matmul(input, 1, c.hidden_dim, *w.wk, k.data(), 1, kvd, s.mode, s.threads);
    matmul(input, 1, c.hidden_dim, *w.wv, v.data(), 1, kvd, s.mode, s.threads);
  }
  if (c.unpack_llama_gguf_qk) {
    unpack_qk_row(q.data(), c.n_heads, hd);
    if (borrow < 0) unpack_qk_row(k.data(), c.n_kv_heads, hd);
  }
  head_rmsnorm(q.data(), c.n_heads, hd, w.attn_q_norm, c.rms_norm_eps);
  if (borrow < 0) head_rmsnorm(k.data(), c.n_kv_heads, hd, w.attn_k_norm, c.rms_norm_eps);
  if (borrow < 0 && c.family == GEMMA4)
    for (size_t h = 0; h < c.n_kv_heads; ++h) rmsnorm_no_scale(&v[h * hd], hd, c.rms_norm_eps);
  size_t fl;
  const float* ff = rope_ff(w, &fl);
  for (size_t h = 0; h < c.n_heads; ++h)
    rope(&q[h * hd], hd, la.rope_theta, rope_pos, (uint32_t)hd, (uint32_t)la.rope_rotary_dim, ff, fl);
  if (borrow < 0)
    for (size_t h = 0; h < c.n_kv_heads; ++h)
      rope(&k[h * hd], hd, la.rope_theta, rope_pos, (uint32_t)hd, (uint32_t)la.rope_rotary_dim, ff, fl);
  if (borrow < 0) append_kv(own, k.data(), v.data());
  size_t src_idx = borrow >= 0 ? (size_t)borrow : li;
  const KVCache& src = s.kv[src_idx];
  size_t total = src.current_pos;
  size_t j_min = 0;
  if (la.sliding_window >= 0) j_min = total > (size_t)la.sliding_window ? total - (size_t)la.sliding_window : 0;
  float scale = c.family == GEMMA4 ? 1.0f : 1.0f / sqrtf((float)hd);
  std::vector<float> out(qd, 0.0f);
  decode_heads(q.data(), src, c.n_heads, total, j_min, scale, out.data(), s.threads);
  std::vector<float> proj(c.hidden_dim);
  matmul(out.data(), 1, qd, *w.wo, proj.data(), 1, c.hidden_dim, s.mode, s.threads);
  return proj;
}

// *_attention_with_norm (attention.rs:696-940): pre-norm, attention, [Gemma post-norm], residual.
static std::vector<float> attention_with_norm(Session& s, const State& in, size_t li, bool decode) {
  const ModelConfig& c = s.model->cfg;
  const LayerW& w = s.model->w.layers[li];
  size_t seq = in.seq_len, H = in.hidden_dim;
  if (w.attn_norm->f32_len() != H) fail(E_MODEL, "attn_norm weights len != hidden_dim");
  std::vector<float> normed(seq * H);
  for (size_t p = 0; p < seq; ++p) rmsnorm(&in.hidden[p * H], w.attn_norm->f32(), H, c.rms_norm_eps, &normed[p * H]);
  std::vector<float> ao = decode ? decode_attention(s, normed.data(), li) : prefill_attention(s, normed.data(), seq, li);
  if (c.family == GEMMA4) {
    if (!w.attn_post_norm) fail(E_MODEL, "Gemma 4: missing post_attention_norm");
    std::vector<float> tmp(H);
    for (size_t p = 0; p < seq; ++p) {
      rmsnorm(&ao[p * H], w.attn_post_norm->f32(), H, c.rms_norm_eps, tmp.data());
      memcpy(&ao[p * H], tmp.data(), H * 4);
    }
  }
  std::vector<float> res(seq * H);
  residual_add(in.hidden.data(), ao.data(), res.data(), seq * H);
  return res;
}

// prefill_ffn + *_prefill_ffn_with_norm (src/layers/ffn.rs:16-167)
static std::vector<float> ffn_with_norm(Session& s, const std::vector<float>& in, size_t seq, size_t li) {
  const ModelConfig& c = s.model->cfg;
  const LayerW& w = s.model->w.layers[li];
  size_t H = c.hidden_dim, F = c.layer_dims[li].ffn_dim;
  if (w.ffn_norm->f32_len() != H) fail(E_MODEL, "ffn_norm weights len != hidden_dim");
  std::vector<float> normed(seq * H);
  for (size_t p = 0; p < seq; ++p) rmsnorm(&in[p * H], w.ffn_norm->f32(), H, c.rms_norm_eps, &normed[p * H]);
  std::vector<float> g(seq * F), u(seq * F), act(seq * F);
  matmul(normed.data(), seq, H, *w.w_gate, g.data(), seq, F, s.mode, s.threads);
  matmul(normed.data(), seq, H, *w.w_up, u.data(), seq, F, s.mode, s.threads);
  if (c.family == GEMMA4) {
    for (size_t i = 0; i < seq * F; ++i) act[i] = gelu_tanh(g[i]) * u[i];
  } else {
    swiglu(g.data(), u.data(), act.data(), seq * F);
  }
  std::vector<float> down(seq * H);
  matmul(act.data(), seq, F, *w.w_down, down.data(), seq, H, s.mode, s.threads);
  if (c.family == GEMMA4) {
    if (!w.ffn_post_norm) fail(E_MODEL, "Gemma 4: missing post_ffw_norm");
    std::vector<float> tmp(H);
    for (size_t p = 0; p < seq; ++p) {
      rmsnorm(&down[p * H], w.ffn_post_norm->f32(), H, c.rms_norm_eps, tmp.data());
      memcpy(&down[p * H], tmp.data(), H * 4);
    }
  }
  std::vector<float> res(seq * H);
  residual_add(in.data(), down.data(), res.data(), seq * H);
  return res;
}

// apply_per_layer_tail (ffn.rs:170-240)
static void ple_tail(Session& s, std::vector<float>& hidden, size_t seq, size_t li, const std::vector<float>& packed) {
  const ModelConfig& c = s.model->cfg;
  const LayerW& w = s.model->w.layers[li];
  size_t pd = c.embedding_length_per_layer, H = c.hidden_dim;
  if (pd == 0) return;
  size_t pack = c.n_layers * pd;
  if (packed.size() != seq * pack) fail(E_MODEL, "PLE packed len != seq_len * pack");
  if (!w.ple_inp_gate) fail(E_MODEL, "PLE: missing inp_gate");
  if (!w.ple_proj) fail(E_MODEL, "PLE: missing proj");
  if (!w.ple_post_norm) fail(E_MODEL, "PLE: missing post_norm");
  std::vector<float> go(seq * pd);
  matmul(hidden.data(), seq, H, *w.ple_inp_gate, go.data(), seq, pd, s.mode, s.threads);
  for (size_t p = 0; p < seq; ++p)
    for (size_t i = 0; i < pd; ++i) go[p * pd + i] = gelu_tanh(go[p * pd + i]) * packed[p * pack + li * pd + i];
  std::vector<float> po(seq * H);
  matmul(go.data(), seq, pd, *w.ple_proj, po.data(), seq, H, s.mode, s.threads);
  if (w.ple_post_norm->f32_len() != H) fail(E_MODEL, "PLE post_norm weight len mismatch");
  std::vector<float> nr(H);
  for (size_t p = 0; p < seq; ++p) {
    rmsnorm(&po[p * H], w.ple_post_norm->f32(), H, c.rms_norm_eps, nr.data());
    for (size_t i = 0; i < H; ++i) hidden[p * H + i] += nr[i];
  }
}

// apply_gemma_layer_output_scale (ffn.rs:242-278)
static void layer_scale(std::vector<float>& hidden, const Tensor* t) {
  if (!t) return;
  float sc;
  if (t->dtype == T_F32) {
    if (t->f32_len() == 0) fail(E_MODEL, "layer_output_scale: empty F32 tensor");
    sc = t->f32()[0];
  } else if (t->dtype == T_Q8_0) {
    if (t->buf.size() < Q8_0_BYTES) fail(E_MODEL, "layer_output_scale: Q8_0 buffer too small");
    float dq[32];
    dequant_q8_0(t->buf.data(), dq);
    sc = dq[0];
  } else {
    fail(E_MODEL, "layer_output_scale: unsupported dtype for scalar");
  }
  for (auto& v : hidden) v *= sc;
}

// prefill_layer_block / decode_layer_block (src/layers/block.rs:12-89)
static void layer_block(Session& s, State& st, size_t li, bool decode) {
  std::vector<float> a = attention_with_norm(s, st, li, decode);
  std::vector<float> f = ffn_with_norm(s, a, st.seq_len, li);
  if (s.model->cfg.embedding_length_per_layer > 0) ple_tail(s, f, st.seq_len, li, st.ple_packed);
  layer_scale(f, s.model->w.layers[li].layer_output_scale);
  st.hidden = std::move(f);
}

// kv_caches_for_config (attention.rs:129-135)
static void reset_kv(Session& s) {
  const ModelConfig& c = s.model->cfg;
  s.kv.clear();
  for (auto& d : c.layer_dims) {
    KVCache kv;
    kv.max_seq_len = c.context_length;
    kv.n_kv_heads = c.n_kv_heads;
    kv.head_dim = d.head_dim;
    kv.k.assign(c.context_length * c.n_kv_heads * d.head_dim, 0.0f);
    kv.v.assign(c.context_length * c.n_kv_heads * d.head_dim, 0.0f);
    s.kv.push_back(std::move(kv));
  }
}

static size_t n_blocks(const Session& s) {
  size_t n = s.model->w.layers.size();
  return s.layer_limit ? std::min(n, s.layer_limit) : n;
}

// InferenceSession::prefill -> prefill_forward (src/engine/session.rs:44-56, runtime.rs:14-32)
void session_prefill(Session& s, const uint32_t* ids, size_t n) {
  State st = embed_tokens(s, ids, n, true);
  if (s.kv.size() != s.model->w.layers.size()) fail(E_MODEL, "prefill_forward: kv_caches len != number of layers");
  for (size_t li = 0; li < n_blocks(s); ++li) layer_block(s, st, li, false);
  s.state = std::move(st);
}

// InferenceSession::decode_token -> decode_forward (session.rs:58-69, runtime.rs:37-61)
void session_decode(Session& s, uint32_t id) {
  State st = embed_tokens(s, &id, 1, false);
  for (size_t li = 0; li < n_blocks(s); ++li) layer_block(s, st, li, true);
  s.state = std::move(st);
}

// final_logits_last_token (runtime.rs:76-116): norm of the last row, LM head, optional softcap.
void session_logits(Session& s, float* out) {
  const ModelConfig& c = s.model->cfg;
  const State& st = s.state;
  if (st.seq_len == 0) fail(E_MODEL, "final_logits_last_token: empty input");
  size_t H = st.hidden_dim;
  if (s.model->w.output_norm->f32_len() != H) fail(E_MODEL, "final_logits_last_token: output_norm len != hidden_dim");
  std::vector<float> normed(H);
  rmsnorm(&st.hidden[(st.seq_len - 1) * H], s.model->w.output_norm->f32(), H, c.rms_norm_eps, normed.data());
  matmul(normed.data(), 1, H, *s.model->w.lm_head, out, 1, c.vocab_size, s.mode, s.threads);
  if (c.has_softcap)
    for (size_t i = 0; i < c.vocab_size; ++i) out[i] = c.softcap * tanhf(out[i] / c.softcap);
}

}  // namespace orc

// =============================================================================================
// C ABI used by tests (ctypes). Status = orc::Err; message via orc_last_error().
// =============================================================================================
using namespace orc;

#define ORC_TRY(...)                     \
  try {                                  \
    __VA_ARGS__;                         \
    return 0;                            \
  } catch (const Error& e) {             \
    g_last_error = e.msg;                \
    return e.code;                       \
  } catch (const std::exception& e) {    \
    g_last_error = e.what();             \
    return E_OP;                         \
  }

extern "C" {

const char* orc_last_error(void) { return g_last_error.c_str(); }

float orc_f16_to_f32(uint16_t b) { return f16_to_f32(b); }
void orc_extract_scale_min_k4(size_t j, const uint8_t* scales, uint8_t* sc, uint8_t* m) {
  extract_scale_min_k4(j, scales, sc, m);
}
// Block dequant over `nblocks` consecutive blocks.
int orc_dequantize(int ttype, const uint8_t* blocks, size_t nblocks, float* out) {
  ORC_TRY({
    if (ttype == T_F32) fail(E_TENSOR, "dequantize: F32 is not a block type");
    size_t be = block_elems(ttype), bb = block_bytes(ttype);
    for (size_t b = 0; b < nblocks; ++b) dequant_block(ttype, blocks + b * bb, out + b * be);
  })
}

int orc_matmul(int ttype, const float* a, size_t m, size_t k, const uint8_t* w, size_t wbytes, size_t n, float* out,
               int mode, int threads) {
  ORC_TRY({
    Tensor t;
    t.dtype = ttype;
    t.dims = {k, n};
    t.buf.assign(w, w + wbytes);
    matmul(a, m, k, t, out, m, n, mode, threads);
  })
}

int orc_rmsnorm(const float* in, const float* w, size_t dim, float eps, float* out) {
  ORC_TRY(rmsnorm(in, w, dim, eps, out))
}
int orc_rmsnorm_no_scale(float* x, size_t dim, float eps) { ORC_TRY(rmsnorm_no_scale(x, dim, eps)) }
int orc_rope(float* v, size_t len, float base, uint32_t pos, uint32_t head_dim, uint32_t rotary_dim, const float* ff,
             size_t ff_len) {
  ORC_TRY(rope(v, len, base, pos, head_dim, rotary_dim, ff, ff_len))
}
int orc_softmax(const float* in, float* out, size_t n) { ORC_TRY(softmax(in, out, n)) }
int orc_swiglu(const float* g, const float* u, float* out, size_t n) { ORC_TRY(swiglu(g, u, out, n)) }
float orc_gelu_tanh(float x) { return gelu_tanh(x); }
int orc_residual_add(const float* a, const float* b, float* out, size_t n) { ORC_TRY(residual_add(a, b, out, n)) }
long orc_argmax(const float* l, size_t n) { return argmax(l, n); }
long orc_sample_temperature(const float* l, size_t n, float temperature, float r) {
  return sample_temperature(l, n, temperature, r);
}
int orc_model_tokenizer_prompt(void* mp, int* add_bos, int* add_eos, uint32_t* bos, uint32_t* eos) {
  ORC_TRY({
    const ModelConfig& c = ((Model*)mp)->cfg;
    *add_bos = c.add_bos_token;
    *add_eos = c.add_eos_token;
    *bos = c.bos_token_id;
    *eos = c.eos_token_id;
  })
}
int orc_unpack_qk_row(float* row, size_t ng, size_t hd) { ORC_TRY(unpack_qk_row(row, ng, hd)) }
// decode_heads over a KVCache holding `total` positions ([total][n_kv][head_dim] k and v);
// sliding_window < 0 = none.
int orc_attention_decode(const float* q, const float* k, const float* v, size_t n_heads, size_t n_kv, size_t hd,
                         size_t total, long sliding_window, float scale, float* out) {
  ORC_TRY({
    if (n_kv == 0 || n_heads % n_kv != 0) fail(E_MODEL, "attention: n_heads % n_kv_heads != 0");
    KVCache kv;
    kv.n_kv_heads = n_kv;
    kv.head_dim = hd;
    kv.max_seq_len = kv.current_pos = total;
    kv.k.assign(k, k + total * n_kv * hd);
    kv.v.assign(v, v + total * n_kv * hd);
    size_t j_min = 0;
    if (sliding_window >= 0) j_min = total > (size_t)sliding_window ? total - (size_t)sliding_window : 0;
    std::fill(out, out + n_heads * hd, 0.0f);
    decode_heads(q, kv, n_heads, total, j_min, scale, out, 1);
  })
}

// The head loop of prefill_attention_layer over the layer's own k / v ([seq][n_kv][head_dim]),
// q [seq][n_heads][head_dim] (RoPE already applied); sliding_window < 0 = none.
int orc_attention_prefill(const float* q, const float* k, const float* v, size_t seq, size_t n_heads, size_t n_kv,
                          size_t hd, long sliding_window, float scale, float* out) {
  ORC_TRY({
    if (n_kv == 0 || n_heads % n_kv != 0) fail(E_MODEL, "attention: n_heads % n_kv_heads != 0");
    const size_t kvd = n_kv * hd;
    std::fill(out, out + seq * n_heads * hd, 0.0f);
    auto krow = [&](size_t j, size_t kvh) -> const float* { return &k[j * kvd + kvh * hd]; };
    auto vrow = [&](size_t j, size_t kvh) -> const float* { return &v[j * kvd + kvh * hd]; };
    prefill_heads(q, seq, n_heads, n_kv, hd, sliding_window, scale, krow, vrow, out,
                  (int)std::max(1u, std::thread::hardware_concurrency()));
  })
}

// ---- model / session ----
struct orc_cfg {
  int32_t family;
  uint64_t context_length, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim, ffn_dim, vocab_size;
  float rope_theta, rms_norm_eps;
  int32_t unpack_qk;
  uint64_t ple_dim;
  int32_t has_softcap;
  float softcap;
};

int orc_model_load(const char* path, void** out) { ORC_TRY(*out = model_load(path)) }
void orc_model_free(void* m) { delete (Model*)m; }
// Raw bytes, dtype and ggml dims of a loaded tensor (for tests that recompose a layer by hand).
int orc_model_tensor(void* mp, const char* name, const uint8_t** data, size_t* nbytes, int* dtype, uint64_t* ne0,
                     uint64_t* ne1) {
  ORC_TRY({
    const Tensor* t = ((Model*)mp)->gguf.get(name);
    if (!t) fail(E_MODEL, std::string("no tensor ") + name);
    *data = t->buf.data();
    *nbytes = t->buf.size();
    *dtype = t->dtype;
    *ne0 = t->dims.empty() ? 0 : t->dims[0];
    *ne1 = t->dims.size() > 1 ? t->dims[1] : 1;
  })
}
int orc_model_config(void* mp, orc_cfg* o) {
  ORC_TRY({
    const ModelConfig& c = ((Model*)mp)->cfg;
    o->family = c.family;
    o->context_length = c.context_length;
    o->hidden_dim = c.hidden_dim;
    o->n_layers = c.n_layers;
    o->n_heads = c.n_heads;
    o->n_kv_heads = c.n_kv_heads;
    o->head_dim = c.head_dim;
    o->ffn_dim = c.ffn_dim;
    o->vocab_size = c.vocab_size;
    o->rope_theta = c.rope_theta;
    o->rms_norm_eps = c.rms_norm_eps;
    o->unpack_qk = c.unpack_llama_gguf_qk;
    o->ple_dim = c.embedding_length_per_layer;
    o->has_softcap = c.has_softcap;
    o->softcap = c.softcap;
  })
}
// Per-layer attention spec: sliding window (-1 = none), theta, rotary dim, kv borrow (-1 = none).
int orc_model_layer_spec(void* mp, size_t li, long* window, float* theta, uint64_t* rot, long* borrow,
                         uint64_t* head_dim, uint64_t* ffn_dim) {
  ORC_TRY({
    const ModelConfig& c = ((Model*)mp)->cfg;
    if (li >= c.n_layers) fail(E_MODEL, "layer index out of range");
    *window = c.layer_attention[li].sliding_window;
    *theta = c.layer_attention[li].rope_theta;
    *rot = c.layer_attention[li].rope_rotary_dim;
    *borrow = c.kv_borrow_from[li];
    *head_dim = c.layer_dims[li].head_dim;
    *ffn_dim = c.layer_dims[li].ffn_dim;
  })
}

int orc_session_new(void* mp, int mode, int threads, void** out) {
  ORC_TRY({
    Session* s = new Session();
    s->model = (Model*)mp;
    s->mode = mode;
    s->threads = threads > 0 ? threads : (int)std::max(1u, std::thread::hardware_concurrency());
    reset_kv(*s);
    *out = s;
  })
}
void orc_session_free(void* s) { delete (Session*)s; }
// Timing aid only: run just the first n blocks per step (0 = all). Not a reference behaviour.
void orc_session_set_layer_limit(void* s, size_t n) { ((Session*)s)->layer_limit = n; }
int orc_session_reset(void* s) { ORC_TRY(reset_kv(*(Session*)s)) }
int orc_session_prefill(void* s, const uint32_t* ids, size_t n) { ORC_TRY(session_prefill(*(Session*)s, ids, n)) }
int orc_session_decode(void* s, uint32_t id) { ORC_TRY(session_decode(*(Session*)s, id)) }
int orc_session_logits(void* s, float* out) { ORC_TRY(session_logits(*(Session*)s, out)) }
// Copy the last state's hidden rows [seq, hidden] (for layer-level parity checks).
int orc_session_hidden(void* sp, float* out, size_t cap, uint64_t* seq) {
  ORC_TRY({
    Session* s = (Session*)sp;
    *seq = s->state.seq_len;
    if (cap < s->state.hidden.size()) fail(E_OP, "hidden buffer too small");
    memcpy(out, s->state.hidden.data(), s->state.hidden.size() * 4);
  })
}
uint64_t orc_session_kv_len(void* sp, size_t layer) { return ((Session*)sp)->kv[layer].current_pos; }
// Copy K or V rows [0, n) of a layer as f32 [n][n_kv][head_dim].
int orc_session_kv(void* sp, size_t layer, int which_v, float* out, size_t n) {
  ORC_TRY({
    Session* s = (Session*)sp;
    KVCache& kv = s->kv[layer];
    if (n > kv.current_pos) fail(E_KVCACHE, "position out of bounds");
    size_t e = kv.n_kv_heads * kv.head_dim;
    memcpy(out, (which_v ? kv.v : kv.k).data(), n * e * 4);
  })
}

}  // extern "C"
