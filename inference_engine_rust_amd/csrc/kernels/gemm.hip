// Prefill matmul (M > 1): out[m, n] = sum_k a[m, k] * W(k, n) with W in its native GGUF blocks.
// Tiled SIMT kernel: a 64x64 output tile per 256-thread block; each 32-wide K slab of W is
// dequantised into LDS once and reused by all 64 rows of the tile.
#include "common.cuh"
#include "../iek_internal.h"

namespace iek {

constexpr int GBM = 64, GBN = 64, GBK = 32;

__global__ __launch_bounds__(256) void gemm_simt_kernel(int dt, const uint8_t* __restrict__ w,
                                                        const float* __restrict__ a, int M, int K, int N,
                                                        float* __restrict__ out, const float* __restrict__ resid) {
  __shared__ float As[GBK][GBM + 4];
  __shared__ float Ws[GBK][GBN + 4];
  const int tid = threadIdx.x;
  const int m0 = blockIdx.y * GBM, n0 = blockIdx.x * GBN;
  const int tm = (tid / 16) * 4, tn = (tid % 16) * 4;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += GBK) {
    for (int e = tid; e < GBM * GBK; e += 256) {
      int r = e / GBK, c = e % GBK;
      int gm = m0 + r, gk = k0 + c;
      As[c][r] = (gm < M && gk < K) ? a[(size_t)gm * K + gk] : 0.f;
    }
    for (int e = tid; e < GBN * GBK; e += 256) {
      int cn = e / GBK, c = e % GBK;
      int gn = n0 + cn, gk = k0 + c;
      Ws[c][cn] = (gn < N && gk < K) ? flat_elem(dt, w, (size_t)gk + (size_t)gn * K) : 0.f;
    }
    __syncthreads();
#pragma unroll 8
    for (int kk = 0; kk < GBK; ++kk) {
      float av[4], wv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        av[i] = As[kk][tm + i];
        wv[i] = Ws[kk][tn + i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += av[i] * wv[j];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int gm = m0 + tm + i, gn = n0 + tn + j;
      if (gm < M && gn < N) {
        float v = acc[i][j];
        if (resid) v = resid[(size_t)gm * N + gn] + v;
        out[(size_t)gm * N + gn] = v;
      }
    }
}

void launch_gemm_f32(int dt, const void* w, const float* a, int M, int K, int N, float* out, const float* resid,
                     hipStream_t st) {
  dim3 grid((N + GBN - 1) / GBN, (M + GBM - 1) / GBM);
  hipLaunchKernelGGL(gemm_simt_kernel, grid, dim3(256), 0, st, dt, (const uint8_t*)w, a, M, K, N, out, resid);
}

// Op-level matmul (M > 1). On the matrix cores the activation enters as an fp16 (hi, lo) pair;
// each row is first scaled by a power of two that keeps its values and per-32 sums inside the
// pair's range (launch_split_scaled), and the output row is scaled back afterwards, so any finite
// f32 activation is taken.
void launch_gemm(int dt, const void* w, const float* a, int M, int K, int N, float* out, const float* resid,
                 hipStream_t st) {
  const bool kq = gemm_q_ok(dt, w, K) && (reinterpret_cast<uintptr_t>(a) & 15) == 0;
  const bool mf = !kq && gemm_mfma_ok(dt, w, K, N) && (reinterpret_cast<uintptr_t>(a) & 15) == 0 && K % 32 == 0;
  if (resid || !(kq || mf)) {
    launch_gemm_f32(dt, w, a, M, K, N, out, resid, st);
    return;
  }
  // stream-ordered scratch: the fp16 pair, the per-32 sums, the row factors, a split-K partial and
  // (Q6_K) the regrouped weights
  const size_t n = (size_t)M * K;
  const bool q6r = kq && dt == DT_Q6K && K % QK_K == 0;
  const size_t wr = q6r ? (size_t)N * q6r_row_bytes((size_t)K / QK_K) : 0;
  const size_t xbytes = (n * 2 * sizeof(__half) + (n / 32 + 64) * sizeof(float) + 255) / 256 * 256;
  const size_t ibytes = ((size_t)M * sizeof(float) + 255) / 256 * 256;
  const size_t pbytes = kq ? ((size_t)M * N * sizeof(float) + 255) / 256 * 256 : 0;  // split-K partial
  void* buf = nullptr;
  check_hip(hipMallocAsync(&buf, xbytes + ibytes + pbytes + wr, st), "hipMallocAsync");
  char* base = static_cast<char*>(buf);
  __half* xh = reinterpret_cast<__half*>(base);
  float* xs = reinterpret_cast<float*>(xh + 2 * n);
  float* inv = reinterpret_cast<float*>(base + xbytes);
  launch_split_scaled(a, M, K, xh, xh + n, xs, inv, st);
  if (kq) {
    const void* wq = w;
    int wdt = dt;
    if (q6r) {
      void* r = base + xbytes + ibytes + pbytes;
      launch_repack_q6k(w, K, N, r, st);
      wq = r;
      wdt = DT_Q6K_R;
    }
    GemmQSeg seg{wq, out, N};
    launch_gemm_q(wdt, &seg, 1, xh, xh + n, xs, M, K, nullptr, st, reinterpret_cast<float*>(base + xbytes + ibytes));
  } else {
    launch_gemm_mfma(dt, w, xh, xh + n, M, K, N, out, nullptr, st);
  }
  launch_row_scale(out, M, N, inv, st);
  check_hip(hipFreeAsync(buf, st), "hipFreeAsync");
}

}  // namespace iek
