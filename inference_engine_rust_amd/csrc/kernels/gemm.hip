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

void launch_gemm(int dt, const void* w, const float* a, int M, int K, int N, float* out, const float* resid,
                 hipStream_t st) {
  if (gemm_q_ok(dt, w, K) && (reinterpret_cast<uintptr_t>(a) & 15) == 0) {
    // scale-factored K-quant GEMM: stream-ordered scratch for the fp16 pair and the per-32 sums;
    // Q6_K is first regrouped (the layout the model path keeps beside the native tensor), which
    // the wave-tiled matrix-core kernel reads
    const size_t n = (size_t)M * K;
    const bool q6r = dt == DT_Q6K && K % QK_K == 0;
    const size_t wr = q6r ? (size_t)N * q6r_row_bytes((size_t)K / QK_K) : 0;
    const size_t xbytes = (n * 2 * sizeof(__half) + (n / 32 + 64) * sizeof(float) + 255) / 256 * 256;
    const size_t pbytes = ((size_t)M * N * sizeof(float) + 255) / 256 * 256;  // split-K partial
    void* buf = nullptr;
    check_hip(hipMallocAsync(&buf, xbytes + pbytes + wr, st), "hipMallocAsync");
    __half* xh = static_cast<__half*>(buf);
    float* xs = reinterpret_cast<float*>(xh + 2 * n);
    launch_split_f16(a, n, xh, xh + n, st);
    launch_block_sums(a, M, K, xs, st);
    const void* wq = w;
    int wdt = dt;
    if (q6r) {
      void* r = static_cast<char*>(buf) + xbytes + pbytes;
      launch_repack_q6k(w, K, N, r, st);
      wq = r;
      wdt = DT_Q6K_R;
    }
    GemmQSeg seg{wq, out, N};
    launch_gemm_q(wdt, &seg, 1, xh, xh + n, xs, M, K, resid, st,
                  reinterpret_cast<float*>(static_cast<char*>(buf) + xbytes));
    check_hip(hipFreeAsync(buf, st), "hipFreeAsync");
    return;
  }
  if (gemm_mfma_ok(dt, w, K, N) && (reinterpret_cast<uintptr_t>(a) & 15) == 0) {
    // stream-ordered scratch for the fp16 activation pair
    const size_t n = (size_t)M * K;
    void* buf = nullptr;
    check_hip(hipMallocAsync(&buf, n * 2 * sizeof(__half), st), "hipMallocAsync");
    __half* xh = static_cast<__half*>(buf);
    launch_split_f16(a, n, xh, xh + n, st);
    launch_gemm_mfma(dt, w, xh, xh + n, M, K, N, out, resid, st);
    check_hip(hipFreeAsync(buf, st), "hipFreeAsync");
    return;
  }
  dim3 grid((N + GBN - 1) / GBN, (M + GBM - 1) / GBM);
  hipLaunchKernelGGL(gemm_simt_kernel, grid, dim3(256), 0, st, dt, (const uint8_t*)w, a, M, K, N, out, resid);
}

}  // namespace iek
