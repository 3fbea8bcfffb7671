// fp32 engine on gfx950: the matmul / Linear of momijo's Float32 tensor
// engine (tensor/broadcast.mojo:1543-1684, learn/nn/layers.mojo:383-433).
//
// gemm_f32_kernel: C = epi(A @ B + bias) on v_mfma_f32_16x16x4f32 (full fp32
// products), 64x64 tile per 256-thread workgroup, 16-wide K stages staged
// through LDS (k-major, padded).  Operands come as (pointer, row stride,
// column stride), which covers the reference's zero-copy transpose views;
// the loader walks whichever dimension has unit stride with consecutive
// lanes so global reads stay coalesced.
#include "common.h"
#include "launch.h"

namespace mj {

constexpr int kFBM = 64, kFBN = 64, kFBK = 16;

__global__ __launch_bounds__(256) void gemm_f32_kernel(int M, int N, int K, const float *__restrict__ A,
                                                       int64_t sAm, int64_t sAk,
                                                       const float *__restrict__ B, int64_t sBk,
                                                       int64_t sBn, const float *__restrict__ bias,
                                                       int epi, float *__restrict__ C,
                                                       int64_t ldc) {
  __shared__ float As[2][kFBK][kFBM + 4];
  __shared__ float Bs[2][kFBK][kFBN + 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_n = (N + kFBN - 1) / kFBN;
  const int m0 = (blockIdx.x / tiles_n) * kFBM;
  const int n0 = (blockIdx.x % tiles_n) * kFBN;

  const bool a_k_fast = (sAk == 1);
  const bool b_n_fast = (sBn == 1) || (sBk != 1);

  float ra[4], rb[4];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int m, k;
      if (a_k_fast) { k = tid & 15; m = (tid >> 4) + 16 * i; }
      else          { m = tid & 63; k = (tid >> 6) + 4 * i; }
      const int gm = m0 + m, gk = k0 + k;
      ra[i] = (gm < M && gk < K) ? A[(int64_t)gm * sAm + (int64_t)gk * sAk] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int n, k;
      if (b_n_fast) { n = tid & 63; k = (tid >> 6) + 4 * i; }
      else          { k = tid & 15; n = (tid >> 4) + 16 * i; }
      const int gn = n0 + n, gk = k0 + k;
      rb[i] = (gn < N && gk < K) ? B[(int64_t)gk * sBk + (int64_t)gn * sBn] : 0.0f;
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int m, k;
      if (a_k_fast) { k = tid & 15; m = (tid >> 4) + 16 * i; }
      else          { m = tid & 63; k = (tid >> 6) + 4 * i; }
      As[buf][k][m] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int n, k;
      if (b_n_fast) { n = tid & 63; k = (tid >> 6) + 4 * i; }
      else          { k = tid & 15; n = (tid >> 4) + 16 * i; }
      Bs[buf][k][n] = rb[i];
    }
  };

  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = (K + kFBK - 1) / kFBK;
  load(0);
  store(0);
  __syncthreads();
  const int fr = lane & 15, fk = lane >> 4;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load((kt + 1) * kFBK);
#pragma unroll
    for (int kk = 0; kk < kFBK; kk += 4) {
      float a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = As[buf][kk + fk][wm * 32 + i * 16 + fr];
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = Bs[buf][kk + fk][wn * 32 + j * 16 + fr];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }

  // 16x16 output layout: lane l holds rows 4*(l/16) + r, column l%16.
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wn * 32 + j * 16 + (lane & 15);
    if (n >= N) continue;
    const float bb = bias ? bias[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + r;
        if (m < M) {
          float v = acc[i][j][r];
          if (bias) {
#pragma clang fp contract(off)
            v = v + bb;
          }
          C[(int64_t)m * ldc + n] = apply_epi(epi, v);
        }
      }
  }
}

hipError_t launch_gemm_f32(int64_t M, int64_t N, int64_t K, const float *A, int64_t sAm,
                           int64_t sAk, const float *B, int64_t sBk, int64_t sBn,
                           const float *bias, int epi, float *C, int64_t ldc,
                           hipStream_t stream) {
  const int tiles = (int)((M + kFBM - 1) / kFBM) * (int)((N + kFBN - 1) / kFBN);
  hipLaunchKernelGGL(gemm_f32_kernel, dim3(tiles), dim3(256), 0, stream, (int)M, (int)N, (int)K,
                     A, sAm, sAk, B, sBk, sBn, bias, epi, C, ldc);
  return hipGetLastError();
}

// y[m] = sum_n A[m,n] x[n]: one wave per row, lanes stride over n.
__global__ __launch_bounds__(256) void matvec_f32_kernel(int M, int N, const float *__restrict__ A,
                                                         int64_t sAm, int64_t sAn,
                                                         const float *__restrict__ x, int64_t sx,
                                                         float *__restrict__ y) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const float *a = A + (int64_t)row * sAm;
  float acc = 0.0f;
  for (int n = lane; n < N; n += 64) acc += a[(int64_t)n * sAn] * x[(int64_t)n * sx];
  acc = wave_sum(acc);
  if (lane == 0) y[row] = acc;
}

hipError_t launch_matvec_f32(int64_t M, int64_t N, const float *A, int64_t sAm, int64_t sAn,
                             const float *x, int64_t sx, float *y, hipStream_t stream) {
  hipLaunchKernelGGL(matvec_f32_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, stream,
                     (int)M, (int)N, A, sAm, sAn, x, sx, y);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void activation_f32_kernel(int epi, const float *x, float *y,
                                                             int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = apply_epi(epi, x[i]);
}

hipError_t launch_activation_f32(int epi, const float *x, float *y, int64_t n,
                                 hipStream_t stream) {
  int64_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(activation_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, epi,
                     x, y, n);
  return hipGetLastError();
}

}  // namespace mj
