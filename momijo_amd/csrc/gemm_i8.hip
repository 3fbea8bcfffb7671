// int8 x int8 -> int32 GEMM on gfx950 int8 MFMA (v_mfma_i32_32x32x32_i8):
// matmul_i8_i8_to_i32 (learn/api/functional.mojo:249-279) with the weight
// given in its stored layout w_q [N,K], optionally with the dequantize of
// QuantLinear (learn/nn/layers.mojo:1681-1685) fused into the epilogue.
// Integer products and sums are exact, so the result is bit-identical to
// the reference's i-j-p loop in any summation order (|acc| <= 127*128*K).
//
// 128x128 tile per 256-thread workgroup, 64-wide K stages of int8 in LDS
// (rows padded to 80 B so 16-byte fragment reads of 16 lanes hit distinct
// banks), double-buffered through registers.  It only runs where the
// one-wave-per-SIMD kernel (gemm_i8_w4_kernel in gemm_nt.hip, 256 x 256 or
// 256 x 128 tiles) cannot address a tile with 32-bit offsets (256 K >= 2^31):
// that kernel is faster at every measured shape.  MI355X, bit-identical
// outputs, settled A/B timed alternately, this kernel against it: 4096^3
// 114.8 / 59.7 us, 3072 x 4096 x 4096 75.6 / 53.7, 2048 x 4096 x 4096 58.4 /
// 35.3, 1024 x 4096 x 4096 47.3 / 29.9, 512 x 11008 x 4096 53.2 / 33.3,
// 512 x 4096 x 11008 109.5 / 65.1, 1024 x 1024 x 4096 40.7 / 28.4, 1000 x
// 3000 x 1040 20.3 / 16.4, 300 x 520 x 4112 39.7 / 25.1, 512 x 512 x 4096
// 39.2 / 24.6.
#include "common.h"
#include "launch.h"

namespace mj {

constexpr int kIBM = 128, kIBN = 128, kIBK = 64;
constexpr int kILds = kIBK + 16;  // bytes per LDS row

__global__ __launch_bounds__(256) void gemm_i8_kernel(const int8_t *__restrict__ A,
                                                      const int8_t *__restrict__ B,
                                                      int32_t *__restrict__ C,
                                                      float *__restrict__ Y, float sf,
                                                      const float *__restrict__ bias, int M,
                                                      int N, int K) {
  __shared__ __attribute__((aligned(16))) int8_t As[2][kIBM * kILds];
  __shared__ __attribute__((aligned(16))) int8_t Bs[2][kIBN * kILds];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_m = (M + kIBM - 1) / kIBM, tiles_n = (N + kIBN - 1) / kIBN;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, 4, tm, tn);
  const int m0 = tm * kIBM, n0 = tn * kIBN;

  // 4 chunks of 16 B per 64-byte row: thread -> (row t/4 + 64 i, chunk t%4)
  const int c = tid & 3, r0 = tid >> 2;
  uint4 ra[2], rb[2];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int m = m0 + r0 + 64 * i, n = n0 + r0 + 64 * i, k = k0 + c * 16;
      ra[i] = (m < M && k < K) ? *(const uint4 *)(A + (size_t)m * K + k) : make_uint4(0, 0, 0, 0);
      rb[i] = (n < N && k < K) ? *(const uint4 *)(B + (size_t)n * K + k) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      *(uint4 *)(&As[buf][(r0 + 64 * i) * kILds + c * 16]) = ra[i];
      *(uint4 *)(&Bs[buf][(r0 + 64 * i) * kILds + c * 16]) = rb[i];
    }
  };

  i32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  const int nk = (K + kIBK - 1) / kIBK;
  load(0);
  store(0);
  __syncthreads();
  const int fr = lane & 31, fk = (lane >> 5) * 16;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load((kt + 1) * kIBK);
#pragma unroll
    for (int ks = 0; ks < kIBK; ks += 32) {
      i32x4 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *(const i32x4 *)(&As[buf][(wm * 64 + i * 32 + fr) * kILds + ks + fk]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = *(const i32x4 *)(&Bs[buf][(wn * 64 + j * 32 + fr) * kILds + ks + fk]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wn * 64 + j * 32 + (lane & 31);
    if (n >= N) continue;
    const float bb = Y ? bias[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m >= M) continue;
        if (Y) {
#pragma clang fp contract(off)
          const float v = (float)acc[i][j][r] * sf;
          Y[(size_t)m * N + n] = v + bb;
        } else {
          C[(size_t)m * N + n] = acc[i][j][r];
        }
      }
  }
}

hipError_t launch_gemm_i8_t128(const int8_t *A, const int8_t *B, int32_t *C, float *y, float sf,
                               const float *b, int64_t M, int64_t N, int64_t K,
                               hipStream_t stream) {
  const int tiles = (int)((M + kIBM - 1) / kIBM) * (int)((N + kIBN - 1) / kIBN);
  hipLaunchKernelGGL(gemm_i8_kernel, dim3(tiles), dim3(256), 0, stream, A, B, C, y, sf, b, (int)M,
                     (int)N, (int)K);
  return hipGetLastError();
}

hipError_t launch_gemm_i8(const int8_t *A, const int8_t *B, int32_t *C, float *y, float sf,
                          const float *b, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  if (256 * K < ((int64_t)1 << 31) && K % 16 == 0 && (((uintptr_t)A | (uintptr_t)B) & 15) == 0)
    return launch_gemm_i8_w4(A, B, C, y, sf, b, M, N, K, stream);
  return launch_gemm_i8_t128(A, B, C, y, sf, b, M, N, K, stream);
}

// Scalar int8 GEMM, one thread per output, for layouts the MFMA kernel does
// not take: literal = 1 is the reference's indexing bt._data[p*N + j]
// (functional.mojo:274), B read as a row-major [K,N] matrix; literal = 0 is
// the intended w_q [N,K] read for K not a multiple of 16 or unaligned data.
__global__ __launch_bounds__(256) void gemm_i8_scalar_kernel(const int8_t *__restrict__ A,
                                                             const int8_t *__restrict__ B,
                                                             int32_t *__restrict__ C,
                                                             float *__restrict__ Y, float sf,
                                                             const float *__restrict__ bias,
                                                             int64_t M, int64_t N, int64_t K,
                                                             int literal) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= M * N) return;
  const int64_t i = t / N, j = t - i * N;
  const int64_t sp = literal ? N : 1, sj = literal ? 1 : K;
  int32_t acc = 0;
  for (int64_t p = 0; p < K; ++p) acc += (int32_t)A[i * K + p] * (int32_t)B[p * sp + j * sj];
  if (Y) {
#pragma clang fp contract(off)
    const float v = (float)acc * sf;
    Y[t] = v + bias[j];
  } else {
    C[t] = acc;
  }
}

hipError_t launch_gemm_i8_scalar(const int8_t *A, const int8_t *B, int32_t *C, float *y,
                                 float sf, const float *b, int64_t M, int64_t N, int64_t K,
                                 bool literal, hipStream_t stream) {
  const unsigned blocks = (unsigned)((M * N + 255) / 256);
  hipLaunchKernelGGL(gemm_i8_scalar_kernel, dim3(blocks), dim3(256), 0, stream, A, B, C, y, sf,
                     b, M, N, K, literal ? 1 : 0);
  return hipGetLastError();
}

}  // namespace mj
