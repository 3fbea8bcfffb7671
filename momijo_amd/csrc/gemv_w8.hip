// Skinny-M W8A16 Linear (decode): y[m,n] = bf16(epi((x[m,:] . Q[n,:]) *
// scales[n] + bias[n])) for M <= 8, int8 weights Q [N,K] streamed once.
//
// The kernel is HBM-bound (1 byte of weight per multiply-add), so the design
// goal is bytes in flight: each wave owns RPW consecutive weight rows and
// issues all of its 16-byte weight loads for a K block before doing any math;
// lane l covers K chunks l, l+64, ... of 16 int8, so a wave reads 1 KiB
// contiguous per instruction.  x (bf16, a few KiB, L2-resident) is loaded
// per chunk and widened to fp32 once for all RPW rows.  Each int8 is widened
// exactly to fp32 and multiplied with fp32 accumulation; a 64-lane butterfly
// reduction finishes each dot, then scale, bias and the activation are
// applied in fp32 and the result is rounded to bf16.
#include "common.h"
#include "launch.h"

namespace mj {

template <int MB, int RPW, int CPL>
__global__ __launch_bounds__(256) void gemv_w8a16_kernel(const uint16_t *__restrict__ x,
                                                         const int8_t *__restrict__ Q,
                                                         const float *__restrict__ scales,
                                                         const float *__restrict__ bias, int epi,
                                                         uint16_t *__restrict__ y, int M, int N,
                                                         int K) {
  const int lane = threadIdx.x & 63;
  const int wave_id = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int row0 = wave_id * RPW;
  if (row0 >= N) return;
  const int nchunks = K >> 4;  // 16-element chunks per row

  float acc[RPW][MB];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[r][m] = 0.0f;

  for (int cb = 0; cb < nchunks; cb += 64 * CPL) {
    // issue every weight load of this K block first
    uint4 q[RPW][CPL];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const int row = row0 + r < N ? row0 + r : N - 1;
      const uint4 *qrow = (const uint4 *)(Q + (size_t)row * K);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int ch = cb + c * 64 + lane;
        q[r][c] = ch < nchunks ? load_nt16(qrow + ch) : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ch = cb + c * 64 + lane;
      if (ch >= nchunks) continue;
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        if (m >= M) break;
        const uint4 *xr = (const uint4 *)(x + (size_t)m * K + ch * 16);
        const uint4 x0 = xr[0], x1 = xr[1];
        const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        float xf[16];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          xf[2 * e] = __uint_as_float(xw[e] << 16);
          xf[2 * e + 1] = __uint_as_float(xw[e] & 0xFFFF0000u);
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          const uint32_t qw[4] = {q[r][c].x, q[r][c].y, q[r][c].z, q[r][c].w};
          float a = acc[r][m];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int32_t v = (int32_t)qw[e];
            a += xf[4 * e + 0] * (float)((v << 24) >> 24);
            a += xf[4 * e + 1] * (float)((v << 16) >> 24);
            a += xf[4 * e + 2] * (float)((v << 8) >> 24);
            a += xf[4 * e + 3] * (float)(v >> 24);
          }
          acc[r][m] = a;
        }
      }
    }
  }

#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int n = row0 + r;
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      const float s = wave_sum(acc[r][m]);
      if (lane == r * MB + m && n < N && m < M) {
        float v;
        {
#pragma clang fp contract(off)
          v = s * scales[n];
          if (bias) v = v + bias[n];
        }
        v = apply_epi(epi, v);
        y[(size_t)m * N + n] = (uint16_t)f32_to_bf16_bits(v);
      }
    }
  }
}

template <int MB>
static hipError_t launch_mb(const uint16_t *x, const int8_t *Q, const float *scales,
                            const float *bias, int epi, uint16_t *y, int64_t M, int64_t N,
                            int64_t K, hipStream_t stream) {
  constexpr int RPW = MB <= 2 ? 2 : 1;
  constexpr int CPL = 4;
  const int64_t waves = (N + RPW - 1) / RPW;
  const unsigned blocks = (unsigned)((waves + 3) / 4);
  hipLaunchKernelGGL((gemv_w8a16_kernel<MB, RPW, CPL>), dim3(blocks), dim3(256), 0, stream, x, Q,
                     scales, bias, epi, y, (int)M, (int)N, (int)K);
  return hipGetLastError();
}

hipError_t launch_gemv_w8a16(const uint16_t *x, const int8_t *Q, const float *scales,
                             const float *bias, int epi, uint16_t *y, int64_t M, int64_t N,
                             int64_t K, hipStream_t stream) {
  if (M <= 1) return launch_mb<1>(x, Q, scales, bias, epi, y, M, N, K, stream);
  if (M <= 2) return launch_mb<2>(x, Q, scales, bias, epi, y, M, N, K, stream);
  if (M <= 4) return launch_mb<4>(x, Q, scales, bias, epi, y, M, N, K, stream);
  return launch_mb<8>(x, Q, scales, bias, epi, y, M, N, K, stream);
}

}  // namespace mj
