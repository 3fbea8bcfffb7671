// Skinny-M W8A16 Linear (decode): y[m,n] = bf16(epi((x[m,:] . Q[n,:]) *
// scales[n] + bias[n])) for M <= 8, int8 weights Q [N,K] streamed once.
//
// The kernel is HBM-bound (1 byte of weight per multiply-add), so the design
// goal is bytes in flight: each wave owns RPW consecutive weight rows and
// issues all of its 16-byte weight loads for a K block before doing any math;
// lane l covers K chunks l, l+64, ... of 16 int8, so a wave reads 1 KiB
// contiguous per instruction.  The weight loads are raw buffer loads over the
// wave's rows (chunks past K and rows past N read zero), so every wave issues
// exactly RPW * CPL of them per block, branch-free, with the nontemporal bit.
//
// x (bf16, M*K elements) is staged once per workgroup in LDS when it fits
// (XLDS): its direct-to-LDS loads are issued before the weight loads, and
// since the vector-memory counter retires in order, waiting until only the
// RPW*CPL weight loads are outstanding means exactly that x has landed; the
// weight stream therefore starts at once instead of behind an x round trip.
// Larger x is read per chunk from L2.  Each int8 is widened exactly to fp32
// (one SDWA convert) and multiplied with fp32 accumulation; a DPP reduction
// finishes each dot, then scale, bias and the activation are applied in fp32
// and the result is rounded to bf16.
#include "common.h"
#include "launch.h"

namespace mj {

constexpr int kGemvXsElems = 8192;  // 16 KiB of LDS per workgroup for staged x

typedef __attribute__((address_space(3))) void gemv_lds_void;

template <int MB, int RPW, int CPL, bool XLDS>
__global__ __launch_bounds__(256) void gemv_w8a16_kernel(const uint16_t *__restrict__ x,
                                                         const int8_t *__restrict__ Q,
                                                         const float *__restrict__ scales,
                                                         const float *__restrict__ bias, int epi,
                                                         uint16_t *__restrict__ y, int M, int N,
                                                         int K) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[XLDS ? kGemvXsElems : 8];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * 4 + wave) * RPW;
  const int nchunks = K >> 4;  // 16-element chunks per row
  const int rows = N - row0 < RPW ? N - row0 : RPW;  // <= 0 for trailing waves
  const __amdgpu_buffer_rsrc_t rQ =
      make_rsrc(Q + (size_t)(row0 < N ? row0 : 0) * K, rows > 0 ? (int64_t)rows * K : 0);

  if constexpr (XLDS) {
    // M*K bf16 in 1-KiB blocks, block i by wave i % 4
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (int64_t)M * K * 2);
    const int blocks = (M * K * 2 + 1023) / 1024;
    for (int i = wave; i < blocks; i += 4)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (gemv_lds_void *)(xs + i * 512), 16,
                                               (uint32_t)(i * 1024 + lane * 16), 0, 0, 0);
    // the wait below counts on the x loads being issued before the weight
    // loads: keep the scheduler from moving anything across this point
    __builtin_amdgcn_sched_barrier(0);
  }

  // the output lane of (row r, x row m) is r * MB + m: it fetches that row's
  // scale and bias now, so no dependent load sits on the wave's tail (these
  // loads precede the weight loads, which keeps the x-landed wait below exact)
  const int my_r = lane / MB < RPW ? lane / MB : 0;
  const int my_n = row0 + my_r < N ? row0 + my_r : N - 1;
  const float my_s = scales[my_n];
  const float my_b = bias ? bias[my_n] : 0.0f;

  float acc[RPW][MB];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[r][m] = 0.0f;

  uint4 q[RPW][CPL];
  auto issue = [&](int cb) {
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int ch = cb + c * 64 + lane;
        const uint32_t off = ch < nchunks ? (uint32_t)(r * K + ch * 16) : kOobOffset;
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rQ, off, 0, 2 /* nt */);
        q[r][c] = make_uint4(v[0], v[1], v[2], v[3]);
      }
  };
  issue(0);
  if constexpr (XLDS) {
    // the x loads were issued first: once at most the weight loads are
    // outstanding, this wave's x blocks have landed
    __builtin_amdgcn_s_waitcnt(0x0F70 | ((RPW * CPL) & 0xF) | (((RPW * CPL) >> 4) << 14));
    __syncthreads();
  }
  if (rows <= 0) return;

  for (int cb = 0; cb < nchunks; cb += 64 * CPL) {
    if (cb > 0) issue(cb);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ch = cb + c * 64 + lane;
      if (ch >= nchunks) continue;
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        if (m >= M) break;
        uint4 x0, x1;
        if constexpr (XLDS) {
          x0 = *(const uint4 *)(xs + m * K + ch * 16);
          x1 = *(const uint4 *)(xs + m * K + ch * 16 + 8);
        } else {
          const uint4 *xr = (const uint4 *)(x + (size_t)m * K + ch * 16);
          x0 = xr[0];
          x1 = xr[1];
        }
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
      const float s = wave_sum_dpp(acc[r][m]);
      if (lane == r * MB + m && n < N && m < M) {
        float v;
        {
#pragma clang fp contract(off)
          v = s * my_s;
          if (bias) v = v + my_b;
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
  // a wave's weight rows (RPW * K bytes) are addressed by 32-bit buffer offsets
  if ((int64_t)RPW * K >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
  if (M * K <= kGemvXsElems)
    hipLaunchKernelGGL((gemv_w8a16_kernel<MB, RPW, CPL, true>), dim3(blocks), dim3(256), 0,
                       stream, x, Q, scales, bias, epi, y, (int)M, (int)N, (int)K);
  else
    hipLaunchKernelGGL((gemv_w8a16_kernel<MB, RPW, CPL, false>), dim3(blocks), dim3(256), 0,
                       stream, x, Q, scales, bias, epi, y, (int)M, (int)N, (int)K);
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
