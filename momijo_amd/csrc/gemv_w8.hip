// Skinny-M W8A16 Linear (decode): y[m,n] = bf16(epi((x[m,:] . Q[n,:]) *
// scales[n] + bias[n])) for M <= 16, int8 weights Q [N,K] streamed once:
// the streaming kernel below for M <= 2, the MFMA kernel after it above.
//
// The streaming kernel is HBM-bound (1 byte of weight per multiply-add), so the design
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
        v = apply_epi_b16(epi, v);
        y[(size_t)m * N + n] = (uint16_t)f32_to_bf16_bits(v);
      }
    }
  }
}

// Skinny-M W8A16 GEMV on MFMA (3 <= M <= 16): with several x rows the
// per-lane multiply-adds (M per weight) make the VALU kernel above compute
// bound, so here the products go to v_mfma_f32_16x16x32_bf16 and the lanes
// only widen the weights (int8 -> bf16, exact).  A workgroup owns 16 weight
// rows; its KQ waves take consecutive parts of K, and their
// 16 x 16 fp32 partial tiles are added in part order through LDS (a fixed
// order: deterministic).  Per 64-deep K block a lane loads 16 int8 of one
// weight row (row lane % 16, k chunk lane / 16: 1 KB per load, 64 bytes per
// row) and 2 x 16 bytes of the same k range of x row lane % 16 (rows past M
// read zero); the first 8 k of the chunk feed the block's first MFMA and the
// other 8 the second, for weights and x alike, so each MFMA still sums
// matching k.  Loads run four blocks ahead through a register ring.
__device__ __forceinline__ bf16x8 i8x8_bf16(uint32_t lo, uint32_t hi) {
  uint32_t o[4];
  const uint32_t w[2] = {lo, hi};
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int32_t v = (int32_t)w[i];
    o[2 * i] = __builtin_amdgcn_perm(__float_as_uint((float)((v << 16) >> 24)),
                                     __float_as_uint((float)((v << 24) >> 24)), 0x07060302u);
    o[2 * i + 1] = __builtin_amdgcn_perm(__float_as_uint((float)(v >> 24)),
                                         __float_as_uint((float)((v << 8) >> 24)), 0x07060302u);
  }
  return __builtin_bit_cast(bf16x8, make_uint4(o[0], o[1], o[2], o[3]));
}

// KQ waves per workgroup, each a consecutive 1/KQ of K; RT tiles of 16 weight
// rows per workgroup, which share each x fragment (x is read once per 16*RT
// weight rows; wave t < RT finishes tile t)
template <int KQ, int RT>
__global__ __launch_bounds__(KQ * 64) void gemv_w8a16_mfma_kernel(const uint16_t *__restrict__ x,
                                                              const int8_t *__restrict__ Q,
                                                              const float *__restrict__ scales,
                                                              const float *__restrict__ bias,
                                                              int epi, uint16_t *__restrict__ y,
                                                              int M, int N, int K) {
  static_assert(RT <= KQ, "one finishing wave per row tile");
  __shared__ f32x4 red[KQ][RT][64];
  constexpr int D = 4;  // blocks in flight per wave
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 16 * RT;
  const int r = lane & 15, c = lane >> 4;
  const int rows = N - n0 < 16 * RT ? N - n0 : 16 * RT;
  const __amdgpu_buffer_rsrc_t rQ = make_rsrc(Q + (size_t)n0 * K, (int64_t)rows * K);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (int64_t)M * K * 2);
  const int nblk = (K + 63) / 64;
  const int per = (nblk + KQ - 1) / KQ;
  const int b0 = wave * per;
  const int b1 = b0 + per < nblk ? b0 + per : nblk;
  const bool xrow = r < M;
  uint4 qw[D][RT], xa[D], xb[D];
  auto issue = [&](int b, int slot) {
    const int k = b * 64 + c * 16;
    const bool ok = b < b1 && k < K;
#pragma unroll
    for (int t = 0; t < RT; ++t) {  // rows past the tile read zero (buffer bounds)
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
          rQ, ok ? (uint32_t)((t * 16 + r) * K + k) : kOobOffset, 0, 2 /* nt */);
      qw[slot][t] = make_uint4(v[0], v[1], v[2], v[3]);
    }
    if (xrow) {  // lanes of x rows past M keep zeros
      const uint32_t xo = ok ? (uint32_t)((r * K + k) * 2) : kOobOffset;
      const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);
      const u32x4 bb = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 16, 0, 0);
      xa[slot] = make_uint4(a[0], a[1], a[2], a[3]);
      xb[slot] = make_uint4(bb[0], bb[1], bb[2], bb[3]);
    }
  };
  f32x4 acc[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int d = 0; d < D; ++d) xa[d] = xb[d] = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int d = 0; d < D; ++d) issue(b0 + d, d);
  for (int b = b0; b < b1; b += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (b + d < b1) {
#pragma unroll
        for (int t = 0; t < RT; ++t) {
          const bf16x8 w0 = i8x8_bf16(qw[d][t].x, qw[d][t].y);
          const bf16x8 w1 = i8x8_bf16(qw[d][t].z, qw[d][t].w);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0, __builtin_bit_cast(bf16x8, xa[d]),
                                                           acc[t], 0, 0, 0);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1, __builtin_bit_cast(bf16x8, xb[d]),
                                                           acc[t], 0, 0, 0);
        }
        issue(b + d + D, d);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < RT; ++t) red[wave][t][lane] = acc[t];
  __syncthreads();
  if (wave >= RT) return;
  f32x4 sum = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int w = 0; w < KQ; ++w) sum += red[w][wave][lane];
  // lane: x row m = lane % 16, weight rows n0 + 16 wave + 4 (lane / 16) + q
  const int m = r;
  if (m >= M) return;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int n = n0 + 16 * wave + 4 * c + q;
    if (n >= N) break;
    float v;
    {
#pragma clang fp contract(off)
      v = sum[q] * scales[n];
      if (bias) v = v + bias[n];
    }
    y[(size_t)m * N + n] = (uint16_t)f32_to_bf16_bits(apply_epi_b16(epi, v));
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

// x rows from which the MFMA kernel takes the GEMV.  11008 x 4096 on MI355X
// (graph replay, weights rotated past the MALL): M = 2 13.3 us VALU against
// 15.2 MFMA; M = 3 18.7 / 15.6; M = 4 21.4 / 16.1; M = 8 35.0 / 17.9.  With
// 8 waves per workgroup (K in eighths) or 8 blocks in flight per wave the
// MFMA kernel measured 1-2 us slower.
constexpr int kGemvMfmaMinM = 3;

hipError_t launch_gemv_w8a16(const uint16_t *x, const int8_t *Q, const float *scales,
                             const float *bias, int epi, uint16_t *y, int64_t M, int64_t N,
                             int64_t K, hipStream_t stream) {
  if (M >= kGemvMfmaMinM && M <= kGemvMaxM) {
    // 32-bit buffer offsets over the x rows and the 64 weight rows of a workgroup
    if (M * K * 2 >= ((int64_t)1 << 31) - 64 || 64 * K >= ((int64_t)1 << 31))
      return hipErrorInvalidValue;
    if (M > 8)  // 4 row tiles: M = 16 22.0 -> 19.4 us; slower at M <= 4 (15.4 -> 17.5)
      hipLaunchKernelGGL((gemv_w8a16_mfma_kernel<4, 4>), dim3((unsigned)((N + 63) / 64)),
                         dim3(256), 0, stream, x, Q, scales, bias, epi, y, (int)M, (int)N,
                         (int)K);
    else
      hipLaunchKernelGGL((gemv_w8a16_mfma_kernel<4, 1>), dim3((unsigned)((N + 15) / 16)),
                         dim3(256), 0, stream, x, Q, scales, bias, epi, y, (int)M, (int)N,
                         (int)K);
    return hipGetLastError();
  }
  if (M <= 1) return launch_mb<1>(x, Q, scales, bias, epi, y, M, N, K, stream);
  if (M <= 2) return launch_mb<2>(x, Q, scales, bias, epi, y, M, N, K, stream);
  return hipErrorInvalidValue;  // M > kGemvMaxM is the GEMM's
}

}  // namespace mj
