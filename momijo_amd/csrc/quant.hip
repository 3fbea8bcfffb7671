// int8 quantize / pack and the small int8 helpers of momijo's PTQ path
// (learn/api/functional.mojo:206-302, learn/api/sequential.mojo:217-263).
//
// quantize_rowwise: one wave per weight row.  For K <= 4096 (K % 256 == 0)
// the row is read once with 16-byte loads into registers (16 KiB per row),
// reduced to its absmax / min-max with a wave butterfly, then quantized from
// registers and written as 4-byte words: the kernel touches every byte of W
// and Q exactly once, so it is HBM-bound.  The division w/scale is the IEEE
// correctly rounded one (built with -fhip-fp32-correctly-rounded-divide-sqrt)
// so results are bit-identical to a CPU fp32 division; the RHE register paths
// get the same integers from a multiply by 1/scale and divide only the rare
// elements whose quotient lies within 2^-14 of a half-integer (quant_rhe_r),
// which halves their VALU work.
#include "common.h"
#include "launch.h"

namespace mj {

enum Rounding : int { ROUND_RHE = 0, ROUND_LEGACY = 1 };

// _round_to_i32 + _clamp_int8 (functional.mojo:208-217): fp32 add of +-0.5,
// truncation toward zero, clamp to [-128, 127]; NaN -> 0.
__device__ __forceinline__ int quant_legacy(float x, float scale) {
#pragma clang fp contract(off)
  const float v = x / scale;
  const float t = v + (v >= 0.0f ? 0.5f : -0.5f);
  if (t != t) return 0;
  if (t >= 127.0f) return 127;
  if (t <= -128.0f) return -128;
  return (int)t;
}

// round half to even, clamp to [-127, 127]; NaN -> 0 (a NaN weight, or a
// NaN scale, quantizes to zero instead of an undefined float-to-int cast).
__device__ __forceinline__ int quant_rhe(float x, float scale) {
  float v = __builtin_rintf(x / scale);
  if (v != v) return 0;
  v = v > 127.0f ? 127.0f : v;
  v = v < -127.0f ? -127.0f : v;
  return (int)v;
}

// quant_rhe from r = 1 / scale (correctly rounded, once per row) instead of a
// division per element (quant4_rhe_r below).  t = x * r is within two roundings of 2^-24 each of
// x / scale, and |x / scale| <= 127.5 (scale = max|row| / 127), so t differs
// from the correctly rounded quotient fl(x / scale) by less than 2^-15.7:
// rint(t) = rint(fl(x / scale)) unless one of them lies within that distance
// of a half-integer (t - floor(t), and its distance to 0.5, are exact).
// Those elements (about one in 8000 of random data, every element of a row of
// exact ties) take the division.  NaN -> 0 and the scale-inf row (r = 0: every
// finite x gives 0, as x / inf does) agree with quant_rhe; a scale whose
// reciprocal overflows must use quant_rhe (callers check r once per row).
// rint(x * r) and whether x is one of the elements that need the division.
__device__ __forceinline__ float rhe_r_fast(float x, float r, bool &amb) {
#pragma clang fp contract(off)
  const float t = x * r;
  const float d = t - floorf(t);
  amb = fabsf(d - 0.5f) < 0x1p-14f;
  return __builtin_rintf(t);
}

// A rounded quotient (NaN for a NaN input) -> int8 range, NaN -> 0.
__device__ __forceinline__ int rhe_clamp(float v) {
  return v != v ? 0 : (int)__builtin_amdgcn_fmed3f(v, -127.0f, 127.0f);
}

// Four elements by quant_rhe_r's rule.  The division runs only when some lane
// of the wave holds an element that needs it (a uniform branch, taken by about
// 3 % of the 256-element groups of random data).
__device__ __forceinline__ void quant4_rhe_r(const float (&x)[4], float scale, float r,
                                             int (&q)[4]) {
  bool amb[4];
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = rhe_r_fast(x[e], r, amb[e]);
  if (__builtin_amdgcn_ballot_w64(amb[0] | amb[1] | amb[2] | amb[3])) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (amb[e]) v[e] = __builtin_rintf(x[e] / scale);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) q[e] = rhe_clamp(v[e]);
}

// MinMaxObserver.observe's NaN rule (sequential.mojo:232-240): min and max
// start at the first element and are replaced only when v < mn / v > mx, so
// a NaN first element makes both NaN and later NaNs are skipped.  The
// reductions use fminf / fmaxf, which skip every NaN; this restores the first
// element's case.
__device__ __forceinline__ void observer_nan_rule(float first, float &mn, float &mx) {
  if (first != first) mn = mx = first;
}

__device__ __forceinline__ float row_scale(int rounding, float amax, float mn, float mx) {
  if (rounding == ROUND_RHE) {
    const float s = amax / 127.0f;
    return s == 0.0f ? 1.0f : s;
  }
  // MinMaxObserver.scale_symmetric(127) (sequential.mojo:252-263)
  const float a = mn < 0.0f ? -mn : mn;
  const float b = mx < 0.0f ? -mx : mx;
  const float m = b > a ? b : a;
  if (m <= 0.0f) return 1.0f;
  return m / 127.0f;
}

// rounding: ROUND_RHE, ROUND_LEGACY, or kRheRecip (RHE by quant_rhe_r with
// r = 1 / s).
constexpr int kRheRecip = 2;

__device__ __forceinline__ uint32_t quant4(int rounding, float4 w, float s, float r) {
  int q0, q1, q2, q3;
  if (rounding == kRheRecip) {
    int q[4];
    quant4_rhe_r({w.x, w.y, w.z, w.w}, s, r, q);
    q0 = q[0]; q1 = q[1]; q2 = q[2]; q3 = q[3];
  } else if (rounding == ROUND_RHE) {
    q0 = quant_rhe(w.x, s); q1 = quant_rhe(w.y, s); q2 = quant_rhe(w.z, s); q3 = quant_rhe(w.w, s);
  } else {
    q0 = quant_legacy(w.x, s); q1 = quant_legacy(w.y, s);
    q2 = quant_legacy(w.z, s); q3 = quant_legacy(w.w, s);
  }
  return (uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8) | ((uint32_t)(q2 & 0xFF) << 16) |
         ((uint32_t)(q3 & 0xFF) << 24);
}

// Register path: K == CH * 256.
template <int CH>
__global__ __launch_bounds__(256) void quantize_rowwise_reg(const float *__restrict__ W, int N,
                                                            int K, int rounding,
                                                            int8_t *__restrict__ Q,
                                                            float *__restrict__ scales) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= N) return;
  const float4 *w4 = (const float4 *)(W + (size_t)row * K);
  float4 w[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) w[c] = load_nt16f(w4 + c * 64 + lane);
  float amax = 0.0f, mn = w[0].x, mx = w[0].x;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(w[c].x), fabsf(w[c].y)), fmaxf(fabsf(w[c].z), fabsf(w[c].w))));
    mn = fminf(mn, fminf(fminf(w[c].x, w[c].y), fminf(w[c].z, w[c].w)));
    mx = fmaxf(mx, fmaxf(fmaxf(w[c].x, w[c].y), fmaxf(w[c].z, w[c].w)));
  }
  amax = wave_max(amax);
  mn = wave_min(mn);
  mx = wave_max(mx);
  observer_nan_rule(__shfl(w[0].x, 0, 64), mn, mx);
  const float s = row_scale(rounding, amax, mn, mx);
  const float r = 1.0f / s;
  uint32_t *q4 = (uint32_t *)(Q + (size_t)row * K);
  if (rounding == ROUND_RHE && r < __builtin_inff()) {
#pragma unroll
    for (int c = 0; c < CH; ++c) q4[c * 64 + lane] = quant4(kRheRecip, w[c], s, r);
  } else {
#pragma unroll
    for (int c = 0; c < CH; ++c) q4[c * 64 + lane] = quant4(rounding, w[c], s, r);
  }
  if (lane == 0) scales[row] = s;
}

// Generic path: any K, two passes over the row (the second mostly from L2).
__global__ __launch_bounds__(256) void quantize_rowwise_any(const float *__restrict__ W, int N,
                                                            int K, int rounding,
                                                            int8_t *__restrict__ Q,
                                                            float *__restrict__ scales) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= N) return;
  const float *w = W + (size_t)row * K;
  float amax = 0.0f, mn = w[0], mx = w[0];
  for (int k = lane; k < K; k += 64) {
    const float v = w[k];
    amax = fmaxf(amax, fabsf(v));
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
  amax = wave_max(amax);
  mn = wave_min(mn);
  mx = wave_max(mx);
  observer_nan_rule(w[0], mn, mx);
  const float s = row_scale(rounding, amax, mn, mx);
  for (int k = lane; k < K; k += 64)
    Q[(size_t)row * K + k] = (int8_t)(rounding == ROUND_RHE ? quant_rhe(w[k], s) : quant_legacy(w[k], s));
  if (lane == 0) scales[row] = s;
}

hipError_t launch_quantize_rowwise(const float *W, int64_t N, int64_t K, int rounding,
                                   int8_t *Q, float *scales, hipStream_t stream) {
  const unsigned blocks = (unsigned)((N + 3) / 4);
  const bool aligned = ((uintptr_t)W % 16 == 0) && ((uintptr_t)Q % 4 == 0);
  if (aligned && K % 256 == 0 && K <= 4096) {
    switch (K / 256) {
#define MJ_Q_CASE(ch)                                                                        \
  case ch:                                                                                   \
    hipLaunchKernelGGL(quantize_rowwise_reg<ch>, dim3(blocks), dim3(256), 0, stream, W,       \
                       (int)N, (int)K, rounding, Q, scales);                                   \
    return hipGetLastError();
      MJ_Q_CASE(1) MJ_Q_CASE(2) MJ_Q_CASE(3) MJ_Q_CASE(4) MJ_Q_CASE(5) MJ_Q_CASE(6)
      MJ_Q_CASE(7) MJ_Q_CASE(8) MJ_Q_CASE(9) MJ_Q_CASE(10) MJ_Q_CASE(11) MJ_Q_CASE(12)
      MJ_Q_CASE(13) MJ_Q_CASE(14) MJ_Q_CASE(15) MJ_Q_CASE(16)
#undef MJ_Q_CASE
      default: break;
    }
  }
  hipLaunchKernelGGL(quantize_rowwise_any, dim3(blocks), dim3(256), 0, stream, W, (int)N, (int)K,
                     rounding, Q, scales);
  return hipGetLastError();
}

// Dynamic per-row activation quantize for the W8A8 Linear: x [M, K] bf16 ->
// xq [M, K] int8 and sx [M] fp32 with the RHE rule of quantize_rowwise
// (scale = max|row| / 127, 1.0 for an all-zero row; q = clamp(rne(x / scale),
// -127, 127); bf16 -> fp32 is exact).  For K = 512 n (n <= 16) the row is
// held in registers (8 bf16 per 16-byte load), so x and xq are each touched
// once; other K take a two-pass kernel with one wave per row.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

__device__ __forceinline__ float amax8(uint4 v) {
  const float a = fmaxf(fmaxf(fabsf(bf16_lo(v.x)), fabsf(bf16_hi(v.x))),
                        fmaxf(fabsf(bf16_lo(v.y)), fabsf(bf16_hi(v.y))));
  const float b = fmaxf(fmaxf(fabsf(bf16_lo(v.z)), fabsf(bf16_hi(v.z))),
                        fmaxf(fabsf(bf16_lo(v.w)), fabsf(bf16_hi(v.w))));
  return fmaxf(a, b);
}

template <bool RECIP>
__device__ __forceinline__ uint32_t quant_pair2(uint32_t w0, uint32_t w1, float s, float r) {
  const float x[4] = {bf16_lo(w0), bf16_hi(w0), bf16_lo(w1), bf16_hi(w1)};
  int q[4];
  if (RECIP) {
    quant4_rhe_r(x, s, r, q);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) q[e] = quant_rhe(x[e], s);
  }
  return (uint32_t)(q[0] & 0xFF) | ((uint32_t)(q[1] & 0xFF) << 8) |
         ((uint32_t)(q[2] & 0xFF) << 16) | ((uint32_t)(q[3] & 0xFF) << 24);
}

// W waves per row (W = 1, 2 or 4; 4 / W rows per workgroup), CH 16-byte
// loads per lane: K = 512 W CH.  Several waves per row keep more loads in
// flight than one wave holding the whole row (the kernel is latency-bound at
// C4's 2048 rows with one); the row's absmax is combined through LDS.  x is
// an activation the previous layer has just written, so it is read with
// plain loads (nontemporal ones measured 3 % slower: 9.08 against 8.82 us
// for C4's 2048 x 4096 on MI355X).
template <int W, int CH>
__global__ __launch_bounds__(256) void quantize_rows_bf16_reg(const uint16_t *__restrict__ x,
                                                              int M, int K,
                                                              int8_t *__restrict__ xq,
                                                              float *__restrict__ sx) {
  __shared__ float part[4];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (4 / W) + wave / W;
  const int t = (wave % W) * 64 + lane;  // lane within the row
  const bool live = row < M;
  const uint4 *x4 = (const uint4 *)(x + (size_t)(live ? row : 0) * K);
  uint4 v[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c)
    v[c] = live ? x4[c * 64 * W + t] : make_uint4(0, 0, 0, 0);
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c) amax = fmaxf(amax, amax8(v[c]));
  amax = wave_max(amax);
  if (W > 1) {
    if (lane == 0) part[wave] = amax;
    __syncthreads();
    const int w0 = wave - wave % W;
#pragma unroll
    for (int w = 0; w < W; ++w) amax = fmaxf(amax, part[w0 + w]);
  }
  if (!live) return;
  const float s = row_scale(ROUND_RHE, amax, 0.0f, 0.0f);
  const float r = 1.0f / s;
  uint2 *q2 = (uint2 *)(xq + (size_t)row * K);
  if (r < __builtin_inff()) {
#pragma unroll
    for (int c = 0; c < CH; ++c)
      q2[c * 64 * W + t] = make_uint2(quant_pair2<true>(v[c].x, v[c].y, s, r),
                                      quant_pair2<true>(v[c].z, v[c].w, s, r));
  } else {
#pragma unroll
    for (int c = 0; c < CH; ++c)
      q2[c * 64 * W + t] = make_uint2(quant_pair2<false>(v[c].x, v[c].y, s, r),
                                      quant_pair2<false>(v[c].z, v[c].w, s, r));
  }
  if (t == 0) sx[row] = s;
}

__global__ __launch_bounds__(256) void quantize_rows_bf16_any(const uint16_t *__restrict__ x,
                                                              int M, int K,
                                                              int8_t *__restrict__ xq,
                                                              float *__restrict__ sx) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const uint16_t *r = x + (size_t)row * K;
  float amax = 0.0f;
  for (int k = lane; k < K; k += 64) amax = fmaxf(amax, fabsf(bf16_lo(r[k])));
  amax = wave_max(amax);
  const float s = row_scale(ROUND_RHE, amax, 0.0f, 0.0f);
  for (int k = lane; k < K; k += 64) xq[(size_t)row * K + k] = (int8_t)quant_rhe(bf16_lo(r[k]), s);
  if (lane == 0) sx[row] = s;
}

template <int W, int CH>
static hipError_t launch_rows_reg(const uint16_t *x, int64_t M, int64_t K, int8_t *xq, float *sx,
                                 hipStream_t stream) {
  const unsigned blocks = (unsigned)((M + 4 / W - 1) / (4 / W));
  hipLaunchKernelGGL((quantize_rows_bf16_reg<W, CH>), dim3(blocks), dim3(256), 0, stream, x,
                     (int)M, (int)K, xq, sx);
  return hipGetLastError();
}

hipError_t launch_quantize_rows_bf16(const uint16_t *x, int64_t M, int64_t K, int8_t *xq,
                                     float *sx, hipStream_t stream) {
  const bool aligned = ((uintptr_t)x % 16 == 0) && ((uintptr_t)xq % 8 == 0);
  if (aligned && K % 512 == 0 && K <= 8192) {
    // K = 512 n: 4 waves per row when n % 4 == 0, else 2 when n is even
    switch (K / 512) {
      case 1: return launch_rows_reg<1, 1>(x, M, K, xq, sx, stream);
      case 2: return launch_rows_reg<2, 1>(x, M, K, xq, sx, stream);
      case 3: return launch_rows_reg<1, 3>(x, M, K, xq, sx, stream);
      case 4: return launch_rows_reg<4, 1>(x, M, K, xq, sx, stream);
      case 5: return launch_rows_reg<1, 5>(x, M, K, xq, sx, stream);
      case 6: return launch_rows_reg<2, 3>(x, M, K, xq, sx, stream);
      case 7: return launch_rows_reg<1, 7>(x, M, K, xq, sx, stream);
      case 8: return launch_rows_reg<4, 2>(x, M, K, xq, sx, stream);
      case 9: return launch_rows_reg<1, 9>(x, M, K, xq, sx, stream);
      case 10: return launch_rows_reg<2, 5>(x, M, K, xq, sx, stream);
      case 11: return launch_rows_reg<1, 11>(x, M, K, xq, sx, stream);
      case 12: return launch_rows_reg<4, 3>(x, M, K, xq, sx, stream);
      case 13: return launch_rows_reg<1, 13>(x, M, K, xq, sx, stream);
      case 14: return launch_rows_reg<2, 7>(x, M, K, xq, sx, stream);
      case 15: return launch_rows_reg<1, 15>(x, M, K, xq, sx, stream);
      case 16: return launch_rows_reg<4, 4>(x, M, K, xq, sx, stream);
      default: break;
    }
  }
  const unsigned blocks = (unsigned)((M + 3) / 4);
  hipLaunchKernelGGL(quantize_rows_bf16_any, dim3(blocks), dim3(256), 0, stream, x, (int)M,
                     (int)K, xq, sx);
  return hipGetLastError();
}

// quant_legacy from r = 1 / scale (correctly rounded, once) instead of a
// division per element.  v' = x * r is within two roundings of 2^-24 each of
// x / scale, so for |v'| < 128 it differs from fl(x / scale) by less than
// 2^-15: away from the half-integers (where v + 0.5 or v - 0.5 crosses an
// integer) both give the same t after the +-0.5 add (whose own rounding is at
// most 2^-17 there) and the same truncation; for |v'| >= 128 both clamp the
// same way.  Elements within 2^-14 of a half-integer take the division (a
// uniform branch when any lane of the wave needs it).  NaN -> 0 and an
// infinite x agree with quant_legacy; a scale whose reciprocal overflows must
// use quant_legacy (the caller checks r once).
__device__ __forceinline__ uint32_t quant4_legacy_r(float4 w, float s, float r) {
  const float x[4] = {w.x, w.y, w.z, w.w};
  float v[4];
  bool amb[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
#pragma clang fp contract(off)
    v[e] = x[e] * r;
    const float a = fabsf(v[e]);
    amb[e] = a < 128.0f && fabsf((a - floorf(a)) - 0.5f) < 0x1p-14f;
  }
  if (__builtin_amdgcn_ballot_w64(amb[0] | amb[1] | amb[2] | amb[3])) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (amb[e]) v[e] = x[e] / s;
  }
  uint32_t out = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    int qe;
    {
#pragma clang fp contract(off)
      const float t = v[e] + (v[e] >= 0.0f ? 0.5f : -0.5f);
      qe = t != t ? 0 : t >= 127.0f ? 127 : t <= -128.0f ? -128 : (int)t;
    }
    out |= (uint32_t)(qe & 0xFF) << (8 * e);
  }
  return out;
}

// quantize_symmetric_int8 (functional.mojo:231-247), per-tensor scale: four
// elements per thread and step (16-byte loads, 4-byte stores) by the
// reciprocal rule above, the remainder (and unaligned pointers) one element
// at a time by quant_legacy.
__global__ __launch_bounds__(256) void quantize_tensor_legacy(const float *__restrict__ x, int64_t n,
                                                              float scale,
                                                              int8_t *__restrict__ q) {
  const float s = scale == 0.0f ? 1.0f : scale;
  const float r = 1.0f / s;
  const bool recip = fabsf(r) < __builtin_inff();
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t done = 0;
  if ((((uintptr_t)x | (uintptr_t)q) & 15) == 0) {
    const int64_t n4 = n >> 2;
    const float4 *x4 = (const float4 *)x;
    uint32_t *q4 = (uint32_t *)q;
    for (int64_t c = t0; c < n4; c += stride) {
      const float4 w = x4[c];
      q4[c] = recip ? quant4_legacy_r(w, s, r) : quant4(ROUND_LEGACY, w, s, 0.0f);
    }
    done = n4 << 2;
  }
  for (int64_t i = done + t0; i < n; i += stride) q[i] = (int8_t)quant_legacy(x[i], s);
}

hipError_t launch_quantize_tensor_legacy(const float *x, int64_t n, float scale, int8_t *q,
                                         hipStream_t stream) {
  int64_t blocks = (n / 4 + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(quantize_tensor_legacy, dim3((unsigned)blocks), dim3(256), 0, stream, x, n,
                     scale, q);
  return hipGetLastError();
}

// MinMaxObserver: per-workgroup min/max partials, then one workgroup folds
// them and applies scale_symmetric.
constexpr int kMinMaxBlocks = 1024;
int minmax_partials() { return kMinMaxBlocks; }

__global__ __launch_bounds__(256) void minmax_partial_kernel(const float *__restrict__ x, int64_t n,
                                                             float *__restrict__ part) {
  __shared__ float smn[4], smx[4];
  float mn = __builtin_inff(), mx = -__builtin_inff();
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float v = x[i];
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
  mn = wave_min(mn);
  mx = wave_max(mx);
  if ((threadIdx.x & 63) == 0) { smn[threadIdx.x >> 6] = mn; smx[threadIdx.x >> 6] = mx; }
  __syncthreads();
  if (threadIdx.x == 0) {
    part[2 * blockIdx.x] = fminf(fminf(smn[0], smn[1]), fminf(smn[2], smn[3]));
    part[2 * blockIdx.x + 1] = fmaxf(fmaxf(smx[0], smx[1]), fmaxf(smx[2], smx[3]));
  }
}

// Folds the partials; with max_q < 0 it writes {min, max} instead of the
// scale.
__global__ __launch_bounds__(64) void minmax_final_kernel(const float *__restrict__ x,
                                                          const float *__restrict__ part, int np,
                                                          int64_t n, float max_q,
                                                          float *__restrict__ out) {
  float mn = __builtin_inff(), mx = -__builtin_inff();
  for (int i = threadIdx.x; i < np; i += 64) {
    mn = fminf(mn, part[2 * i]);
    mx = fmaxf(mx, part[2 * i + 1]);
  }
  mn = wave_min(mn);
  mx = wave_max(mx);
  if (n > 0) observer_nan_rule(x[0], mn, mx);
  if (threadIdx.x == 0 && max_q < 0.0f) {
    out[0] = mn;
    out[1] = mx;
  } else if (threadIdx.x == 0) {
    float s = 1.0f;
    if (n > 0 && max_q > 0.0f) {
      const float a = mn < 0.0f ? -mn : mn;
      const float b = mx < 0.0f ? -mx : mx;
      const float m = b > a ? b : a;
      s = m <= 0.0f ? 1.0f : m / max_q;
    }
    *out = s;
  }
}

static hipError_t minmax_impl(const float *x, int64_t n, float max_q, float *partials,
                              float *out, hipStream_t stream) {
  int64_t blocks = (n + 255) / 256;
  if (blocks > kMinMaxBlocks) blocks = kMinMaxBlocks;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(minmax_partial_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, x, n,
                     partials);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(minmax_final_kernel, dim3(1), dim3(64), 0, stream, x, partials, (int)blocks,
                     n, max_q, out);
  return hipGetLastError();
}

hipError_t launch_minmax(const float *x, int64_t n, float *partials, float *minmax_out,
                         hipStream_t stream) {
  return minmax_impl(x, n, -1.0f, partials, minmax_out, stream);
}

// max_q <= 0 yields scale 1.0 (scale_symmetric's guard); it is passed as 0
// so the final kernel does not take the {min, max} branch.
hipError_t launch_minmax_scale(const float *x, int64_t n, float max_q, float *partials,
                               float *scale_out, hipStream_t stream) {
  return minmax_impl(x, n, max_q > 0.0f ? max_q : 0.0f, partials, scale_out, stream);
}

// dequantize_i32_to_f32_add_bias (functional.mojo:281-302).
__global__ __launch_bounds__(256) void dequant_i32_bias_kernel(const int32_t *__restrict__ acc,
                                                               float sf,
                                                               const float *__restrict__ b,
                                                               float *__restrict__ y, int64_t M,
                                                               int64_t N) {
  const int64_t total = M * N;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
#pragma clang fp contract(off)
    const float v = (float)acc[i] * sf;
    y[i] = v + b[i % N];
  }
}

hipError_t launch_dequant_i32_bias(const int32_t *acc, float sf, const float *b, float *y,
                                   int64_t M, int64_t N, hipStream_t stream) {
  int64_t blocks = (M * N + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(dequant_i32_bias_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, acc,
                     sf, b, y, M, N);
  return hipGetLastError();
}

// Per-channel (and optionally per-row) dequantize of int32 sums:
// y[m, n] = float(acc[m, n]) * (sx[m] * sw[n]) + b[n], each fp32 operation
// rounded on its own (sx null: the factor is sw[n]; b null: no add).  The
// W8A8 Linear's epilogue as an operator on int32 sums, and the per-channel
// form of dequantize_i32_to_f32_add_bias (functional.mojo:281-302).  Four
// consecutive columns per thread.
__global__ __launch_bounds__(256) void dequant_i32_scaled_kernel(const int32_t *__restrict__ acc,
                                                                 const float *__restrict__ sx,
                                                                 const float *__restrict__ sw,
                                                                 const float *__restrict__ b,
                                                                 float *__restrict__ y, int64_t M,
                                                                 int64_t N) {
  const int64_t n4 = (N + 3) / 4;
  const int64_t total = M * n4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += stride) {
    const int64_t m = t / n4;
    const int64_t n0 = (t - m * n4) * 4;
    const float r = sx ? sx[m] : 1.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t n = n0 + q;
      if (n >= N) break;
      {
#pragma clang fp contract(off)
        const float sf = sx ? r * sw[n] : sw[n];
        float v = (float)acc[m * N + n] * sf;
        if (b) v = v + b[n];
        y[m * N + n] = v;
      }
    }
  }
}

hipError_t launch_dequant_i32_scaled(const int32_t *acc, const float *sx, const float *sw,
                                     const float *b, float *y, int64_t M, int64_t N,
                                     hipStream_t stream) {
  int64_t blocks = (M * ((N + 3) / 4) + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(dequant_i32_scaled_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, acc,
                     sx, sw, b, y, M, N);
  return hipGetLastError();
}

}  // namespace mj
