// Shared device helpers for the gfx950 kernels: vector types, bf16
// conversion, the activation epilogues and small launch utilities.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mj {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
typedef __attribute__((__vector_size__(16 * sizeof(int)))) int i32x16;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;

// Buffer resource over [base, base + bytes) for raw buffer loads: a load whose
// byte offset lies outside the range returns zero, which gives branch-free
// zero fill at matrix edges.  bytes is clamped to the 31-bit offset range.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, int64_t bytes) {
  const int32_t n = bytes > 0x7FFFFFF0LL ? 0x7FFFFFF0 : (int32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, n, 0x00020000);
}

// An offset no resource above ever covers: loads from it return zero.
constexpr uint32_t kOobOffset = 0x7FFFFFF0u;

__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ float4 load_nt16f(const void *p) {
  const f32x4 v = __builtin_nontemporal_load((const f32x4 *)p);
  return make_float4(v[0], v[1], v[2], v[3]);
}

// Every epilogue function below disables FMA contraction so that its
// rounding sequence is the reference's (one rounding per operation).
// Epilogue ids; identical values to MJ_EPI_* in include/momijo_hip.h.
enum Epi : int {
  EPI_NONE = 0,
  EPI_RELU = 1,
  EPI_GELU_TANH = 2,
  EPI_SILU = 3,
  EPI_GELU_TANH_APPROX = 4,
  EPI_SILU_APPROX = 5,
  EPI_RELU_UNARY = 6,
};

// ---------------------------------------------------------------- bf16
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;

// Two fp32 -> packed bf16 bits (lo in bits 0-15), round to nearest even, NaN
// kept a quiet NaN of the same sign and top payload bits: one
// v_cvt_pk_bf16_f32.  Its results equal the bit-level rounding
// u + 0x7FFF + ((u >> 16) & 1) on every finite input, denormals included
// (fp32 denormals are not flushed in these kernels), and (u >> 16) | 0x40 on
// NaNs; the GPU tests check this on ties, denormals, overflow and NaNs.
// Against that bit-level sequence (about six VALU operations per value) it
// halves the C2 GEMM's output time.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return pack_bf16x2(f, 0.0f) & 0xFFFFu;
}

// ---------------------------------------------------------------- activations
// Tensor-engine family (tensor/math.mojo:272-295): exp is the accurate expf.
__device__ __forceinline__ float sigmoid32(float x) {
#pragma clang fp contract(off)
  return 1.0f / (1.0f + expf(-x));
}

__device__ __forceinline__ float silu32(float x) {
#pragma clang fp contract(off)
  return x * sigmoid32(x);
}

// gelu32 with its literal tanh (e^{2t}-1)/(e^{2t}+1); where e^{2t} overflows
// (the reference returns NaN there) the limit tanh = 1 is used.
__device__ __forceinline__ float gelu32(float x) {
#pragma clang fp contract(off)
  const float k = 0.7978845608028654f, c = 0.044715f;
  float x3 = x * x * x;
  float t = k * (x + c * x3);
  float e2x = expf(2.0f * t);
  float th = __builtin_isinf(e2x) ? 1.0f : (e2x - 1.0f) / (e2x + 1.0f);
  return 0.5f * x * (1.0f + th);
}

// learn.nn.activations family (learn/nn/activations.mojo:34-51,137-163).
__device__ __forceinline__ float clamp_ref(float v, float lo, float hi) {
  if (v < lo) v = lo;
  if (v > hi) v = hi;
  return v;
}

__device__ __forceinline__ float exp_approx32(float x) {
#pragma clang fp contract(off)
  float xv = clamp_ref(x, -20.0f, 20.0f);
  float y = 1.0f + xv / 64.0f;
  y = y * y; y = y * y; y = y * y; y = y * y; y = y * y; y = y * y;
  return y;
}

__device__ __forceinline__ float tanh_approx32(float x) {
#pragma clang fp contract(off)
  float xv = clamp_ref(x, -10.0f, 10.0f);
  float e2x = exp_approx32(2.0f * xv);
  return (e2x - 1.0f) / (e2x + 1.0f);
}

__device__ __forceinline__ float gelu_approx32(float x) {
#pragma clang fp contract(off)
  const float s = 0.7978845608028654f;
  float x3 = x * x * x;
  float inner = s * (x + 0.044715f * x3);
  return 0.5f * x * (1.0f + tanh_approx32(inner));
}

__device__ __forceinline__ float silu_approx32(float x) {
#pragma clang fp contract(off)
  return x * (1.0f / (1.0f + exp_approx32(-x)));
}

__device__ __forceinline__ float apply_epi(int epi, float v) {
  switch (epi) {
    case EPI_RELU: return v > 0.0f ? v : 0.0f;
    case EPI_GELU_TANH: return gelu32(v);
    case EPI_SILU: return silu32(v);
    case EPI_GELU_TANH_APPROX: return gelu_approx32(v);
    case EPI_SILU_APPROX: return silu_approx32(v);
    case EPI_RELU_UNARY: return v < 0.0f ? 0.0f : v;
    default: return v;
  }
}

// GELU (tanh form) and SiLU for results that are rounded to bf16 (the bf16
// and W8A16 GEMM/GEMV epilogues).  0.5 x (1 + tanh t) = x * sigmoid(2t), so
// gelu = x / (1 + 2^(-2 t log2 e)) and silu = x / (1 + 2^(-x log2 e)), with
// the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32, about 1 ulp each).
// The relative error is a few 1e-6 (mostly the rounding of the exponent's
// argument), so the bf16 result equals that of gelu32 / silu32 except within
// about 1e-6 of a bf16 rounding boundary, and except GELU at x < -2: there
// gelu32's 1 + tanh(t) cancels and loses more than a bf16 step of its tiny
// result (|gelu| < 0.05, absolute error < 1e-6), which this form does not.
// Limits as gelu32 / silu32: +inf
// -> +inf, -inf -> NaN, large negative x -> -0, NaN -> NaN.  It costs about
// a quarter of the VALU cycles of the expf + IEEE division forms, which a
// GEMM epilogue spends with nothing left to overlap (C4: 128 GELUs per lane,
// 16 us of a 71 us launch before this form).
// The exponent -2 k log2(e) (x + 0.044715 x^3) is evaluated as x (a + a c x^2)
// (one multiply fewer than the literal nesting; the two differ by an ulp or
// two of the exponent, inside the error stated above).
__device__ __forceinline__ float gelu_b16(float x) {
  constexpr float a = (float)(-2.0 * 0.7978845608028654 * 1.4426950408889634);  // -2 k log2(e)
  constexpr float ac = (float)(-2.0 * 0.7978845608028654 * 1.4426950408889634 * 0.044715);
  const float z = x * __builtin_fmaf(x * x, ac, a);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z));
}

__device__ __forceinline__ float silu_b16(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// acc * s + b in fp32, one rounding each (the per-column scale and bias of
// the int8-weight epilogues)
__device__ __forceinline__ float epi_scale_bias(float acc, float s, float b, bool has_s,
                                                bool has_b) {
#pragma clang fp contract(off)
  float v = acc;
  if (has_s) v = v * s;
  if (has_b) v = v + b;
  return v;
}

__device__ __forceinline__ float apply_epi_b16(int epi, float v) {
  switch (epi) {
    case EPI_GELU_TANH: return gelu_b16(v);
    case EPI_SILU: return silu_b16(v);
    default: return apply_epi(epi, v);
  }
}

// ---------------------------------------------------------------- reductions
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// 64-lane sum without LDS traffic: two quad permutes and two row rotations
// (DPP) leave every lane holding its 16-lane row's sum, and the four row sums
// are read out with readlane.  Summation order: within rows pairwise by the
// DPP pattern, then (row0 + row1) + (row2 + row3).
#define MJ_DPP_F(v, ctrl) \
  __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, false))
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += MJ_DPP_F(v, 0xB1);   // quad_perm [1,0,3,2]
  v += MJ_DPP_F(v, 0x4E);   // quad_perm [2,3,0,1]
  v += MJ_DPP_F(v, 0x124);  // row_ror:4
  v += MJ_DPP_F(v, 0x128);  // row_ror:8
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}
#undef MJ_DPP_F

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fminf(v, __shfl_xor(v, off, 64));
  return v;
}

// ---------------------------------------------------------------- tiles
// Maps a linear workgroup id onto a (tile_m, tile_n) pair so that the
// workgroups the hardware places on one XCD (ids congruent mod 8) form a
// compact block of tiles that shares A rows and B rows in that XCD's L2:
// the ids are first regrouped per XCD, then walked GROUP_M tile rows at a
// time, column by column.
// The walk: logical tile index -> (tile_m, tile_n), GROUP_M tile rows at a
// time, column by column.
__device__ __forceinline__ void group_coords(int logical, int tiles_m, int tiles_n, int group_m,
                                             int &tm, int &tn) {
  const int per_group = group_m * tiles_n;
  const int g = logical / per_group;
  const int first_m = g * group_m;
  int gsize = tiles_m - first_m;
  if (gsize > group_m) gsize = group_m;
  const int in_g = logical - g * per_group;
  tm = first_m + in_g % gsize;
  tn = in_g / gsize;
}

__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int group_m,
                                            int &tm, int &tn) {
  const int total = tiles_m * tiles_n;
  // workgroup bid runs on XCD bid % 8; XCD x takes the contiguous logical
  // range [x q + min(x, r), ...) of c_x = q + (x < r) tiles (q = total / 8,
  // r = total % 8), so neighbouring tiles, which share operand panels, share
  // an L2
  const int x = bid & 7, q = total >> 3, r = total & 7;
  const int logical = x * q + (x < r ? x : r) + (bid >> 3);
  group_coords(logical, tiles_m, tiles_n, group_m, tm, tn);
}

// Split-K grids of `splits` K slices of `tiles` tiles: when splits divides 8
// and the grid is a multiple of 8, XCD x runs K slice x / (8 / splits), so
// the A and B panels of a slice are fetched by 8 / splits XCDs instead of
// all eight; otherwise slice-major order with tile_coords within a slice.
__device__ __forceinline__ void split_tile_coords(int bid, int tiles_m, int tiles_n, int splits,
                                                  int group_m, int &split, int &tm, int &tn) {
  const int tiles = tiles_m * tiles_n;
  if (splits > 1 && (8 % splits) == 0 && ((tiles * splits) & 7) == 0) {
    const int xs = 8 / splits, x = bid & 7;
    split = x / xs;
    group_coords((x % xs) * (tiles / xs) + (bid >> 3), tiles_m, tiles_n, group_m, tm, tn);
    return;
  }
  split = bid / tiles;
  tile_coords(bid - split * tiles, tiles_m, tiles_n, group_m, tm, tn);
}

}  // namespace mj
