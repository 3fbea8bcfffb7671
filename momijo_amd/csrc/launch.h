// Host-side launchers shared between the kernel files and the C ABI (api.hip).
// All sizes are validated by the caller; these only pick a configuration and
// enqueue on `stream`.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mj {

// ---- gemm_nt.hip: bf16 A x (bf16 | int8) B^T on MFMA ---------------------
enum BKind : int { B_BF16 = 0, B_INT8 = 1 };

struct GemmNT {
  const uint16_t *A = nullptr;  // [M,K] bf16, leading dim lda
  int64_t lda = 0;
  const void *B = nullptr;      // [N,K] bf16 or int8, leading dim ldb
  int64_t ldb = 0;
  const void *B2 = nullptr;     // gate/up mode: the "up" weight [N,K]
  const float *scales = nullptr;   // per output column (int8 B) or null
  const float *scales2 = nullptr;  // gate/up mode: scales of B2
  const float *bias = nullptr;     // per output column or null
  int epi = 0;
  uint16_t *C = nullptr;        // [M,N] bf16, leading dim ldc
  int64_t ldc = 0;
  int64_t M = 0, N = 0, K = 0;
  int bkind = B_BF16;
  bool gate_up = false;         // C = silu(A B^T * s) * (A B2^T * s2)
  float *part = nullptr;        // split-K partials [splits][M][N] fp32 (workspace)
  int splits = 1;
};

// Tile shape and K split chosen for a problem (the split needs a workspace of
// splits * M * N fp32 passed as GemmNT::part).
struct GemmPlan {
  int bm = 256, bn = 256, splits = 1;
  bool iglp = false;  // K loop built with the compiler's MFMA interleave
  bool pf2 = false;   // distance-2 load pipeline (bf16 B)
  bool tile_kernel = false;  // the dedicated tile kernels: bf16 256 x 256 (two waves per
                             // SIMD), W8A16 256 x 128 (128 x 128 or 128 x 192 up to 128
                             // rows), gate/up 128 or 256 rows x 128, 192 or 256 (one wave
                             // per SIMD)
  int wm = 128;              // W8A16 tile kernels: wave tile height; the planner sets 256
                             // (1 x 4 waves of 256 rows: each widened B fragment feeds 16
                             // MFMAs)
  int depth = 2;             // W8A16 tile kernels: stages of loads in flight (2, or a ring of
                             // 3 where the weights stream from HBM once: M <= 256)
  size_t workspace_bytes(const GemmNT &p) const {
    return splits > 1 ? (size_t)splits * (size_t)p.M * (size_t)p.N * sizeof(float) : 0;
  }
};

GemmPlan plan_gemm_nt(const GemmNT &p);

hipError_t launch_gemm_nt(const GemmNT &p, const GemmPlan &plan, hipStream_t stream);

// ---- gemm_f32.hip ---------------------------------------------------------
// Broadcast batch of matrices: element offsets of batch index b are
// sum_d i_d * stride_d over the multi-index (i_0..i_{rank-1}) of b in shape.
struct BatchDesc {
  static constexpr int kMaxRank = 5;  // tensordot's generic path nests 5 batch loops
  int rank = 0;
  int64_t shape[kMaxRank] = {1, 1, 1, 1, 1};
  int64_t a_stride[kMaxRank] = {0, 0, 0, 0, 0};
  int64_t b_stride[kMaxRank] = {0, 0, 0, 0, 0};
};

hipError_t launch_gemm_f32_batched(int64_t M, int64_t N, int64_t K, const float *A, int64_t sAm,
                                   int64_t sAk, const float *B, int64_t sBk, int64_t sBn,
                                   float *C, const BatchDesc &bd, int64_t batches,
                                   hipStream_t stream);
hipError_t launch_gemm_f64(int64_t M, int64_t N, int64_t K, const double *A, int64_t sAm,
                           int64_t sAk, const double *B, int64_t sBk, int64_t sBn, double *C,
                           int64_t ldc, int accum, hipStream_t stream);
// Column sums of a row-major [N, OutF] fp32 matrix; segs from colsum_segments
// (1 = strict ascending-n order); part holds segs * OutF floats when segs > 1.
int64_t colsum_segments(int64_t N, int64_t OutF);
hipError_t launch_colsum_f32(const float *X, int64_t N, int64_t OutF, float *out, float *part,
                             int64_t segs, hipStream_t stream);
hipError_t launch_matvec_f64(int64_t M, int64_t N, const double *A, int64_t sAm, int64_t sAn,
                             const double *x, int64_t sx, double *y, hipStream_t stream);
hipError_t launch_gemm_f32(int64_t M, int64_t N, int64_t K, const float *A, int64_t sAm,
                           int64_t sAk, const float *B, int64_t sBk, int64_t sBn,
                           const float *bias, int epi, float *C, int64_t ldc,
                           hipStream_t stream);
// C = A @ B, or with accum C = C + A @ B (one rounding of the fp32 product
// sum onto the old value: the tape's grads[p].add(g)).
hipError_t launch_gemm_f32_accum(int64_t M, int64_t N, int64_t K, const float *A, int64_t sAm,
                                 int64_t sAk, const float *B, int64_t sBk, int64_t sBn, float *C,
                                 int64_t ldc, int accum, hipStream_t stream);
hipError_t launch_matvec_f32(int64_t M, int64_t N, const float *A, int64_t sAm, int64_t sAn,
                             const float *x, int64_t sx, float *y, hipStream_t stream);
hipError_t launch_activation_f32(int epi, const float *x, float *y, int64_t n,
                                 hipStream_t stream);
// Conv2d.forward, NCHW fp32, as an implicit GEMM per image (gemm_f32.hip):
// x [N,C,H,W], w [OC,C,kH,kW], b [OC] or null, y [N,OC,OH,OW]; OH, OW from
// the caller (>= 1); C H W, OC C kH kW and OC OH OW below 2^31.
hipError_t launch_conv2d_f32(const float *x, const float *w, const float *b, float *y, int64_t N,
                             int64_t C, int64_t H, int64_t W, int64_t OC, int64_t kH,
                             int64_t kW, int64_t sH, int64_t sW, int64_t pH, int64_t pW,
                             int64_t OH, int64_t OW, int epi, hipStream_t stream);
// y = x >= s ? x : s elementwise (Tensor[Float32].maximum_scalar).
hipError_t launch_maximum_scalar_f32(const float *x, float s, float *y, int64_t n,
                                     hipStream_t stream);
// y = Float32(x) elementwise, round to nearest even (astype_f32_from_int).
hipError_t launch_cast_i64_f32(const int64_t *x, float *y, int64_t n, hipStream_t stream);

// ---- gemv_w8.hip: skinny-M W8A16 -----------------------------------------
// Largest x row count the W8A16 GEMV kernels take; larger M runs the int8
// MFMA GEMM (at M = 9..16 the GEMV's MFMA kernel takes 18-22 us on
// 11008 x 4096 where the 256-row GEMM tile takes 38 us).
constexpr int64_t kGemvMaxM = 16;
// Whether launch_gemv_w8a16 takes an M-row W8A16 product: every M <= 16, and
// 17..48 rows when K = 1024 j <= 4096 (the skinny MFMA GEMV with two or four
// 16-row x groups).
inline bool gemv_w8a16_takes(int64_t M, int64_t K) {
  return M <= kGemvMaxM || (M <= 48 && K % 1024 == 0 && K > 0 && K <= 4096);
}
hipError_t launch_gemv_w8a16(const uint16_t *x, const int8_t *Q, const float *scales,
                             const float *bias, int epi, uint16_t *y, int64_t M, int64_t N,
                             int64_t K, hipStream_t stream);
// Whether launch_gemv_gateup_w8a16 takes the FFN's gate/up at M x rows: 1..4
// rows at K % 16 == 0, K <= 16384 (the K-split GEMVs), 5..32 rows at K = 1024 j
// <= 4096 (the skinny MFMA GEMV, which also takes 3..4 rows at such K).
inline bool gemv_gateup_w8a16_takes(int64_t M, int64_t K) {
  if (K <= 0 || K % 16 || M < 1) return false;
  if (M <= 4) return K <= 16384;
  return M <= 32 && K % 1024 == 0 && K <= 4096;
}
// The FFN's gate/up as a GEMV: h [M,N] = bf16(silu(x Wg^T * sg) * (x Wu^T *
// su)) for the shapes gemv_gateup_w8a16_takes accepts; 16-byte aligned x, Wg, Wu.
hipError_t launch_gemv_gateup_w8a16(const uint16_t *x, const int8_t *Wg, const float *sg,
                                    const int8_t *Wu, const float *su, uint16_t *h, int64_t M,
                                    int64_t N, int64_t K, hipStream_t stream);

// ---- quant.hip -------------------------------------------------------------
hipError_t launch_quantize_rowwise(const float *W, int64_t N, int64_t K, int rounding,
                                   int8_t *Q, float *scales, hipStream_t stream);
hipError_t launch_quantize_tensor_legacy(const float *x, int64_t n, float scale, int8_t *q,
                                         hipStream_t stream);
// partials must hold 2 * minmax_partials() floats
int minmax_partials();
hipError_t launch_minmax(const float *x, int64_t n, float *partials, float *minmax_out,
                         hipStream_t stream);
hipError_t launch_minmax_scale(const float *x, int64_t n, float max_q, float *partials,
                               float *scale_out, hipStream_t stream);
hipError_t launch_dequant_i32_bias(const int32_t *acc, float sf, const float *b, float *y,
                                   int64_t M, int64_t N, hipStream_t stream);
// y = float(acc) * (sx[m] * sw[n]) + b[n] (sx, b may be null).
hipError_t launch_dequant_i32_scaled(const int32_t *acc, const float *sx, const float *sw,
                                     const float *b, float *y, int64_t M, int64_t N,
                                     hipStream_t stream);
// x [M,K] bf16 -> xq [M,K] int8, sx [M] fp32: per-row RHE quantize (the W8A8
// Linear's dynamic activation scales).
hipError_t launch_quantize_rows_bf16(const uint16_t *x, int64_t M, int64_t K, int8_t *xq,
                                     float *sx, hipStream_t stream);

// ---- gemm_i8.hip -----------------------------------------------------------
// C (int32) = A int8 [M,K] x B^T, B int8 [N,K]; or, with y != null, the fused
// dequantize y = float(acc)*sf + b.  K % 16 == 0 and 16-byte aligned A and B;
// large problems go to the 256 x 256 kernel below.
hipError_t launch_gemm_i8(const int8_t *A, const int8_t *B, int32_t *C, float *y, float sf,
                          const float *b, int64_t M, int64_t N, int64_t K, hipStream_t stream);
// The int8 GEMM on 256 x 256 (or, below 192 such tiles, 256 x 128) tiles
// (gemm_nt.hip), same arguments and conditions as launch_gemm_i8.
hipError_t launch_gemm_i8_w4(const int8_t *A, const int8_t *B, int32_t *C, float *y, float sf,
                             const float *b, int64_t M, int64_t N, int64_t K, hipStream_t stream);
// The W8A8 Linear's GEMM on the same kernel: y [M,N] bf16 =
// bf16(epi(float(xq Wq^T) * (sx[m] * sw[n]) + bias[n])); bias may be null.
// K % 16 == 0, 16-byte aligned xq and Wq.
hipError_t launch_linear_w8a8(const int8_t *xq, const float *sx, const int8_t *Wq,
                              const float *sw, const float *bias, int epi, uint16_t *y,
                              int64_t M, int64_t N, int64_t K, hipStream_t stream);
// The 128 x 128 kernel alone (gemm_i8.hip).
hipError_t launch_gemm_i8_t128(const int8_t *A, const int8_t *B, int32_t *C, float *y, float sf,
                               const float *b, int64_t M, int64_t N, int64_t K,
                               hipStream_t stream);
// Scalar fallback: literal = the reference's stride-ignoring [K,N] read of B,
// otherwise B [N,K] for shapes/alignments the MFMA kernel does not take.
hipError_t launch_gemm_i8_scalar(const int8_t *A, const int8_t *B, int32_t *C, float *y,
                                 float sf, const float *b, int64_t M, int64_t N, int64_t K,
                                 bool literal, hipStream_t stream);

}  // namespace mj
