/*
 * momijo_hip.h -- C ABI of the MI355X (gfx950) backend for momijo's
 * tensor-engine hot path: dense matmul / Linear, the int8 weight path and the
 * bias + activation epilogue.
 *
 * Every entry point is `extern "C"`, takes plain pointers and sizes, returns
 * an int32 status (MJ_OK = 0) and never throws.  Unless a name ends in `_h`
 * (or is one of the memory-copy entry points), pointers are DEVICE pointers (HIP global memory of the current device) and
 * the call is asynchronous on `stream` (a hipStream_t; NULL = the null
 * stream).  `_h` variants take HOST pointers, copy in, run and copy out
 * synchronously, which is the ownership model of the reference's own device
 * seam (tensor/gpu/runtime.mojo:539-631).
 *
 * Layout conventions: row-major with explicit leading dimensions / strides in
 * ELEMENTS.  bf16 values travel as uint16_t bit patterns.  Weights follow the
 * reference's Linear layout [out_features, in_features] (learn/nn/layers.mojo:
 * 347-348), so y = x W^T is an "NT" product.
 *
 * Workspace.  Calls that need scratch device memory (the split-K W8A16 and
 * bf16 GEMMs, the FFN when it splits K, QuantLinear, the W8A8 Linear,
 * Linear.backward's column sums for N > 1024, the min/max observer) take it
 * from one buffer per (device, stream) that the library keeps and grows;
 * hipStreamPerThread gets one per (device, host thread).  A call holds that
 * buffer from its first to its last enqueue, so host threads may share a
 * stream.  While `stream` is being captured into a HIP graph these calls
 * return MJ_ERR_UNSUPPORTED and enqueue nothing: the library never allocates
 * on a capturing stream.  Everything else (the GEMV, GEMMs without a K split,
 * quantizers, mj_quant_linear_f32_noalloc) can be captured.
 *
 * Reference citations are relative to /root/reference/legacy/src/momijo/.
 */
#ifndef MOMIJO_HIP_H
#define MOMIJO_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes --------------------------------------------------- */
#define MJ_OK 0
#define MJ_ERR_ARG 1         /* null pointer, bad enum, negative size       */
#define MJ_ERR_SHAPE 2       /* operand shapes disagree                     */
#define MJ_ERR_UNSUPPORTED 3 /* alignment / divisibility the kernels need   */
#define MJ_ERR_DEVICE 4      /* a HIP runtime error (launch, copy, sync)    */
#define MJ_ERR_NO_DEVICE 5   /* no gfx950 device is visible                 */
#define MJ_ERR_ALLOC 6       /* device allocation failed                    */

/* ---- epilogues: applied to the fp32 result after scale and bias ----- */
#define MJ_EPI_NONE 0
#define MJ_EPI_RELU 1              /* ReLU.forward: v > 0 ? v : 0 (layers.mojo:117-137)      */
#define MJ_EPI_GELU_TANH 2         /* gelu32 (tensor/math.mojo:288-295), finite past x~10.06 */
#define MJ_EPI_SILU 3              /* silu32 (tensor/math.mojo:283-285)                      */
#define MJ_EPI_GELU_TANH_APPROX 4  /* learn.nn gelu via _exp_approx (activations.mojo:158-163) */
#define MJ_EPI_SILU_APPROX 5       /* learn.nn silu via _exp_approx (activations.mojo:137-152) */
/* Entry points with fp32 outputs evaluate GELU_TANH and SILU literally (expf,
 * IEEE division).  Entry points with bf16 outputs (the bf16 and W8A16 GEMMs,
 * GEMVs and the FFN) evaluate the same functions as x / (1 + 2^(-2t log2 e))
 * and x / (1 + 2^(-x log2 e)) with the hardware exp2 and reciprocal: the bf16
 * bits differ from the literal form's in a few outputs in 10^4 (near a
 * rounding boundary) and, for GELU at x < -2, where the literal form's
 * 1 + tanh cancels; every output stays within one bf16 step or 1e-6. */
#define MJ_EPI_RELU_UNARY 6        /* Tensor.relu, apply_unary op 8 (tensor/math.mojo:582-585) */

/* ---- int8 rounding rules -------------------------------------------- */
#define MJ_ROUND_RHE 0     /* round half to even, clamp [-127,127] (per-channel spec)   */
#define MJ_ROUND_LEGACY 1  /* fp32 v +- 0.5 then truncate, clamp [-128,127]
                              (functional.mojo:208-217)                                 */

/* ---- runtime ---------------------------------------------------------- */

/* ABI version (major*100 + minor). */
int32_t mj_version(void);

/* 1 if a gfx950 device is usable, else 0.  Replaces gpu_available()
 * (tensor/gpu/runtime.mojo:29-36), which is a compile-time probe there. */
int32_t mj_device_available(void);

/* Message for the last non-OK status returned on this host thread. */
const char *mj_last_error(void);

/* Waits for all work queued on `stream`. */
int32_t mj_stream_synchronize(void *stream);

/* ---- fp32 engine ------------------------------------------------------ */

/* C[M,N] = epi(A @ B + bias) for fp32 operands given as (pointer, row stride,
 * column stride), so transposed views (stride swaps, tensor/transform.mojo:
 * 1248-1294, 2107-2136) need no copy.  bias may be NULL; C has leading
 * dimension ldc.  Replaces matmul_core_mm (tensor/broadcast.mojo:1612-1673),
 * reached from Tensor.matmul (tensor/tensor.mojo:3168-3169) and
 * tensor.matmul (tensor/__init__.mojo:123). */
int32_t mj_matmul_f32(int64_t M, int64_t N, int64_t K,
                      const float *A, int64_t sAm, int64_t sAk,
                      const float *B, int64_t sBk, int64_t sBn,
                      const float *bias, int32_t epilogue,
                      float *C, int64_t ldc, void *stream);

/* y[M] = A[M,N] x[N] with strides.  Replaces matmul_core_vec
 * (tensor/broadcast.mojo:1543-1608), Tensor.matmul_vec (tensor.mojo:3180). */
int32_t mj_matvec_f32(int64_t M, int64_t N, const float *A, int64_t sAm, int64_t sAn,
                      const float *x, int64_t sx, float *y, void *stream);

/* y[N,OutF] = epi(x[N,InF] W^T + b), W [OutF,InF] row-major, b [OutF] or
 * NULL.  Replaces Linear.forward / forward_auto (learn/nn/layers.mojo:
 * 383-433, 510-516) with the activation layer that follows it fused in. */
int32_t mj_linear_f32(const float *x, const float *W, const float *bias, int32_t epilogue,
                      float *y, int64_t N, int64_t InF, int64_t OutF, void *stream);

/* fp64 C[M,N] = A @ B with strides, on v_mfma_f64_16x16x4f64.  Replaces the
 * Float64 overloads of matmul_core_mm / matmul (tensor/broadcast.mojo:
 * 1466-1538) and matmul2d (tensor/math.mojo:7838-7880), which autograd's
 * matmul backward calls (tensor/autograd.mojo:1542-1555). */
int32_t mj_matmul_f64(int64_t M, int64_t N, int64_t K,
                      const double *A, int64_t sAm, int64_t sAk,
                      const double *B, int64_t sBk, int64_t sBn,
                      double *C, int64_t ldc, void *stream);

/* fp64 y[M] = A[M,N] x[N].  Replaces matmul_core_vec Float64
 * (tensor/broadcast.mojo:1397-1464). */
int32_t mj_matvec_f64(int64_t M, int64_t N, const double *A, int64_t sAm, int64_t sAn,
                      const double *x, int64_t sx, double *y, void *stream);

/* tensordot(A, B, axes=1) for fp32 (tensor/broadcast.mojo:1694-1900):
 * C[b, :, :] = A[b] @ B[b] over batch_rank <= 5 broadcast batch dimensions
 * of extent batch_shape[d]; the element strides of A's and B's batch
 * dimensions are a_batch_strides[d], b_batch_strides[d] (0 where the operand
 * is broadcast), and A[b], B[b] are (row stride, column stride) views as in
 * mj_matmul_f32.  C is contiguous [batch..., M, N].  The three arrays are
 * host memory. */
int32_t mj_tensordot_f32(int32_t batch_rank, const int64_t *batch_shape,
                         const int64_t *a_batch_strides, const int64_t *b_batch_strides,
                         int64_t M, int64_t N, int64_t K,
                         const float *A, int64_t sAm, int64_t sAk,
                         const float *B, int64_t sBk, int64_t sBn,
                         float *C, void *stream);

/* The MATMUL2D rule of the autograd tape (tensor/autograd.mojo:1542-1555)
 * for y = A @ B, A [M,K], B [K,N], upstream gradient G [M,N], all Float64
 * row-major device arrays:
 *   dA [M,K] (+)= G @ B^T      dB [K,N] (+)= A^T @ G
 * With accumulate != 0 the products are added to the existing dA / dB (the
 * tape's grads[p] = grads[p].add(g)); otherwise they overwrite them.  The
 * transposes are stride views; either output may be NULL. */
int32_t mj_matmul_backward_f64(int64_t M, int64_t N, int64_t K, const double *A, const double *B,
                               const double *G, double *dA, double *dB, int32_t accumulate,
                               void *stream);

/* The same MATMUL2D rule in Float32, the value type of the reference tape
 * (Tape.values / grads are List[Tensor[Float32]], tensor/autograd.mojo:
 * 214-216; GradTensor.matmul / matmul2d record the node, :930-939 and
 * :995-1017): dA (+)= G @ B^T, dB (+)= A^T @ G on the fp32 MFMA engine, the
 * products summed in fp32 and added to the old gradient with one rounding
 * (grads[p].add(g)).  Either output may be NULL. */
int32_t mj_matmul_backward_f32(int64_t M, int64_t N, int64_t K, const float *A, const float *B,
                               const float *G, float *dA, float *dB, int32_t accumulate,
                               void *stream);

/* Host-pointer seam with the signature of launch_1d_linear_fw
 * (tensor/gpu/runtime.mojo:539-631): x [N,InF], wT [InF,OutF] (the layout
 * Linear.forward_gpu builds, layers.mojo:489-497), b [OutF], y [N,OutF];
 * y[n,o] = sum_k x[n,k] wT[k,o] + b[o] as the seam's CPU kernel
 * _kernel_linear_fw (layers.mojo:436-475) defines it.  Synchronous. */
int32_t mj_launch_linear_fw_h(const float *x, const float *wT, const float *b, float *y,
                              int64_t N, int64_t InF, int64_t OutF, int32_t has_bias);

/* Linear.backward (learn/nn/layers.mojo:519-618, 785-787) for x [N,InF],
 * W [OutF,InF], dy [N,OutF] (device pointers, row-major):
 *   dW[o,i] = sum_n dy[n,o] x[n,i]   (dW [OutF,InF], the layer's layout)
 *   db[o]   = sum_n dy[n,o]          (strict ascending n for N <= 1024,
 *                                     else ascending within row segments)
 *   dx[n,i] = sum_o dy[n,o] W[o,i]   (dx [N,InF])
 * dx and dW run on the fp32 MFMA engine over stride views (no transposed
 * copies).  Any output may be NULL to skip it. */
int32_t mj_linear_backward_f32(const float *x, const float *W, const float *dy, float *dW,
                               float *db, float *dx, int64_t N, int64_t InF, int64_t OutF,
                               void *stream);

/* Host-pointer seams with the signatures of launch_1d_linear_bw_dx / _dw /
 * _db (tensor/gpu/runtime.mojo:636-713, 714-832, 834-903).  Layouts follow
 * the seam's CPU kernels _kernel_linear_bw_dx/_dw/_db (layers.mojo:624-729):
 * w and dW are [OutF,InF].  (The seam's GPU kernels, runtime.mojo:75-119,
 * index w and dW as [InF,OutF]; that layout is not reproduced.)  Synchronous. */
int32_t mj_launch_linear_bw_dx_h(const float *dy, const float *w, float *dx, int64_t N,
                                 int64_t InF, int64_t OutF);
int32_t mj_launch_linear_bw_dw_h(const float *dy, const float *x, float *dW, int64_t N,
                                 int64_t InF, int64_t OutF);
int32_t mj_launch_linear_bw_db_h(const float *dy, float *db, int64_t N, int64_t OutF);

/* Elementwise fp32 activation y = epi(x) over n elements (may alias).
 * Replaces Tensor.relu / silu / gelu (tensor/tensor.mojo:3848,4003,4020 ->
 * apply_unary, tensor/math.mojo:566-638) and ReLU.forward (layers.mojo:134). */
int32_t mj_activation_f32(int32_t epilogue, const float *x, float *y, int64_t n, void *stream);

/* ---- conv2d ------------------------------------------------------------- */

/* Conv2d.forward, NCHW fp32 (learn/nn/conv.mojo:600-681, the naive GPU kernel
 * _gpu_conv2d_fw_kernel, tensor/gpu/runtime.mojo:159-200): x [N,C,H,W],
 * w [OC,C,kH,kW], b [OC] or NULL, y [N,OC,OH,OW] with
 * OH = (H + 2 pH - kH) // sH + 1 (floor), OW likewise; zero padding, the
 * bias after the sum, then `epilogue` (MJ_EPI_NONE for the reference's
 * layer).  One implicit GEMM per image on fp32 MFMA: y[n] = w [OC, C kH kW]
 * @ im2col(x[n]), the im2col gathered by the kernel's loader, nothing
 * materialised.  An empty output (OH or OW <= 0) is MJ_OK with nothing
 * written.  Padded taps are multiplied as zeros where the reference skips
 * them: the same sums for finite weights. */
int32_t mj_conv2d_f32(const float *x, const float *w, const float *b, int32_t epilogue, float *y,
                      int64_t N, int64_t C, int64_t H, int64_t W, int64_t OC, int64_t kH,
                      int64_t kW, int64_t sH, int64_t sW, int64_t pH, int64_t pW, void *stream);

/* Host-pointer seam of launch_1d_conv2d_fw (tensor/gpu/runtime.mojo:376-470):
 * the same arguments (OH, OW as the caller computed them, checked against
 * the geometry: MJ_ERR_SHAPE if they disagree), copy in, mj_conv2d_f32,
 * copy out into y; has_bias = 0 ignores b. */
int32_t mj_launch_conv2d_fw_h(const float *x, const float *w, const float *b, float *y, int64_t N,
                              int64_t C, int64_t H, int64_t W, int64_t OH, int64_t OW, int64_t OC,
                              int64_t kH, int64_t kW, int64_t sH, int64_t sW, int64_t pH,
                              int64_t pW, int32_t has_bias);

/* y = x >= s ? x : s over n fp32 elements (may alias): -0 stays -0 at s = 0,
 * NaN gives s.  Replaces Tensor[Float32].maximum_scalar(s) =
 * where_f32(ge_t(self, s), self, s) (tensor/tensor.mojo:4232), which
 * Converted.forward applies between the quantized layers
 * (learn/api/sequential.mojo:423). */
int32_t mj_maximum_scalar_f32(const float *x, float s, float *y, int64_t n, void *stream);

/* y = Float32(x) over n int64 elements, rounded to nearest even.  Replaces
 * astype_f32_from_int (tensor/cast.mojo:5431-5437), the upcast of
 * Tensor[Int].matmul / matmul_vec (tensor/tensor.mojo:3161-3165,3174-3178). */
int32_t mj_cast_i64_f32(const int64_t *x, float *y, int64_t n, void *stream);

/* ---- bf16 -------------------------------------------------------------- */

/* C[M,N] = bf16(epi(A[M,K] B[N,K]^T + bias)), fp32 accumulation on bf16
 * MFMA.  No reference counterpart: momijo has no bf16 matmul (broadcast.mojo
 * has f64/f32 overloads only, :1531,1677); its result is defined as the fp32
 * engine on exactly upcast bf16 inputs.  Needs K % 8 == 0, lda/ldb/ldc % 8
 * == 0 and 16-byte aligned A, B, C. */
int32_t mj_gemm_bf16_nt(int64_t M, int64_t N, int64_t K,
                        const uint16_t *A, int64_t lda, const uint16_t *B, int64_t ldb,
                        const float *bias, int32_t epilogue,
                        uint16_t *C, int64_t ldc, void *stream);

/* ---- int8: legacy per-tensor W8A8 (QuantLinear) ------------------------- */

/* q[i] = clamp(round(x[i]/scale)) with the MJ_ROUND_LEGACY rule; scale 0 is
 * replaced by 1.  Replaces quantize_symmetric_int8 (learn/api/functional.mojo:
 * 231-247). */
int32_t mj_quantize_symmetric_int8(const float *x, int64_t n, float scale, int8_t *q, void *stream);

/* minmax_out (device fp32 [2]) = {min x, max x} over n > 0 elements: the
 * reduction of MinMaxObserver.observe (learn/api/sequential.mojo:232-250). */
int32_t mj_minmax_f32(const float *x, int64_t n, float *minmax_out, void *stream);

/* *scale_out (device fp32) = max(|min x|, |max x|) / max_q, or 1.0 when n == 0,
 * max_q <= 0 or the magnitude is 0.  Replaces MinMaxObserver.observe +
 * scale_symmetric (learn/api/sequential.mojo:232-263). */
int32_t mj_minmax_scale_symmetric(const float *x, int64_t n, float max_q, float *scale_out,
                                  void *stream);

/* C[M,N] int32 = A[M,K] int8 * B^T, B = w_q [N,K] int8, exact int32
 * accumulation on int8 MFMA.  legacy_literal = 1 instead reads B as
 * reshape(w_q.flat, [K,N]) exactly as matmul_i8_i8_to_i32 does when handed
 * the stride view w_q.transpose() (learn/api/functional.mojo:249-279, :274).
 * K % 16 == 0 with 16-byte aligned A and B runs on int8 MFMA; other shapes
 * take a scalar kernel with the same (exact) result. */
int32_t mj_matmul_i8_i8_to_i32(const int8_t *A, const int8_t *B, int32_t *C,
                               int64_t M, int64_t N, int64_t K, int32_t legacy_literal,
                               void *stream);

/* y[M,N] = float(acc) * sf + b[N] (rounded multiply, then rounded add).
 * Replaces dequantize_i32_to_f32_add_bias (learn/api/functional.mojo:281-302). */
int32_t mj_dequantize_i32_to_f32_add_bias(const int32_t *acc, float sf, const float *b, float *y,
                                          int64_t M, int64_t N, void *stream);

/* y[M,N] = float(acc) * (sx[m] * sw[n]) + b[n], each fp32 operation rounded
 * on its own (sx * sw first); sx may be NULL (the factor is then sw[n]) and
 * b may be NULL.  The per-channel (and per-row) form of
 * dequantize_i32_to_f32_add_bias (learn/api/functional.mojo:281-302), for
 * int32 sums from mj_matmul_i8_i8_to_i32 with per-channel weight scales; it
 * is the epilogue of mj_linear_w8a8 as a separate operator. */
int32_t mj_dequantize_i32_scaled_f32(const int32_t *acc, const float *sx, const float *sw,
                                     const float *b, float *y, int64_t M, int64_t N,
                                     void *stream);

/* QuantLinear.forward (learn/nn/layers.mojo:1681-1685): quantize x [M,K]
 * with s_x, int8 GEMM against w_q [N,K], y = float(acc)*(s_x*s_w) + b.
 * The dequantize is fused into the GEMM epilogue; the int8 copy of x lives in
 * a device workspace the library owns. */
int32_t mj_quant_linear_f32(const float *x, const int8_t *Wq, const float *b,
                            float s_w, float s_x, float *y,
                            int64_t M, int64_t N, int64_t K, int32_t legacy_literal,
                            void *stream);

/* mj_quant_linear_f32 without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  The int8
 * copy of x lives in a static 16 MiB device array owned by the library (one
 * per GPU, held until the process ends), so M*K must be at most 16 MiB - 16
 * bytes (MJ_ERR_UNSUPPORTED otherwise).  Results equal mj_quant_linear_f32's.
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (different streams, or host threads without ordering) race. */
int32_t mj_quant_linear_f32_noalloc(const float *x, const int8_t *Wq, const float *b,
                                    float s_w, float s_x, float *y,
                                    int64_t M, int64_t N, int64_t K, int32_t legacy_literal,
                                    void *stream);

/* ---- int8: per-output-channel weight-only (BASELINE spec) -------------- */

/* Q[N,K] int8 and scales[N] from W[N,K] fp32, one scale per output row.
 * MJ_ROUND_RHE: scale = max|row|/127 (1.0 for an all-zero row),
 *               q = clamp(rne(w/scale), -127, 127).
 * MJ_ROUND_LEGACY: scale = MinMax rule per row (sequential.mojo:252-263),
 *               q by functional.mojo:214-217.
 * The per-tensor reference path is quantize_symmetric_int8 + convert
 * (sequential.mojo:436-450); this is its per-row generalisation. */
int32_t mj_quantize_rowwise_i8(const float *W, int64_t N, int64_t K, int32_t rounding,
                               int8_t *Q, float *scales, void *stream);

/* y[M,N] = bf16(epi((x[M,K] . Q[N,K]^T) * scales[N] + bias[N])) with x bf16,
 * fp32 accumulation.  M <= 16 (and M <= 48 when K is a multiple of 1024 up
 * to 4096) runs the GEMV kernels, larger M the MFMA GEMM with int8 -> bf16
 * conversion in registers.  bias may be NULL.  Needs K % 16 == 0 and 16-byte
 * aligned x, Q, y. */
int32_t mj_linear_w8a16(const uint16_t *x, const int8_t *Q, const float *scales,
                        const float *bias, int32_t epilogue, uint16_t *y,
                        int64_t M, int64_t N, int64_t K, void *stream);

/* Dynamic per-row activation quantize: xq[M,K] int8 and sx[M] fp32 from
 * x[M,K] bf16 by the MJ_ROUND_RHE rule of mj_quantize_rowwise_i8 applied to
 * each row of x (sx[m] = max|x[m,:]|/127, 1.0 for an all-zero row;
 * xq = clamp(rne(x/sx[m]), -127, 127); NaN -> 0).  The activation half of
 * mj_linear_w8a8; the per-tensor reference step it generalises is
 * quantize_symmetric_int8 with the observer's scale (learn/api/
 * functional.mojo:231-247, sequential.mojo:232-263). */
int32_t mj_quantize_rows_bf16_i8(const uint16_t *x, int64_t M, int64_t K, int8_t *xq, float *sx,
                                 void *stream);

/* W8A8 Linear with dynamic activation scales:
 *   sx, xq = mj_quantize_rows_bf16_i8(x)
 *   y[m,n] = bf16(epi(float(xq[m,:] . Q[n,:]) * (sx[m] * scales[n]) + bias[n]))
 * with the int32 dot product exact on int8 MFMA and the epilogue rounded
 * step by step in fp32 (sx*scales, then the product, then the bias).  It is
 * QuantLinear.forward (learn/nn/layers.mojo:1681-1685: quantize x, int8
 * matmul, dequantize + bias) with per-row scales for x and per-channel scales
 * for the weights instead of two per-tensor scales.  Same arguments as
 * mj_linear_w8a16; bias may be NULL; xq and sx live in the stream's
 * workspace.  Needs K % 16 == 0, K <= 131072 (the int32 sums cannot
 * overflow) and 16-byte aligned x, Q. */
int32_t mj_linear_w8a8(const uint16_t *x, const int8_t *Q, const float *scales,
                       const float *bias, int32_t epilogue, uint16_t *y,
                       int64_t M, int64_t N, int64_t K, void *stream);

/* Llama-style FFN on W8A16 weights (composition of Linear, silu32 and the
 * elementwise product, tensor/tensor.mojo:4373):
 *   h[M,I] = bf16(silu(x Wg^T * sg) * (x Wu^T * su))   (one fused GEMM; bf16-output silu)
 *   y[M,H] = bf16((h Wd^T) * sd)
 * Wg, Wu [I,K]; Wd [H,I]; h is a caller-owned [M,I] buffer.  The gate/up
 * runs as a GEMV at 1-4 x rows (K <= 16384) and at 5-32 rows when K = 1024 j
 * <= 4096, the down projection as mj_linear_w8a16 runs [M,I] x [H,I]^T; with
 * both as GEMVs the call needs no workspace and can be captured into a HIP
 * graph. */
int32_t mj_mlp_w8a16(const uint16_t *x, const int8_t *Wg, const float *sg,
                     const int8_t *Wu, const float *su, const int8_t *Wd, const float *sd,
                     uint16_t *h, uint16_t *y, int64_t M, int64_t K, int64_t I, int64_t H,
                     void *stream);

/* ---- device memory and streams (api_host.hip) -------------------------- */
/* For a caller that keeps tensors resident across calls (e.g. QuantLinear's
 * w_q uploaded once).  momijo itself has no device-resident tensors
 * (tensor/device.mojo:258-302: to_device round-trips through the host); the
 * reference seam allocates per call with DeviceContext.enqueue_create_buffer
 * (tensor/gpu/runtime.mojo:563-570), which these replace. */

/* *ptr = device allocation of `bytes` bytes (NULL for 0). */
int32_t mj_malloc(void **ptr, int64_t bytes);
/* Frees an mj_malloc allocation (NULL is a no-op). */
int32_t mj_free(void *ptr);
/* Synchronous copies: ordered after the work queued on `stream` (NULL = the
 * null stream) and complete when they return, like the reference's
 * enqueue_copy + synchronize (runtime.mojo:586-598). */
int32_t mj_memcpy_htod(void *dst_device, const void *src_host, int64_t bytes, void *stream);
int32_t mj_memcpy_dtoh(void *dst_host, const void *src_device, int64_t bytes, void *stream);
/* Asynchronous device-to-device copy on `stream`. */
int32_t mj_memcpy_dtod(void *dst_device, const void *src_device, int64_t bytes, void *stream);
/* Non-blocking stream at the default priority; destroy NULL is a no-op.
 * The reference has no stream concept (one DeviceContext per call,
 * runtime.mojo:556). */
int32_t mj_stream_create(void **stream);
int32_t mj_stream_destroy(void *stream);
/* Waits for all work on the device (DeviceContext.synchronize,
 * runtime.mojo:596). */
int32_t mj_device_synchronize(void);

/* ---- host-pointer variants (api_host.hip) -------------------------------- */
/* Same arguments and results as the device entry point without the `_h`
 * suffix, with every pointer a HOST pointer: inputs are copied to one device
 * block, the operator runs, and outputs are copied back before the call
 * returns (the reference seam's copy-in / copy-out contract,
 * tensor/gpu/runtime.mojo:556-604).  Strided operands are copied over the
 * extent their strides span; outputs with a leading dimension are written
 * row by row, leaving padding untouched.  This is what a momijo Tensor[T],
 * whose storage is a host List[T] (tensor/tensor.mojo:776-905), binds. */

/* Tensor.matmul / tensor.matmul Float32 (tensor/tensor.mojo:3168-3169,
 * tensor/__init__.mojo:123 -> matmul_core_mm, tensor/broadcast.mojo:
 * 1612-1673), with the tensor's _strides. */
int32_t mj_matmul_f32_h(int64_t M, int64_t N, int64_t K,
                        const float *A, int64_t sAm, int64_t sAk,
                        const float *B, int64_t sBk, int64_t sBn,
                        const float *bias, int32_t epilogue, float *C, int64_t ldc);
/* Tensor.matmul_vec Float32 (tensor/tensor.mojo:3180 -> matmul_core_vec,
 * tensor/broadcast.mojo:1543-1608). */
int32_t mj_matvec_f32_h(int64_t M, int64_t N, const float *A, int64_t sAm, int64_t sAn,
                        const float *x, int64_t sx, float *y);
/* Float64 matmul / matmul2d (tensor/broadcast.mojo:1466-1538,
 * tensor/math.mojo:7838-7880). */
int32_t mj_matmul_f64_h(int64_t M, int64_t N, int64_t K,
                        const double *A, int64_t sAm, int64_t sAk,
                        const double *B, int64_t sBk, int64_t sBn, double *C, int64_t ldc);
/* Float64 matmul_core_vec (tensor/broadcast.mojo:1397-1464). */
int32_t mj_matvec_f64_h(int64_t M, int64_t N, const double *A, int64_t sAm, int64_t sAn,
                        const double *x, int64_t sx, double *y);
/* tensordot(A, B, axes=1) Float32 (tensor/broadcast.mojo:1694-1900). */
int32_t mj_tensordot_f32_h(int32_t batch_rank, const int64_t *batch_shape,
                           const int64_t *a_batch_strides, const int64_t *b_batch_strides,
                           int64_t M, int64_t N, int64_t K,
                           const float *A, int64_t sAm, int64_t sAk,
                           const float *B, int64_t sBk, int64_t sBn, float *C);
/* Linear.forward (learn/nn/layers.mojo:383-433, 510-516) + fused activation. */
int32_t mj_linear_f32_h(const float *x, const float *W, const float *bias, int32_t epilogue,
                        float *y, int64_t N, int64_t InF, int64_t OutF);
/* Linear.backward (learn/nn/layers.mojo:519-618, 785-787). */
int32_t mj_linear_backward_f32_h(const float *x, const float *W, const float *dy, float *dW,
                                 float *db, float *dx, int64_t N, int64_t InF, int64_t OutF);
/* The MATMUL2D tape rule in Float64 (tensor/autograd.mojo:1542-1555); with
 * accumulate != 0 dA / dB are read as well as written. */
int32_t mj_matmul_backward_f64_h(int64_t M, int64_t N, int64_t K, const double *A,
                                 const double *B, const double *G, double *dA, double *dB,
                                 int32_t accumulate);
/* The MATMUL2D tape rule in Float32 (tensor/autograd.mojo:1542-1555). */
int32_t mj_matmul_backward_f32_h(int64_t M, int64_t N, int64_t K, const float *A,
                                 const float *B, const float *G, float *dA, float *dB,
                                 int32_t accumulate);
/* Tensor.relu / gelu / silu (tensor/tensor.mojo:3848,4003,4020). */
int32_t mj_activation_f32_h(int32_t epilogue, const float *x, float *y, int64_t n);
/* bf16 NT GEMM (no reference counterpart; see mj_gemm_bf16_nt). */
int32_t mj_gemm_bf16_nt_h(int64_t M, int64_t N, int64_t K,
                          const uint16_t *A, int64_t lda, const uint16_t *B, int64_t ldb,
                          const float *bias, int32_t epilogue, uint16_t *C, int64_t ldc);
/* quantize_symmetric_int8 (learn/api/functional.mojo:231-247). */
int32_t mj_quantize_symmetric_int8_h(const float *x, int64_t n, float scale, int8_t *q);
/* MinMaxObserver.observe reduction (learn/api/sequential.mojo:232-250);
 * minmax_out is host float[2]. */
int32_t mj_minmax_f32_h(const float *x, int64_t n, float *minmax_out);
/* MinMaxObserver.observe + scale_symmetric (learn/api/sequential.mojo:
 * 232-263); scale_out is a host float. */
int32_t mj_minmax_scale_symmetric_h(const float *x, int64_t n, float max_q, float *scale_out);
/* matmul_i8_i8_to_i32 (learn/api/functional.mojo:249-279). */
int32_t mj_matmul_i8_i8_to_i32_h(const int8_t *A, const int8_t *B, int32_t *C,
                                 int64_t M, int64_t N, int64_t K, int32_t legacy_literal);
/* dequantize_i32_to_f32_add_bias (learn/api/functional.mojo:281-302). */
int32_t mj_dequantize_i32_to_f32_add_bias_h(const int32_t *acc, float sf, const float *b,
                                            float *y, int64_t M, int64_t N);
/* Per-channel dequantize (see mj_dequantize_i32_scaled_f32); sx and b may be
 * NULL. */
int32_t mj_dequantize_i32_scaled_f32_h(const int32_t *acc, const float *sx, const float *sw,
                                       const float *b, float *y, int64_t M, int64_t N);
/* QuantLinear.forward (learn/nn/layers.mojo:1681-1685). */
int32_t mj_quant_linear_f32_h(const float *x, const int8_t *Wq, const float *b,
                              float s_w, float s_x, float *y,
                              int64_t M, int64_t N, int64_t K, int32_t legacy_literal);
/* Per-row quantize/pack (generalises quantize_symmetric_int8 + convert,
 * learn/api/sequential.mojo:436-450). */
int32_t mj_quantize_rowwise_i8_h(const float *W, int64_t N, int64_t K, int32_t rounding,
                                 int8_t *Q, float *scales);
/* W8A16 Linear (no reference counterpart; see mj_linear_w8a16). */
int32_t mj_linear_w8a16_h(const uint16_t *x, const int8_t *Q, const float *scales,
                          const float *bias, int32_t epilogue, uint16_t *y,
                          int64_t M, int64_t N, int64_t K);
/* W8A8 Linear with dynamic activation scales (see mj_linear_w8a8). */
int32_t mj_linear_w8a8_h(const uint16_t *x, const int8_t *Q, const float *scales,
                         const float *bias, int32_t epilogue, uint16_t *y,
                         int64_t M, int64_t N, int64_t K);
/* W8A16 FFN (no reference counterpart; see mj_mlp_w8a16); h may be NULL,
 * then the intermediate stays on the device. */
int32_t mj_mlp_w8a16_h(const uint16_t *x, const int8_t *Wg, const float *sg,
                       const int8_t *Wu, const float *su, const int8_t *Wd, const float *sd,
                       uint16_t *h, uint16_t *y, int64_t M, int64_t K, int64_t I, int64_t H);

#ifdef __cplusplus
}
#endif

#endif /* MOMIJO_HIP_H */
