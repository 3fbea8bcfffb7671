// Host-memory half of the C ABI (declared in include/momijo_hip.h):
//
//  * device memory and streams for a caller that keeps its tensors resident
//    (mj_malloc / mj_free / mj_memcpy_* / mj_stream_*), and
//  * a host-pointer (_h) variant of every operator entry point, for callers
//    whose tensors live in host memory, as momijo's do (Tensor[T] stores a
//    List[T], tensor/tensor.mojo:776-905; to_device round-trips through the
//    host, tensor/device.mojo:258-302).  Each _h call copies its inputs to
//    one device block, runs the device entry point on the null stream, waits,
//    and copies the outputs back: the ownership model of the reference's own
//    seam (launch_1d_linear_fw, tensor/gpu/runtime.mojo:539-604).  Strided
//    operands are copied over the extent their strides span, so zero-copy
//    transpose views (tensor/transform.mojo:2107-2136) stay views.
//
// Every entry point validates its arguments, returns an int32 status and
// never throws; host pointers may alias nothing the device sees.
#include <hip/hip_runtime.h>

#include <cstring>

#include "../../include/momijo_hip.h"
#include "abi_util.h"
#include "launch.h"

using namespace mj_abi;

namespace {

constexpr size_t F4 = sizeof(float), F8 = sizeof(double);

// bytes of an optional host operand: 0 when absent
size_t opt_bytes(const void *p, size_t bytes) { return p ? bytes : 0; }

// 2-D output of `rows` rows of `cols` elements at leading dimension ld
HostArg out2d(void *host, int64_t rows, int64_t cols, int64_t ld, size_t esz) {
  HostArg a{nullptr, host, (size_t)span2(rows, cols, ld, 1) * esz};
  a.rows = rows;
  a.width = (size_t)cols * esz;
  a.pitch = (size_t)ld * esz;
  return a;
}

}  // namespace

extern "C" {

// ------------------------------------------------------------------ memory
int32_t mj_malloc(void **ptr, int64_t bytes) {
  if (!ptr) return fail(MJ_ERR_ARG, "null result pointer");
  *ptr = nullptr;
  if (bytes < 0) return fail(MJ_ERR_ARG, "negative size");
  if (bytes == 0) return MJ_OK;
  if (hipMalloc(ptr, (size_t)bytes) != hipSuccess) {
    (void)hipGetLastError();
    *ptr = nullptr;
    return fail(MJ_ERR_ALLOC, "hipMalloc(%lld) failed", (long long)bytes);
  }
  return MJ_OK;
}

int32_t mj_free(void *ptr) {
  if (!ptr) return MJ_OK;
  return hip_status(hipFree(ptr), "hipFree");
}

static int32_t copy_sync(void *dst, const void *src, int64_t bytes, hipMemcpyKind kind,
                         void *stream, const char *what) {
  if (bytes < 0) return fail(MJ_ERR_ARG, "negative size");
  if (bytes == 0) return MJ_OK;
  if (!dst || !src) return fail(MJ_ERR_ARG, "null pointer");
  if (!stream) return hip_status(hipMemcpy(dst, src, (size_t)bytes, kind), what);
  // ordered after the work already queued on `stream`, complete on return
  if (int32_t st = hip_status(hipMemcpyAsync(dst, src, (size_t)bytes, kind, S(stream)), what))
    return st;
  return hip_status(hipStreamSynchronize(S(stream)), what);
}

int32_t mj_memcpy_htod(void *dst, const void *src, int64_t bytes, void *stream) {
  return copy_sync(dst, src, bytes, hipMemcpyHostToDevice, stream, "host to device copy");
}

int32_t mj_memcpy_dtoh(void *dst, const void *src, int64_t bytes, void *stream) {
  return copy_sync(dst, src, bytes, hipMemcpyDeviceToHost, stream, "device to host copy");
}

int32_t mj_memcpy_dtod(void *dst, const void *src, int64_t bytes, void *stream) {
  if (bytes < 0) return fail(MJ_ERR_ARG, "negative size");
  if (bytes == 0) return MJ_OK;
  if (!dst || !src) return fail(MJ_ERR_ARG, "null pointer");
  return hip_status(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDeviceToDevice, S(stream)),
                    "device to device copy");
}

int32_t mj_stream_create(void **stream) {
  if (!stream) return fail(MJ_ERR_ARG, "null result pointer");
  *stream = nullptr;
  hipStream_t s = nullptr;
  // default priority (streams of other priorities are not used here)
  if (int32_t st = hip_status(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "stream create"))
    return st;
  *stream = (void *)s;
  return MJ_OK;
}

int32_t mj_stream_destroy(void *stream) {
  if (!stream) return MJ_OK;
  return hip_status(hipStreamDestroy(S(stream)), "stream destroy");
}

int32_t mj_device_synchronize(void) {
  return hip_status(hipDeviceSynchronize(), "hipDeviceSynchronize");
}

// ------------------------------------------------------------------ fp32 / fp64
int32_t mj_matmul_f32_h(int64_t M, int64_t N, int64_t K, const float *A, int64_t sAm,
                        int64_t sAk, const float *B, int64_t sBk, int64_t sBn, const float *bias,
                        int32_t epilogue, float *C, int64_t ldc) {
  if (int32_t s = check_dims(M, N, K)) return s;
  if (!valid_epi(epilogue)) return fail(MJ_ERR_ARG, "unknown epilogue %d", epilogue);
  if (M == 0 || N == 0) return MJ_OK;
  if (!C || (K > 0 && (!A || !B))) return fail(MJ_ERR_ARG, "null operand");
  if (ldc < N) return fail(MJ_ERR_SHAPE, "ldc (%lld) < N (%lld)", (long long)ldc, (long long)N);
  if (sAm < 0 || sAk < 0 || sBk < 0 || sBn < 0) return fail(MJ_ERR_UNSUPPORTED, "negative stride");
  HostArg a[4] = {{A, nullptr, (size_t)span2(M, K, sAm, sAk) * F4},
                  {B, nullptr, (size_t)span2(K, N, sBk, sBn) * F4},
                  {bias, nullptr, opt_bytes(bias, (size_t)N * F4)},
                  out2d(C, M, N, ldc, F4)};
  return with_device_copies(a, 4, [&](void **d) {
    return mj_matmul_f32(M, N, K, (const float *)d[0], sAm, sAk, (const float *)d[1], sBk, sBn,
                         (const float *)d[2], epilogue, (float *)d[3], ldc, nullptr);
  });
}

int32_t mj_matvec_f32_h(int64_t M, int64_t N, const float *A, int64_t sAm, int64_t sAn,
                        const float *x, int64_t sx, float *y) {
  if (int32_t s = check_dims(M, N, 0)) return s;
  if (M == 0) return MJ_OK;
  if (!y || (N > 0 && (!A || !x))) return fail(MJ_ERR_ARG, "null operand");
  if (sAm < 0 || sAn < 0 || sx < 0) return fail(MJ_ERR_UNSUPPORTED, "negative stride");
  HostArg a[3] = {{A, nullptr, (size_t)span2(M, N, sAm, sAn) * F4},
                  {x, nullptr, (size_t)span2(1, N, 0, sx) * F4},
                  {nullptr, y, (size_t)M * F4}};
  return with_device_copies(a, 3, [&](void **d) {
    return mj_matvec_f32(M, N, (const float *)d[0], sAm, sAn, (const float *)d[1], sx,
                         (float *)d[2], nullptr);
  });
}

int32_t mj_matmul_f64_h(int64_t M, int64_t N, int64_t K, const double *A, int64_t sAm,
                        int64_t sAk, const double *B, int64_t sBk, int64_t sBn, double *C,
                        int64_t ldc) {
  if (int32_t s = check_dims(M, N, K)) return s;
  if (M == 0 || N == 0) return MJ_OK;
  if (!C || (K > 0 && (!A || !B))) return fail(MJ_ERR_ARG, "null operand");
  if (ldc < N) return fail(MJ_ERR_SHAPE, "ldc (%lld) < N (%lld)", (long long)ldc, (long long)N);
  if (sAm < 0 || sAk < 0 || sBk < 0 || sBn < 0) return fail(MJ_ERR_UNSUPPORTED, "negative stride");
  HostArg a[3] = {{A, nullptr, (size_t)span2(M, K, sAm, sAk) * F8},
                  {B, nullptr, (size_t)span2(K, N, sBk, sBn) * F8},
                  out2d(C, M, N, ldc, F8)};
  return with_device_copies(a, 3, [&](void **d) {
    return mj_matmul_f64(M, N, K, (const double *)d[0], sAm, sAk, (const double *)d[1], sBk, sBn,
                         (double *)d[2], ldc, nullptr);
  });
}

int32_t mj_matvec_f64_h(int64_t M, int64_t N, const double *A, int64_t sAm, int64_t sAn,
                        const double *x, int64_t sx, double *y) {
  if (int32_t s = check_dims(M, N, 0)) return s;
  if (M == 0) return MJ_OK;
  if (!y || (N > 0 && (!A || !x))) return fail(MJ_ERR_ARG, "null operand");
  if (sAm < 0 || sAn < 0 || sx < 0) return fail(MJ_ERR_UNSUPPORTED, "negative stride");
  HostArg a[3] = {{A, nullptr, (size_t)span2(M, N, sAm, sAn) * F8},
                  {x, nullptr, (size_t)span2(1, N, 0, sx) * F8},
                  {nullptr, y, (size_t)M * F8}};
  return with_device_copies(a, 3, [&](void **d) {
    return mj_matvec_f64(M, N, (const double *)d[0], sAm, sAn, (const double *)d[1], sx,
                         (double *)d[2], nullptr);
  });
}

int32_t mj_tensordot_f32_h(int32_t batch_rank, const int64_t *batch_shape,
                           const int64_t *a_batch_strides, const int64_t *b_batch_strides,
                           int64_t M, int64_t N, int64_t K, const float *A, int64_t sAm,
                           int64_t sAk, const float *B, int64_t sBk, int64_t sBn, float *C) {
  if (int32_t s = check_dims(M, N, K)) return s;
  if (batch_rank < 0 || batch_rank > mj::BatchDesc::kMaxRank)
    return fail(MJ_ERR_UNSUPPORTED, "batch rank must be 0..%d", mj::BatchDesc::kMaxRank);
  if (batch_rank > 0 && (!batch_shape || !a_batch_strides || !b_batch_strides))
    return fail(MJ_ERR_ARG, "null batch description");
  int64_t batches = 1, a_last = 0, b_last = 0;
  for (int d = 0; d < batch_rank; ++d) {
    if (batch_shape[d] < 0) return fail(MJ_ERR_ARG, "negative batch extent");
    if (a_batch_strides[d] < 0 || b_batch_strides[d] < 0)
      return fail(MJ_ERR_UNSUPPORTED, "negative stride");
    batches *= batch_shape[d];
    if (batch_shape[d] > 0) {
      a_last += (batch_shape[d] - 1) * a_batch_strides[d];
      b_last += (batch_shape[d] - 1) * b_batch_strides[d];
    }
  }
  if (batches == 0 || M == 0 || N == 0) return MJ_OK;
  if (!C || (K > 0 && (!A || !B))) return fail(MJ_ERR_ARG, "null operand");
  if (sAm < 0 || sAk < 0 || sBk < 0 || sBn < 0) return fail(MJ_ERR_UNSUPPORTED, "negative stride");
  const int64_t a_span = K > 0 ? a_last + span2(M, K, sAm, sAk) : 0;
  const int64_t b_span = K > 0 ? b_last + span2(K, N, sBk, sBn) : 0;
  HostArg a[3] = {{A, nullptr, (size_t)a_span * F4},
                  {B, nullptr, (size_t)b_span * F4},
                  {nullptr, C, (size_t)(batches * M * N) * F4}};
  return with_device_copies(a, 3, [&](void **d) {
    return mj_tensordot_f32(batch_rank, batch_shape, a_batch_strides, b_batch_strides, M, N, K,
                            (const float *)d[0], sAm, sAk, (const float *)d[1], sBk, sBn,
                            (float *)d[2], nullptr);
  });
}

int32_t mj_linear_f32_h(const float *x, const float *W, const float *bias, int32_t epilogue,
                        float *y, int64_t N, int64_t InF, int64_t OutF) {
  // y = x W^T: B = W^T is the stride view (sBk = 1, sBn = InF) of W
  return mj_matmul_f32_h(N, OutF, InF, x, InF, 1, W, 1, InF, bias, epilogue, y, OutF);
}

int32_t mj_linear_backward_f32_h(const float *x, const float *W, const float *dy, float *dW,
                                 float *db, float *dx, int64_t N, int64_t InF, int64_t OutF) {
  if (int32_t s = check_dims(N, InF, OutF)) return s;
  const bool want_dx = dx && N > 0 && InF > 0;
  const bool want_dW = dW && OutF > 0 && InF > 0;
  const bool want_db = db && OutF > 0;
  if ((want_dx || want_dW || want_db) && N > 0 && !dy) return fail(MJ_ERR_ARG, "null dy");
  if (want_dx && OutF > 0 && !W) return fail(MJ_ERR_ARG, "null W");
  if (want_dW && N > 0 && !x) return fail(MJ_ERR_ARG, "null x");
  if (!want_dx && !want_dW && !want_db) return MJ_OK;
  HostArg a[6] = {{want_dW ? x : nullptr, nullptr, want_dW ? (size_t)(N * InF) * F4 : 0},
                  {want_dx ? W : nullptr, nullptr, want_dx ? (size_t)(OutF * InF) * F4 : 0},
                  {dy, nullptr, (size_t)(N * OutF) * F4},
                  {nullptr, want_dW ? dW : nullptr, want_dW ? (size_t)(OutF * InF) * F4 : 0},
                  {nullptr, want_db ? db : nullptr, want_db ? (size_t)OutF * F4 : 0},
                  {nullptr, want_dx ? dx : nullptr, want_dx ? (size_t)(N * InF) * F4 : 0}};
  return with_device_copies(a, 6, [&](void **d) {
    return mj_linear_backward_f32((const float *)d[0], (const float *)d[1], (const float *)d[2],
                                  (float *)d[3], (float *)d[4], (float *)d[5], N, InF, OutF,
                                  nullptr);
  });
}

int32_t mj_matmul_backward_f64_h(int64_t M, int64_t N, int64_t K, const double *A,
                                 const double *B, const double *G, double *dA, double *dB,
                                 int32_t accumulate) {
  if (int32_t s = check_dims(M, N, K)) return s;
  const bool want_dA = dA && M > 0 && K > 0;
  const bool want_dB = dB && K > 0 && N > 0;
  if ((want_dA || want_dB) && N > 0 && M > 0 && !G) return fail(MJ_ERR_ARG, "null G");
  if (want_dA && N > 0 && !B) return fail(MJ_ERR_ARG, "null B");
  if (want_dB && M > 0 && !A) return fail(MJ_ERR_ARG, "null A");
  if (!want_dA && !want_dB) return MJ_OK;
  // with accumulate the gradients are read as well as written
  HostArg a[5] = {{want_dB ? A : nullptr, nullptr, want_dB ? (size_t)(M * K) * F8 : 0},
                  {want_dA ? B : nullptr, nullptr, want_dA ? (size_t)(K * N) * F8 : 0},
                  {G, nullptr, (size_t)(M * N) * F8},
                  {want_dA && accumulate ? dA : nullptr, want_dA ? dA : nullptr,
                   want_dA ? (size_t)(M * K) * F8 : 0},
                  {want_dB && accumulate ? dB : nullptr, want_dB ? dB : nullptr,
                   want_dB ? (size_t)(K * N) * F8 : 0}};
  return with_device_copies(a, 5, [&](void **d) {
    return mj_matmul_backward_f64(M, N, K, (const double *)d[0], (const double *)d[1],
                                  (const double *)d[2], (double *)d[3], (double *)d[4],
                                  accumulate, nullptr);
  });
}

int32_t mj_matmul_backward_f32_h(int64_t M, int64_t N, int64_t K, const float *A,
                                 const float *B, const float *G, float *dA, float *dB,
                                 int32_t accumulate) {
  if (int32_t s = check_dims(M, N, K)) return s;
  const bool want_dA = dA && M > 0 && K > 0;
  const bool want_dB = dB && K > 0 && N > 0;
  if ((want_dA || want_dB) && N > 0 && M > 0 && !G) return fail(MJ_ERR_ARG, "null G");
  if (want_dA && N > 0 && !B) return fail(MJ_ERR_ARG, "null B");
  if (want_dB && M > 0 && !A) return fail(MJ_ERR_ARG, "null A");
  if (!want_dA && !want_dB) return MJ_OK;
  HostArg a[5] = {{want_dB ? A : nullptr, nullptr, want_dB ? (size_t)(M * K) * F4 : 0},
                  {want_dA ? B : nullptr, nullptr, want_dA ? (size_t)(K * N) * F4 : 0},
                  {G, nullptr, (size_t)(M * N) * F4},
                  {want_dA && accumulate ? dA : nullptr, want_dA ? dA : nullptr,
                   want_dA ? (size_t)(M * K) * F4 : 0},
                  {want_dB && accumulate ? dB : nullptr, want_dB ? dB : nullptr,
                   want_dB ? (size_t)(K * N) * F4 : 0}};
  return with_device_copies(a, 5, [&](void **d) {
    return mj_matmul_backward_f32(M, N, K, (const float *)d[0], (const float *)d[1],
                                  (const float *)d[2], (float *)d[3], (float *)d[4], accumulate,
                                  nullptr);
  });
}

int32_t mj_activation_f32_h(int32_t epilogue, const float *x, float *y, int64_t n) {
  if (!valid_epi(epilogue)) return fail(MJ_ERR_ARG, "unknown epilogue %d", epilogue);
  if (n < 0) return fail(MJ_ERR_ARG, "negative size");
  if (n == 0) return MJ_OK;
  if (!x || !y) return fail(MJ_ERR_ARG, "null operand");
  HostArg a[2] = {{x, nullptr, (size_t)n * F4}, {nullptr, y, (size_t)n * F4}};
  return with_device_copies(a, 2, [&](void **d) {
    return mj_activation_f32(epilogue, (const float *)d[0], (float *)d[1], n, nullptr);
  });
}

// ------------------------------------------------------------------ bf16
int32_t mj_gemm_bf16_nt_h(int64_t M, int64_t N, int64_t K, const uint16_t *A, int64_t lda,
                          const uint16_t *B, int64_t ldb, const float *bias, int32_t epilogue,
                          uint16_t *C, int64_t ldc) {
  if (int32_t s = check_dims(M, N, K)) return s;
  if (!valid_epi(epilogue)) return fail(MJ_ERR_ARG, "unknown epilogue %d", epilogue);
  if (M == 0 || N == 0) return MJ_OK;
  if (!C || (K > 0 && (!A || !B))) return fail(MJ_ERR_ARG, "null operand");
  if (lda < K || ldb < K || ldc < N) return fail(MJ_ERR_SHAPE, "leading dimension too small");
  HostArg a[4] = {{A, nullptr, (size_t)span2(M, K, lda, 1) * 2},
                  {B, nullptr, (size_t)span2(N, K, ldb, 1) * 2},
                  {bias, nullptr, opt_bytes(bias, (size_t)N * F4)},
                  out2d(C, M, N, ldc, 2)};
  return with_device_copies(a, 4, [&](void **d) {
    return mj_gemm_bf16_nt(M, N, K, (const uint16_t *)d[0], lda, (const uint16_t *)d[1], ldb,
                           (const float *)d[2], epilogue, (uint16_t *)d[3], ldc, nullptr);
  });
}

// ------------------------------------------------------------------ int8 legacy
int32_t mj_quantize_symmetric_int8_h(const float *x, int64_t n, float scale, int8_t *q) {
  if (n < 0) return fail(MJ_ERR_ARG, "negative size");
  if (n == 0) return MJ_OK;
  if (!x || !q) return fail(MJ_ERR_ARG, "null operand");
  HostArg a[2] = {{x, nullptr, (size_t)n * F4}, {nullptr, q, (size_t)n}};
  return with_device_copies(a, 2, [&](void **d) {
    return mj_quantize_symmetric_int8((const float *)d[0], n, scale, (int8_t *)d[1], nullptr);
  });
}

int32_t mj_minmax_f32_h(const float *x, int64_t n, float *minmax_out) {
  if (n <= 0) return fail(MJ_ERR_ARG, "minmax needs n > 0");
  if (!x || !minmax_out) return fail(MJ_ERR_ARG, "null operand");
  HostArg a[2] = {{x, nullptr, (size_t)n * F4}, {nullptr, minmax_out, 2 * F4}};
  return with_device_copies(a, 2, [&](void **d) {
    return mj_minmax_f32((const float *)d[0], n, (float *)d[1], nullptr);
  });
}

int32_t mj_minmax_scale_symmetric_h(const float *x, int64_t n, float max_q, float *scale_out) {
  if (n < 0) return fail(MJ_ERR_ARG, "negative size");
  if (!scale_out || (n > 0 && !x)) return fail(MJ_ERR_ARG, "null operand");
  HostArg a[2] = {{n > 0 ? x : nullptr, nullptr, (size_t)n * F4}, {nullptr, scale_out, F4}};
  return with_device_copies(a, 2, [&](void **d) {
    return mj_minmax_scale_symmetric((const float *)d[0], n, max_q, (float *)d[1], nullptr);
  });
}

int32_t mj_matmul_i8_i8_to_i32_h(const int8_t *A, const int8_t *B, int32_t *C, int64_t M,
                                 int64_t N, int64_t K, int32_t legacy_literal) {
  if (int32_t s = check_dims(M, N, K)) return s;
  if (M == 0 || N == 0) return MJ_OK;
  if (!C || (K > 0 && (!A || !B))) return fail(MJ_ERR_ARG, "null operand");
  HostArg a[3] = {{A, nullptr, (size_t)(M * K)}, {B, nullptr, (size_t)(N * K)},
                  {nullptr, C, (size_t)(M * N) * 4}};
  return with_device_copies(a, 3, [&](void **d) {
    return mj_matmul_i8_i8_to_i32((const int8_t *)d[0], (const int8_t *)d[1], (int32_t *)d[2], M,
                                  N, K, legacy_literal, nullptr);
  });
}

int32_t mj_dequantize_i32_to_f32_add_bias_h(const int32_t *acc, float sf, const float *b,
                                            float *y, int64_t M, int64_t N) {
  if (int32_t s = check_dims(M, N, 0)) return s;
  if (M == 0 || N == 0) return MJ_OK;
  if (!acc || !b || !y) return fail(MJ_ERR_ARG, "null operand");
  HostArg a[3] = {{acc, nullptr, (size_t)(M * N) * 4}, {b, nullptr, (size_t)N * F4},
                  {nullptr, y, (size_t)(M * N) * F4}};
  return with_device_copies(a, 3, [&](void **d) {
    return mj_dequantize_i32_to_f32_add_bias((const int32_t *)d[0], sf, (const float *)d[1],
                                             (float *)d[2], M, N, nullptr);
  });
}

int32_t mj_quant_linear_f32_h(const float *x, const int8_t *Wq, const float *b, float s_w,
                              float s_x, float *y, int64_t M, int64_t N, int64_t K,
                              int32_t legacy_literal) {
  if (int32_t s = check_dims(M, N, K)) return s;
  if (M == 0 || N == 0) return MJ_OK;
  if (!y || !b || (K > 0 && (!x || !Wq))) return fail(MJ_ERR_ARG, "null operand");
  HostArg a[4] = {{x, nullptr, (size_t)(M * K) * F4}, {Wq, nullptr, (size_t)(N * K)},
                  {b, nullptr, (size_t)N * F4}, {nullptr, y, (size_t)(M * N) * F4}};
  return with_device_copies(a, 4, [&](void **d) {
    return mj_quant_linear_f32((const float *)d[0], (const int8_t *)d[1], (const float *)d[2],
                               s_w, s_x, (float *)d[3], M, N, K, legacy_literal, nullptr);
  });
}

// ------------------------------------------------------------------ int8 per-channel
int32_t mj_quantize_rowwise_i8_h(const float *W, int64_t N, int64_t K, int32_t rounding,
                                 int8_t *Q, float *scales) {
  if (int32_t s = check_dims(N, 0, K)) return s;
  if (rounding != MJ_ROUND_RHE && rounding != MJ_ROUND_LEGACY)
    return fail(MJ_ERR_ARG, "unknown rounding %d", rounding);
  if (N == 0) return MJ_OK;
  if (K == 0) return fail(MJ_ERR_SHAPE, "K must be positive");
  if (!W || !Q || !scales) return fail(MJ_ERR_ARG, "null operand");
  HostArg a[3] = {{W, nullptr, (size_t)(N * K) * F4}, {nullptr, Q, (size_t)(N * K)},
                  {nullptr, scales, (size_t)N * F4}};
  return with_device_copies(a, 3, [&](void **d) {
    return mj_quantize_rowwise_i8((const float *)d[0], N, K, rounding, (int8_t *)d[1],
                                  (float *)d[2], nullptr);
  });
}

int32_t mj_linear_w8a16_h(const uint16_t *x, const int8_t *Q, const float *scales,
                          const float *bias, int32_t epilogue, uint16_t *y, int64_t M, int64_t N,
                          int64_t K) {
  if (int32_t s = check_dims(M, N, K)) return s;
  if (!valid_epi(epilogue)) return fail(MJ_ERR_ARG, "unknown epilogue %d", epilogue);
  if (M == 0 || N == 0) return MJ_OK;
  if (!y || !scales || (K > 0 && (!x || !Q))) return fail(MJ_ERR_ARG, "null operand");
  HostArg a[5] = {{x, nullptr, (size_t)(M * K) * 2}, {Q, nullptr, (size_t)(N * K)},
                  {scales, nullptr, (size_t)N * F4}, {bias, nullptr, opt_bytes(bias, (size_t)N * F4)},
                  {nullptr, y, (size_t)(M * N) * 2}};
  return with_device_copies(a, 5, [&](void **d) {
    return mj_linear_w8a16((const uint16_t *)d[0], (const int8_t *)d[1], (const float *)d[2],
                           (const float *)d[3], epilogue, (uint16_t *)d[4], M, N, K, nullptr);
  });
}

int32_t mj_dequantize_i32_scaled_f32_h(const int32_t *acc, const float *sx, const float *sw,
                                       const float *b, float *y, int64_t M, int64_t N) {
  if (int32_t s = check_dims(M, N, 0)) return s;
  if (M == 0 || N == 0) return MJ_OK;
  if (!acc || !sw || !y) return fail(MJ_ERR_ARG, "null operand");
  HostArg a[5] = {{acc, nullptr, (size_t)(M * N) * 4}, {sx, nullptr, opt_bytes(sx, (size_t)M * F4)},
                  {sw, nullptr, (size_t)N * F4}, {b, nullptr, opt_bytes(b, (size_t)N * F4)},
                  {nullptr, y, (size_t)(M * N) * F4}};
  return with_device_copies(a, 5, [&](void **d) {
    return mj_dequantize_i32_scaled_f32((const int32_t *)d[0], (const float *)d[1],
                                        (const float *)d[2], (const float *)d[3], (float *)d[4], M,
                                        N, nullptr);
  });
}

int32_t mj_linear_w8a8_h(const uint16_t *x, const int8_t *Q, const float *scales,
                         const float *bias, int32_t epilogue, uint16_t *y, int64_t M, int64_t N,
                         int64_t K) {
  if (int32_t s = check_dims(M, N, K)) return s;
  if (!valid_epi(epilogue)) return fail(MJ_ERR_ARG, "unknown epilogue %d", epilogue);
  if (M == 0 || N == 0) return MJ_OK;
  if (!y || !scales || !x || !Q) return fail(MJ_ERR_ARG, "null operand");
  HostArg a[5] = {{x, nullptr, (size_t)(M * K) * 2}, {Q, nullptr, (size_t)(N * K)},
                  {scales, nullptr, (size_t)N * F4}, {bias, nullptr, opt_bytes(bias, (size_t)N * F4)},
                  {nullptr, y, (size_t)(M * N) * 2}};
  return with_device_copies(a, 5, [&](void **d) {
    return mj_linear_w8a8((const uint16_t *)d[0], (const int8_t *)d[1], (const float *)d[2],
                          (const float *)d[3], epilogue, (uint16_t *)d[4], M, N, K, nullptr);
  });
}

int32_t mj_mlp_w8a16_h(const uint16_t *x, const int8_t *Wg, const float *sg, const int8_t *Wu,
                       const float *su, const int8_t *Wd, const float *sd, uint16_t *h,
                       uint16_t *y, int64_t M, int64_t K, int64_t I, int64_t H) {
  if (int32_t s = check_dims(M, I, K)) return s;
  if (int32_t s = check_dims(M, H, I)) return s;
  if (M == 0 || H == 0) return MJ_OK;
  if (!x || !Wg || !sg || !Wu || !su || !Wd || !sd || !y) return fail(MJ_ERR_ARG, "null operand");
  // h is device scratch; it is copied back only when the caller passes a buffer
  HostArg a[9] = {{x, nullptr, (size_t)(M * K) * 2},  {Wg, nullptr, (size_t)(I * K)},
                  {sg, nullptr, (size_t)I * F4},       {Wu, nullptr, (size_t)(I * K)},
                  {su, nullptr, (size_t)I * F4},       {Wd, nullptr, (size_t)(H * I)},
                  {sd, nullptr, (size_t)H * F4},       {nullptr, h, (size_t)(M * I) * 2},
                  {nullptr, y, (size_t)(M * H) * 2}};
  return with_device_copies(a, 9, [&](void **d) {
    return mj_mlp_w8a16((const uint16_t *)d[0], (const int8_t *)d[1], (const float *)d[2],
                        (const int8_t *)d[3], (const float *)d[4], (const int8_t *)d[5],
                        (const float *)d[6], (uint16_t *)d[7], (uint16_t *)d[8], M, K, I, H,
                        nullptr);
  });
}

}  // extern "C"
