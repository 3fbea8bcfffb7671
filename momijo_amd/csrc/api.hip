// C ABI of the backend (declared in include/momijo_hip.h).  Each entry point
// validates its arguments, picks a kernel configuration and enqueues on the
// caller's stream; nothing here throws, every failure is a status code plus a
// per-thread message from mj_last_error().
#include <hip/hip_runtime.h>

#include <cstring>

#include "../../include/momijo_hip.h"
#include "launch.h"

#include "abi_util.h"

#include <atomic>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

// Scratch of mj_quant_linear_f32_noalloc: the int8 copy of x lives in this
// file-scope device array instead of a per-call allocation.  Each GPU holds
// its own copy until the process ends.  In host code `scratch` names a
// host-side stand-in, not device memory: the array is used only through the
// per-device address that hipGetSymbolAddress returns (noalloc_scratch).
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) int8_t scratch[kNoAllocScratchBytes];

namespace {

using namespace mj_abi;

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
constexpr int kMaxScratchDevices = 64;
std::atomic<void *> g_scratch_addr[kMaxScratchDevices];
std::mutex g_scratch_mu;

int32_t noalloc_scratch(int8_t **out) {
  int dev = 0;
  if (int32_t st = hip_status(hipGetDevice(&dev), "hipGetDevice")) return st;
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(MJ_ERR_UNSUPPORTED, "device %d is beyond the %d devices the scratch table holds",
                dev, kMaxScratchDevices);
  void *p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (!p) {
      if (int32_t st = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                                  "hipGetSymbolAddress(scratch)"))
        return st;
      if (!p) return fail(MJ_ERR_DEVICE, "hipGetSymbolAddress(scratch) returned NULL");
      g_scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *out = (int8_t *)p;
  return MJ_OK;
}

// Workspace of the split-K partials, of QuantLinear's int8 copy of x, of the
// W8A8 Linear's int8 x and row scales, and of the column-sum and min/max
// partials: one device buffer per (device, stream), kept by the library and
// reused by every later call on that stream, so such a call makes no
// allocation call once its stream has seen a call of that size.  The one
// handle value hipStreamPerThread names a different stream on each host
// thread, so its buffers are kept per (device, thread).
// A call holds its buffer's lock from acquiring it until its last kernel is
// enqueued: kernels on one stream run in enqueue order, so two host threads
// sharing a stream cannot interleave their kernels between one call's writes
// and reads of the buffer.
// A buffer that has to grow is replaced by one of at least twice its size; the
// old one is kept until the process ends, since work already queued on the
// stream may still read it.  A stream handle that is destroyed and created
// again inherits the buffer: work still running on the destroyed stream must
// have finished first.  These calls are refused under graph capture
// (MJ_ERR_UNSUPPORTED) before anything is enqueued: the library allocates
// nothing on a capturing stream, and a graph replayed on another stream would
// share the buffer with eager calls.  Capture-safe callers use the entry
// points that need no workspace, or mj_quant_linear_f32_noalloc.
struct StreamWorkspace {
  int dev = 0;
  hipStream_t stream = nullptr;
  std::thread::id thread;  // the calling thread for hipStreamPerThread
  void *ptr = nullptr;
  size_t bytes = 0;
  std::mutex mu;           // held by the call using the buffer
};
std::mutex g_ws_mu;        // guards g_ws and g_ws_retired
std::vector<std::unique_ptr<StreamWorkspace>> g_ws;
std::vector<void *> g_ws_retired;

// MJ_ERR_UNSUPPORTED (and nothing enqueued) while `stream` is being captured.
int32_t refuse_capture(hipStream_t stream) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (int32_t st = hip_status(hipStreamIsCapturing(stream, &cs), "hipStreamIsCapturing"))
    return st;
  if (cs != hipStreamCaptureStatusNone)
    return fail(MJ_ERR_UNSUPPORTED,
                "this call needs the library's per-stream workspace, which is not available "
                "under graph capture (mj_quant_linear_f32_noalloc, the GEMVs and "
                "the GEMMs without a K split can be captured)");
  return MJ_OK;
}

// The workspace of one call: acquire() refuses capture, finds or grows the
// buffer of (device, stream) and locks it until the lease is destroyed, i.e.
// until the call has enqueued its kernels.
class WorkspaceLease {
 public:
  void *ptr = nullptr;

  int32_t acquire(size_t bytes, hipStream_t stream) {
    if (int32_t st = refuse_capture(stream)) return st;
    int dev = 0;
    if (int32_t st = hip_status(hipGetDevice(&dev), "hipGetDevice")) return st;
    const std::thread::id me =
        stream == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id();
    StreamWorkspace *e = nullptr;
    {
      std::lock_guard<std::mutex> g(g_ws_mu);
      for (auto &w : g_ws)
        if (w->dev == dev && w->stream == stream && w->thread == me) e = w.get();
      if (!e) {
        g_ws.push_back(std::make_unique<StreamWorkspace>());
        e = g_ws.back().get();
        e->dev = dev;
        e->stream = stream;
        e->thread = me;
      }
    }
    lock_ = std::unique_lock<std::mutex>(e->mu);
    if (e->bytes < bytes) {
      size_t want = bytes;
      if (want < 2 * e->bytes) want = 2 * e->bytes;
      want = (want + ((size_t)2 << 20) - 1) & ~(((size_t)2 << 20) - 1);
      void *p = nullptr;
      if (hipMalloc(&p, want) != hipSuccess) {
        (void)hipGetLastError();
        lock_.unlock();
        return fail(MJ_ERR_ALLOC, "workspace allocation of %zu bytes failed", want);
      }
      if (e->ptr) {
        std::lock_guard<std::mutex> g(g_ws_mu);
        g_ws_retired.push_back(e->ptr);
      }
      e->ptr = p;
      e->bytes = want;
    }
    ptr = e->ptr;
    return MJ_OK;
  }

 private:
  std::unique_lock<std::mutex> lock_;
};

// Output extent of Conv2d.forward: (size + 2 pad - k) // stride + 1 with
// floor division (learn/nn/conv.mojo:496-497); <= 0 means an empty output.
int64_t conv_out(int64_t size, int64_t k, int64_t stride, int64_t pad) {
  const int64_t num = size + 2 * pad - k;
  const int64_t q = num >= 0 ? num / stride : -((-num + stride - 1) / stride);
  return q + 1;
}

// Launches a planned NT GEMM; `part` is the fp32 workspace when the plan
// splits K.
int32_t launch_planned(mj::GemmNT p, const mj::GemmPlan &plan, void *part, hipStream_t stream,
                       const char *what) {
  p.part = (float *)part;
  return hip_status(mj::launch_gemm_nt(p, plan, stream), what);
}

// The tile kernels address a tile's 256 rows of A and of B with 32-bit
// buffer offsets ((r * ld + k) * element size, r < 256): larger leading
// dimensions would wrap or fall outside the buffer resource and read zeros.
int32_t check_tile_offsets(const mj::GemmNT &p, const char *what) {
  const int64_t bsz = p.bkind == mj::B_INT8 ? 1 : 2;
  if (256 * p.lda * 2 >= ((int64_t)1 << 31) || 256 * p.ldb * bsz >= ((int64_t)1 << 31))
    return fail(MJ_ERR_UNSUPPORTED, "%s: leading dimension too large for 32-bit tile offsets "
                "(lda=%lld, ldb=%lld)", what, (long long)p.lda, (long long)p.ldb);
  return MJ_OK;
}

// Plans and launches an NT GEMM, with the fp32 workspace of the stream when
// the plan splits K.
int32_t run_gemm_nt(const mj::GemmNT &p, hipStream_t stream, const char *what) {
  if (int32_t st = check_tile_offsets(p, what)) return st;
  const mj::GemmPlan plan = mj::plan_gemm_nt(p);
  const size_t ws = plan.workspace_bytes(p);
  if (!ws) return launch_planned(p, plan, nullptr, stream, what);
  WorkspaceLease lease;
  if (int32_t st = lease.acquire(ws, stream)) return st;
  return launch_planned(p, plan, lease.ptr, stream, what);
}

// QuantLinear.forward on a caller-provided int8 buffer xq of M*K bytes
// (16-byte aligned): quantize x with s_x, then the int8 GEMM with the
// dequantize fused.  Every byte of xq that the GEMM reads is written by the
// quantize first, so the buffer needs no clearing.
int32_t quant_linear_body(const float *x, const int8_t *Wq, const float *b, float s_w, float s_x,
                          float *y, int64_t M, int64_t N, int64_t K, int32_t legacy_literal,
                          int8_t *xq, hipStream_t stream) {
  const bool fast = !legacy_literal && K % 16 == 0 && aligned16(Wq) && aligned16(xq);
  int32_t st = MJ_OK;
  if (M * K > 0)
    st = hip_status(mj::launch_quantize_tensor_legacy(x, M * K, s_x, xq, stream),
                    "quantize launch");
  // sf = s_x * s_w with the reference's (unguarded) s_x (layers.mojo:1684)
  const float sf = s_x * s_w;
  if (st) return st;
  if (fast)
    return hip_status(mj::launch_gemm_i8(xq, Wq, nullptr, y, sf, b, M, N, K, stream),
                      "gemm_i8 launch");
  return hip_status(mj::launch_gemm_i8_scalar(xq, Wq, nullptr, y, sf, b, M, N, K,
                                              legacy_literal != 0, stream),
                    "gemm_i8 scalar launch");
}

// db = column sums of dy [N, OutF]; `part` holds the segment partials when
// colsum_segments(N, OutF) > 1 (the caller's workspace lease).
int32_t run_colsum(const float *dy, int64_t N, int64_t OutF, float *db, float *part,
                   hipStream_t stream) {
  const int64_t segs = mj::colsum_segments(N, OutF);
  return hip_status(mj::launch_colsum_f32(dy, N, OutF, db, part, segs, stream), "colsum launch");
}

}  // namespace

extern "C" {

int32_t mj_version(void) { return 101; }

int32_t mj_device_available(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    return 0;
  }
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
  return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

const char *mj_last_error(void) { return g_err; }

int32_t mj_stream_synchronize(void *stream) {
  return hip_status(hipStreamSynchronize(S(stream)), "hipStreamSynchronize");
}

// ------------------------------------------------------------------ fp32
int32_t mj_matmul_f32(int64_t M, int64_t N, int64_t K, const float *A, int64_t sAm, int64_t sAk,
                      const float *B, int64_t sBk, int64_t sBn, const float *bias,
                      int32_t epilogue, float *C, int64_t ldc, void *stream) {
  if (int32_t s = check_dims(M, N, K)) return s;
  if (!valid_epi(epilogue)) return fail(MJ_ERR_ARG, "unknown epilogue %d", epilogue);
  if (M == 0 || N == 0) return MJ_OK;
  if (!C || (K > 0 && (!A || !B))) return fail(MJ_ERR_ARG, "null operand");
  if (ldc < N) return fail(MJ_ERR_SHAPE, "ldc (%lld) < N (%lld)", (long long)ldc, (long long)N);
  if (sAm < 0 || sAk < 0 || sBk < 0 || sBn < 0) return fail(MJ_ERR_UNSUPPORTED, "negative stride");
  return hip_status(mj::launch_gemm_f32(M, N, K, A, sAm, sAk, B, sBk, sBn, bias, epilogue, C,
                                        ldc, S(stream)),
                    "gemm_f32 launch");
}

int32_t mj_matvec_f32(int64_t M, int64_t N, const float *A, int64_t sAm, int64_t sAn,
                      const float *x, int64_t sx, float *y, void *stream) {
  if (int32_t s = check_dims(M, N, 0)) return s;
  if (M == 0) return MJ_OK;
  if (!y || (N > 0 && (!A || !x))) return fail(MJ_ERR_ARG, "null operand");
  if (sAm < 0 || sAn < 0 || sx < 0) return fail(MJ_ERR_UNSUPPORTED, "negative stride");
  return hip_status(mj::launch_matvec_f32(M, N, A, sAm, sAn, x, sx, y, S(stream)),
                    "matvec_f32 launch");
}

int32_t mj_matmul_f64(int64_t M, int64_t N, int64_t K, const double *A, int64_t sAm,
                      int64_t sAk, const double *B, int64_t sBk, int64_t sBn, double *C,
                      int64_t ldc, void *stream) {
  if (int32_t s = check_dims(M, N, K)) return s;
  if (M == 0 || N == 0) return MJ_OK;
  if (!C || (K > 0 && (!A || !B))) return fail(MJ_ERR_ARG, "null operand");
  if (ldc < N) return fail(MJ_ERR_SHAPE, "ldc (%lld) < N (%lld)", (long long)ldc, (long long)N);
  if (sAm < 0 || sAk < 0 || sBk < 0 || sBn < 0) return fail(MJ_ERR_UNSUPPORTED, "negative stride");
  return hip_status(mj::launch_gemm_f64(M, N, K, A, sAm, sAk, B, sBk, sBn, C, ldc, 0, S(stream)),
                    "gemm_f64 launch");
}

int32_t mj_matvec_f64(int64_t M, int64_t N, const double *A, int64_t sAm, int64_t sAn,
                      const double *x, int64_t sx, double *y, void *stream) {
  if (int32_t s = check_dims(M, N, 0)) return s;
  if (M == 0) return MJ_OK;
  if (!y || (N > 0 && (!A || !x))) return fail(MJ_ERR_ARG, "null operand");
  if (sAm < 0 || sAn < 0 || sx < 0) return fail(MJ_ERR_UNSUPPORTED, "negative stride");
  return hip_status(mj::launch_matvec_f64(M, N, A, sAm, sAn, x, sx, y, S(stream)),
                    "matvec_f64 launch");
}

int32_t mj_tensordot_f32(int32_t batch_rank, const int64_t *batch_shape,
                         const int64_t *a_batch_strides, const int64_t *b_batch_strides,
                         int64_t M, int64_t N, int64_t K, const float *A, int64_t sAm,
                         int64_t sAk, const float *B, int64_t sBk, int64_t sBn, float *C,
                         void *stream) {
  if (int32_t s = check_dims(M, N, K)) return s;
  if (batch_rank < 0 || batch_rank > mj::BatchDesc::kMaxRank)
    return fail(MJ_ERR_UNSUPPORTED, "batch rank must be 0..%d", mj::BatchDesc::kMaxRank);
  if (batch_rank > 0 && (!batch_shape || !a_batch_strides || !b_batch_strides))
    return fail(MJ_ERR_ARG, "null batch description");
  mj::BatchDesc bd;
  bd.rank = batch_rank;
  int64_t batches = 1;
  for (int d = 0; d < batch_rank; ++d) {
    if (batch_shape[d] < 0) return fail(MJ_ERR_ARG, "negative batch extent");
    if (a_batch_strides[d] < 0 || b_batch_strides[d] < 0)
      return fail(MJ_ERR_UNSUPPORTED, "negative stride");
    bd.shape[d] = batch_shape[d];
    bd.a_stride[d] = a_batch_strides[d];
    bd.b_stride[d] = b_batch_strides[d];
    batches *= batch_shape[d];
  }
  if (batches == 0 || M == 0 || N == 0) return MJ_OK;
  if (!C || (K > 0 && (!A || !B))) return fail(MJ_ERR_ARG, "null operand");
  if (sAm < 0 || sAk < 0 || sBk < 0 || sBn < 0) return fail(MJ_ERR_UNSUPPORTED, "negative stride");
  return hip_status(mj::launch_gemm_f32_batched(M, N, K, A, sAm, sAk, B, sBk, sBn, C, bd, batches,
                                                S(stream)),
                    "tensordot launch");
}

int32_t mj_linear_f32(const float *x, const float *W, const float *bias, int32_t epilogue,
                      float *y, int64_t N, int64_t InF, int64_t OutF, void *stream) {
  // y = x W^T: B = W^T is the stride view (sBk = 1, sBn = InF) of W.
  return mj_matmul_f32(N, OutF, InF, x, InF, 1, W, 1, InF, bias, epilogue, y, OutF, stream);
}

int32_t mj_launch_linear_fw_h(const float *x, const float *wT, const float *b, float *y,
                              int64_t N, int64_t InF, int64_t OutF, int32_t has_bias) {
  if (int32_t s = check_dims(N, OutF, InF)) return s;
  if (N == 0 || OutF == 0) return MJ_OK;
  if (!y || (InF > 0 && (!x || !wT)) || (has_bias && !b)) return fail(MJ_ERR_ARG, "null operand");
  const size_t bx = (size_t)N * InF * 4, bw = (size_t)InF * OutF * 4, by = (size_t)N * OutF * 4,
               bb = (size_t)OutF * 4;
  char *dev = nullptr;
  const size_t total = bx + bw + by + bb + 64;
  if (hipMalloc((void **)&dev, total) != hipSuccess) {
    (void)hipGetLastError();
    return fail(MJ_ERR_ALLOC, "hipMalloc(%zu) failed", total);
  }
  float *dx = (float *)dev, *dw = (float *)(dev + bx), *dy = (float *)(dev + bx + bw),
        *db = (float *)(dev + bx + bw + by);
  int32_t st = MJ_OK;
  if (bx) st = hip_status(hipMemcpy(dx, x, bx, hipMemcpyHostToDevice), "copy x");
  if (!st && bw) st = hip_status(hipMemcpy(dw, wT, bw, hipMemcpyHostToDevice), "copy wT");
  if (!st && has_bias) st = hip_status(hipMemcpy(db, b, bb, hipMemcpyHostToDevice), "copy b");
  if (!st)
    st = hip_status(mj::launch_gemm_f32(N, OutF, InF, dx, InF, 1, dw, OutF, 1,
                                        has_bias ? db : nullptr, MJ_EPI_NONE, dy, OutF, nullptr),
                    "gemm_f32 launch");
  if (!st) st = hip_status(hipMemcpy(y, dy, by, hipMemcpyDeviceToHost), "copy y");
  (void)hipFree(dev);
  return st;
}

// ------------------------------------------------------------------ backward

int32_t mj_linear_backward_f32(const float *x, const float *W, const float *dy, float *dW,
                               float *db, float *dx, int64_t N, int64_t InF, int64_t OutF,
                               void *stream) {
  if (int32_t s = check_dims(N, InF, OutF)) return s;
  const bool want_dx = dx && N > 0 && InF > 0;
  const bool want_dW = dW && OutF > 0 && InF > 0;
  const bool want_db = db && OutF > 0;
  if ((want_dx || want_dW || want_db) && N > 0 && !dy) return fail(MJ_ERR_ARG, "null dy");
  if (want_dx && OutF > 0 && !W) return fail(MJ_ERR_ARG, "null W");
  if (want_dW && N > 0 && !x) return fail(MJ_ERR_ARG, "null x");
  const hipStream_t st = S(stream);
  // the column-sum partials: acquired before anything is enqueued, so a
  // refusal (graph capture) leaves the stream untouched
  WorkspaceLease lease;
  const int64_t segs = want_db ? mj::colsum_segments(N, OutF) : 1;
  if (segs > 1) {
    if (int32_t e = lease.acquire((size_t)segs * (size_t)OutF * sizeof(float), st)) return e;
  }
  // dx [N, InF] = dy [N, OutF] @ W [OutF, InF]
  if (want_dx) {
    if (int32_t e = hip_status(mj::launch_gemm_f32(N, InF, OutF, dy, OutF, 1, W, InF, 1, nullptr,
                                                   MJ_EPI_NONE, dx, InF, st),
                               "linear backward dx"))
      return e;
  }
  // dW [OutF, InF] = dy^T @ x: A is the transposed view (row stride 1) of dy
  if (want_dW) {
    if (int32_t e = hip_status(mj::launch_gemm_f32(OutF, InF, N, dy, 1, OutF, x, InF, 1, nullptr,
                                                   MJ_EPI_NONE, dW, InF, st),
                               "linear backward dW"))
      return e;
  }
  if (want_db) return run_colsum(dy, N, OutF, db, (float *)lease.ptr, st);
  return MJ_OK;
}

int32_t mj_launch_linear_bw_dx_h(const float *dy, const float *w, float *dx, int64_t N,
                                 int64_t InF, int64_t OutF) {
  if (int32_t s = check_dims(N, InF, OutF)) return s;
  if (N == 0 || InF == 0) return MJ_OK;
  if (!dx || (OutF > 0 && (!dy || !w))) return fail(MJ_ERR_ARG, "null operand");
  HostArg a[3] = {{dy, nullptr, (size_t)N * OutF * 4}, {w, nullptr, (size_t)OutF * InF * 4},
                  {nullptr, dx, (size_t)N * InF * 4}};
  return with_device_copies(a, 3, [&](void **d) {
    return mj_linear_backward_f32(nullptr, (const float *)d[1], (const float *)d[0], nullptr,
                                  nullptr, (float *)d[2], N, InF, OutF, nullptr);
  });
}

int32_t mj_launch_linear_bw_dw_h(const float *dy, const float *x, float *dW, int64_t N,
                                 int64_t InF, int64_t OutF) {
  if (int32_t s = check_dims(N, InF, OutF)) return s;
  if (OutF == 0 || InF == 0) return MJ_OK;
  if (!dW || (N > 0 && (!dy || !x))) return fail(MJ_ERR_ARG, "null operand");
  HostArg a[3] = {{dy, nullptr, (size_t)N * OutF * 4}, {x, nullptr, (size_t)N * InF * 4},
                  {nullptr, dW, (size_t)OutF * InF * 4}};
  return with_device_copies(a, 3, [&](void **d) {
    return mj_linear_backward_f32((const float *)d[1], nullptr, (const float *)d[0],
                                  (float *)d[2], nullptr, nullptr, N, InF, OutF, nullptr);
  });
}

int32_t mj_launch_linear_bw_db_h(const float *dy, float *db, int64_t N, int64_t OutF) {
  if (int32_t s = check_dims(N, OutF, 0)) return s;
  if (OutF == 0) return MJ_OK;
  if (!db || (N > 0 && !dy)) return fail(MJ_ERR_ARG, "null operand");
  HostArg a[2] = {{dy, nullptr, (size_t)N * OutF * 4}, {nullptr, db, (size_t)OutF * 4}};
  return with_device_copies(a, 2, [&](void **d) {
    return mj_linear_backward_f32(nullptr, nullptr, (const float *)d[0], nullptr, (float *)d[1],
                                  nullptr, N, 1, OutF, nullptr);
  });
}

int32_t mj_launch_conv2d_fw_h(const float *x, const float *w, const float *b, float *y, int64_t N,
                              int64_t C, int64_t H, int64_t W, int64_t OH, int64_t OW, int64_t OC,
                              int64_t kH, int64_t kW, int64_t sH, int64_t sW, int64_t pH,
                              int64_t pW, int32_t has_bias) {
  if (N < 0 || C < 0 || H < 0 || W < 0 || OC < 0 || kH < 1 || kW < 1 || sH < 1 || sW < 1 ||
      pH < 0 || pW < 0)
    return fail(MJ_ERR_ARG, "conv2d: negative size, or kernel / stride below 1");
  // the seam returns at once when there is nothing to compute
  // (tensor/gpu/runtime.mojo:398-400)
  if (N * OC * OH * OW <= 0 || OH <= 0 || OW <= 0) return MJ_OK;
  if (OH != conv_out(H, kH, sH, pH) || OW != conv_out(W, kW, sW, pW))
    return fail(MJ_ERR_SHAPE, "conv2d: OH x OW = %lld x %lld, the geometry gives %lld x %lld",
                (long long)OH, (long long)OW, (long long)conv_out(H, kH, sH, pH),
                (long long)conv_out(W, kW, sW, pW));
  if (!y || !w || (C > 0 && !x) || (has_bias && !b)) return fail(MJ_ERR_ARG, "null operand");
  HostArg a[4] = {{x, nullptr, (size_t)(N * C * H * W) * 4},
                  {w, nullptr, (size_t)(OC * C * kH * kW) * 4},
                  {has_bias ? b : nullptr, nullptr, has_bias ? (size_t)OC * 4 : 0},
                  {nullptr, y, (size_t)(N * OC * OH * OW) * 4}};
  return with_device_copies(a, 4, [&](void **d) {
    return mj_conv2d_f32((const float *)d[0], (const float *)d[1],
                         has_bias ? (const float *)d[2] : nullptr, MJ_EPI_NONE, (float *)d[3], N,
                         C, H, W, OC, kH, kW, sH, sW, pH, pW, nullptr);
  });
}

int32_t mj_matmul_backward_f64(int64_t M, int64_t N, int64_t K, const double *A, const double *B,
                               const double *G, double *dA, double *dB, int32_t accumulate,
                               void *stream) {
  if (int32_t s = check_dims(M, N, K)) return s;
  const bool want_dA = dA && M > 0 && K > 0;
  const bool want_dB = dB && K > 0 && N > 0;
  if ((want_dA || want_dB) && N > 0 && M > 0 && !G) return fail(MJ_ERR_ARG, "null G");
  if (want_dA && N > 0 && !B) return fail(MJ_ERR_ARG, "null B");
  if (want_dB && M > 0 && !A) return fail(MJ_ERR_ARG, "null A");
  const int accum = accumulate ? 1 : 0;
  const hipStream_t st = S(stream);
  // dA [M, K] (+)= G [M, N] @ B^T: B^T is the view (row stride 1, column stride N) of B [K, N]
  if (want_dA) {
    if (int32_t e = hip_status(mj::launch_gemm_f64(M, K, N, G, N, 1, B, 1, N, dA, K, accum, st),
                               "matmul backward dA"))
      return e;
  }
  // dB [K, N] (+)= A^T @ G: A^T is the view (row stride 1, column stride K) of A [M, K]
  if (want_dB)
    return hip_status(mj::launch_gemm_f64(K, N, M, A, 1, K, G, N, 1, dB, N, accum, st),
                      "matmul backward dB");
  return MJ_OK;
}

int32_t mj_matmul_backward_f32(int64_t M, int64_t N, int64_t K, const float *A, const float *B,
                               const float *G, float *dA, float *dB, int32_t accumulate,
                               void *stream) {
  if (int32_t s = check_dims(M, N, K)) return s;
  const bool want_dA = dA && M > 0 && K > 0;
  const bool want_dB = dB && K > 0 && N > 0;
  if ((want_dA || want_dB) && N > 0 && M > 0 && !G) return fail(MJ_ERR_ARG, "null G");
  if (want_dA && N > 0 && !B) return fail(MJ_ERR_ARG, "null B");
  if (want_dB && M > 0 && !A) return fail(MJ_ERR_ARG, "null A");
  const int accum = accumulate ? 1 : 0;
  const hipStream_t st = S(stream);
  // dA [M, K] (+)= G [M, N] @ B^T: B^T is the view (row stride 1, column stride N) of B [K, N]
  if (want_dA) {
    if (int32_t e = hip_status(
            mj::launch_gemm_f32_accum(M, K, N, G, N, 1, B, 1, N, dA, K, accum, st),
            "matmul backward dA"))
      return e;
  }
  // dB [K, N] (+)= A^T @ G: A^T is the view (row stride 1, column stride K) of A [M, K]
  if (want_dB)
    return hip_status(mj::launch_gemm_f32_accum(K, N, M, A, 1, K, G, N, 1, dB, N, accum, st),
                      "matmul backward dB");
  return MJ_OK;
}

int32_t mj_activation_f32(int32_t epilogue, const float *x, float *y, int64_t n, void *stream) {
  if (!valid_epi(epilogue)) return fail(MJ_ERR_ARG, "unknown epilogue %d", epilogue);
  if (n < 0) return fail(MJ_ERR_ARG, "negative size");
  if (n == 0) return MJ_OK;
  if (!x || !y) return fail(MJ_ERR_ARG, "null operand");
  return hip_status(mj::launch_activation_f32(epilogue, x, y, n, S(stream)), "activation launch");
}

int32_t mj_conv2d_f32(const float *x, const float *w, const float *b, int32_t epilogue, float *y,
                      int64_t N, int64_t C, int64_t H, int64_t W, int64_t OC, int64_t kH,
                      int64_t kW, int64_t sH, int64_t sW, int64_t pH, int64_t pW,
                      void *stream) {
  if (!valid_epi(epilogue)) return fail(MJ_ERR_ARG, "unknown epilogue %d", epilogue);
  if (N < 0 || C < 0 || H < 0 || W < 0 || OC < 0 || kH < 1 || kW < 1 || sH < 1 || sW < 1 ||
      pH < 0 || pW < 0)
    return fail(MJ_ERR_ARG, "conv2d: negative size, or kernel / stride below 1");
  const int64_t OH = conv_out(H, kH, sH, pH), OW = conv_out(W, kW, sW, pW);
  if (N == 0 || OC == 0 || OH <= 0 || OW <= 0) return MJ_OK;
  // every index the kernel forms stays in 32 bits within an image / tile
  const int64_t lim = (int64_t)1 << 31;
  if (C * H * W >= lim || OC * C * kH * kW >= lim || OC * OH * OW >= lim || H + 2 * pH >= lim ||
      W + 2 * pW >= lim || N >= lim)
    return fail(MJ_ERR_UNSUPPORTED, "conv2d: a dimension product exceeds 2^31");
  if (!y || !w || (C > 0 && !x)) return fail(MJ_ERR_ARG, "null operand");
  return hip_status(mj::launch_conv2d_f32(x, w, b, y, N, C, H, W, OC, kH, kW, sH, sW, pH, pW, OH,
                                          OW, epilogue, S(stream)),
                    "conv2d launch");
}

int32_t mj_maximum_scalar_f32(const float *x, float s, float *y, int64_t n, void *stream) {
  if (n < 0) return fail(MJ_ERR_ARG, "negative size");
  if (n == 0) return MJ_OK;
  if (!x || !y) return fail(MJ_ERR_ARG, "null operand");
  return hip_status(mj::launch_maximum_scalar_f32(x, s, y, n, S(stream)),
                    "maximum_scalar launch");
}

int32_t mj_cast_i64_f32(const int64_t *x, float *y, int64_t n, void *stream) {
  if (n < 0) return fail(MJ_ERR_ARG, "negative size");
  if (n == 0) return MJ_OK;
  if (!x || !y) return fail(MJ_ERR_ARG, "null operand");
  return hip_status(mj::launch_cast_i64_f32(x, y, n, S(stream)), "cast launch");
}

// ------------------------------------------------------------------ bf16
int32_t mj_gemm_bf16_nt(int64_t M, int64_t N, int64_t K, const uint16_t *A, int64_t lda,
                        const uint16_t *B, int64_t ldb, const float *bias, int32_t epilogue,
                        uint16_t *C, int64_t ldc, void *stream) {
  if (int32_t s = check_dims(M, N, K)) return s;
  if (!valid_epi(epilogue)) return fail(MJ_ERR_ARG, "unknown epilogue %d", epilogue);
  if (M == 0 || N == 0) return MJ_OK;
  if (!C || (K > 0 && (!A || !B))) return fail(MJ_ERR_ARG, "null operand");
  if (lda < K || ldb < K || ldc < N) return fail(MJ_ERR_SHAPE, "leading dimension too small");
  if (K % 8 || lda % 8 || ldb % 8 || !aligned16(A) || !aligned16(B))
    return fail(MJ_ERR_UNSUPPORTED, "bf16 GEMM needs K, lda, ldb %% 8 == 0 and 16-byte aligned A, B");
  mj::GemmNT p;
  p.A = A; p.lda = lda; p.B = B; p.ldb = ldb; p.bias = bias; p.epi = epilogue;
  p.C = C; p.ldc = ldc; p.M = M; p.N = N; p.K = K; p.bkind = mj::B_BF16;
  return run_gemm_nt(p, S(stream), "gemm_bf16");
}

// ------------------------------------------------------------------ int8 legacy
int32_t mj_quantize_symmetric_int8(const float *x, int64_t n, float scale, int8_t *q,
                                   void *stream) {
  if (n < 0) return fail(MJ_ERR_ARG, "negative size");
  if (n == 0) return MJ_OK;
  if (!x || !q) return fail(MJ_ERR_ARG, "null operand");
  return hip_status(mj::launch_quantize_tensor_legacy(x, n, scale, q, S(stream)),
                    "quantize launch");
}

int32_t mj_minmax_f32(const float *x, int64_t n, float *minmax_out, void *stream) {
  if (n <= 0) return fail(MJ_ERR_ARG, "minmax needs n > 0");
  if (!x || !minmax_out) return fail(MJ_ERR_ARG, "null operand");
  WorkspaceLease lease;
  if (int32_t st = lease.acquire(sizeof(float) * 2 * mj::minmax_partials(), S(stream)))
    return st;
  return hip_status(mj::launch_minmax(x, n, (float *)lease.ptr, minmax_out, S(stream)),
                    "minmax launch");
}

int32_t mj_minmax_scale_symmetric(const float *x, int64_t n, float max_q, float *scale_out,
                                  void *stream) {
  if (n < 0) return fail(MJ_ERR_ARG, "negative size");
  if (!scale_out || (n > 0 && !x)) return fail(MJ_ERR_ARG, "null operand");
  WorkspaceLease lease;
  if (int32_t st = lease.acquire(sizeof(float) * 2 * mj::minmax_partials(), S(stream)))
    return st;
  return hip_status(
      mj::launch_minmax_scale(x, n, max_q, (float *)lease.ptr, scale_out, S(stream)),
      "minmax launch");
}

int32_t mj_matmul_i8_i8_to_i32(const int8_t *A, const int8_t *B, int32_t *C, int64_t M,
                               int64_t N, int64_t K, int32_t legacy_literal, void *stream) {
  if (int32_t s = check_dims(M, N, K)) return s;
  if (M == 0 || N == 0) return MJ_OK;
  if (!C || (K > 0 && (!A || !B))) return fail(MJ_ERR_ARG, "null operand");
  if (legacy_literal || K % 16 || !aligned16(A) || !aligned16(B))
    return hip_status(mj::launch_gemm_i8_scalar(A, B, C, nullptr, 0.f, nullptr, M, N, K,
                                                legacy_literal != 0, S(stream)),
                      "gemm_i8 scalar launch");
  return hip_status(mj::launch_gemm_i8(A, B, C, nullptr, 0.f, nullptr, M, N, K, S(stream)),
                    "gemm_i8 launch");
}

int32_t mj_dequantize_i32_to_f32_add_bias(const int32_t *acc, float sf, const float *b, float *y,
                                          int64_t M, int64_t N, void *stream) {
  if (int32_t s = check_dims(M, N, 0)) return s;
  if (M == 0 || N == 0) return MJ_OK;
  if (!acc || !b || !y) return fail(MJ_ERR_ARG, "null operand");
  return hip_status(mj::launch_dequant_i32_bias(acc, sf, b, y, M, N, S(stream)),
                    "dequant launch");
}

int32_t mj_dequantize_i32_scaled_f32(const int32_t *acc, const float *sx, const float *sw,
                                     const float *b, float *y, int64_t M, int64_t N,
                                     void *stream) {
  if (int32_t s = check_dims(M, N, 0)) return s;
  if (M == 0 || N == 0) return MJ_OK;
  if (!acc || !sw || !y) return fail(MJ_ERR_ARG, "null operand");
  return hip_status(mj::launch_dequant_i32_scaled(acc, sx, sw, b, y, M, N, S(stream)),
                    "dequant_scaled launch");
}

int32_t mj_quant_linear_f32(const float *x, const int8_t *Wq, const float *b, float s_w,
                            float s_x, float *y, int64_t M, int64_t N, int64_t K,
                            int32_t legacy_literal, void *stream) {
  if (int32_t s = check_dims(M, N, K)) return s;
  if (M == 0 || N == 0) return MJ_OK;
  if (!y || !b || (K > 0 && (!x || !Wq))) return fail(MJ_ERR_ARG, "null operand");
  // the int8 copy of x in the stream's workspace
  WorkspaceLease lease;
  if (int32_t st = lease.acquire((size_t)M * K + 16, S(stream))) return st;
  return quant_linear_body(x, Wq, b, s_w, s_x, y, M, N, K, legacy_literal, (int8_t *)lease.ptr,
                           S(stream));
}

int32_t mj_quant_linear_f32_noalloc(const float *x, const int8_t *Wq, const float *b, float s_w,
                                    float s_x, float *y, int64_t M, int64_t N, int64_t K,
                                    int32_t legacy_literal, void *stream) {
  if (int32_t s = check_dims(M, N, K)) return s;
  if (M == 0 || N == 0) return MJ_OK;
  if (!y || !b || (K > 0 && (!x || !Wq))) return fail(MJ_ERR_ARG, "null operand");
  if ((uint64_t)M * (uint64_t)K + 16 > kNoAllocScratchBytes)
    return fail(MJ_ERR_UNSUPPORTED,
                "mj_quant_linear_f32_noalloc: the quantized x needs M*K = %lld bytes; the static "
                "scratch holds %zu (use mj_quant_linear_f32)",
                (long long)(M * K), kNoAllocScratchBytes - 16);
  int8_t *xq = nullptr;
  if (int32_t st = noalloc_scratch(&xq)) return st;
  return quant_linear_body(x, Wq, b, s_w, s_x, y, M, N, K, legacy_literal, xq, S(stream));
}

// ------------------------------------------------------------------ int8 per-channel
int32_t mj_quantize_rowwise_i8(const float *W, int64_t N, int64_t K, int32_t rounding, int8_t *Q,
                               float *scales, void *stream) {
  if (int32_t s = check_dims(N, 0, K)) return s;
  if (rounding != MJ_ROUND_RHE && rounding != MJ_ROUND_LEGACY)
    return fail(MJ_ERR_ARG, "unknown rounding %d", rounding);
  if (N == 0) return MJ_OK;
  if (K == 0) return fail(MJ_ERR_SHAPE, "K must be positive");
  if (!W || !Q || !scales) return fail(MJ_ERR_ARG, "null operand");
  return hip_status(mj::launch_quantize_rowwise(W, N, K, rounding, Q, scales, S(stream)),
                    "quantize_rowwise launch");
}

int32_t mj_linear_w8a16(const uint16_t *x, const int8_t *Q, const float *scales,
                        const float *bias, int32_t epilogue, uint16_t *y, int64_t M, int64_t N,
                        int64_t K, void *stream) {
  if (int32_t s = check_dims(M, N, K)) return s;
  if (!valid_epi(epilogue)) return fail(MJ_ERR_ARG, "unknown epilogue %d", epilogue);
  if (M == 0 || N == 0) return MJ_OK;
  if (!y || !scales || (K > 0 && (!x || !Q))) return fail(MJ_ERR_ARG, "null operand");
  if (K % 16 || !aligned16(x) || !aligned16(Q))
    return fail(MJ_ERR_UNSUPPORTED, "W8A16 Linear needs K %% 16 == 0 and 16-byte aligned x, Q");
  if (mj::gemv_w8a16_takes(M, K))
    return hip_status(mj::launch_gemv_w8a16(x, Q, scales, bias, epilogue, y, M, N, K, S(stream)),
                      "gemv_w8a16 launch");
  mj::GemmNT p;
  p.A = x; p.lda = K; p.B = Q; p.ldb = K; p.scales = scales; p.bias = bias; p.epi = epilogue;
  p.C = y; p.ldc = N; p.M = M; p.N = N; p.K = K; p.bkind = mj::B_INT8;
  return run_gemm_nt(p, S(stream), "gemm_w8a16");
}

int32_t mj_quantize_rows_bf16_i8(const uint16_t *x, int64_t M, int64_t K, int8_t *xq, float *sx,
                                 void *stream) {
  if (int32_t s = check_dims(M, 0, K)) return s;
  if (M == 0) return MJ_OK;
  if (K == 0) return fail(MJ_ERR_SHAPE, "K must be positive");
  if (!x || !xq || !sx) return fail(MJ_ERR_ARG, "null operand");
  return hip_status(mj::launch_quantize_rows_bf16(x, M, K, xq, sx, S(stream)),
                    "quantize_rows_bf16 launch");
}

int32_t mj_linear_w8a8(const uint16_t *x, const int8_t *Q, const float *scales, const float *bias,
                       int32_t epilogue, uint16_t *y, int64_t M, int64_t N, int64_t K,
                       void *stream) {
  if (int32_t s = check_dims(M, N, K)) return s;
  if (!valid_epi(epilogue)) return fail(MJ_ERR_ARG, "unknown epilogue %d", epilogue);
  if (M == 0 || N == 0) return MJ_OK;
  if (K == 0) return fail(MJ_ERR_SHAPE, "K must be positive");
  if (!x || !Q || !scales || !y) return fail(MJ_ERR_ARG, "null operand");
  // K <= 2^17: |sum| <= 127 * 127 * K stays below 2^31, so the int32 sums
  // are exact
  if (K % 16 || K > ((int64_t)1 << 17) || !aligned16(x) || !aligned16(Q))
    return fail(MJ_ERR_UNSUPPORTED,
                "W8A8 Linear needs K %% 16 == 0, K <= 131072 and 16-byte aligned x, Q");
  // xq [M,K] int8 then sx [M] fp32 in the stream's workspace
  const size_t xq_bytes = ((size_t)M * K + 255) & ~(size_t)255;
  WorkspaceLease lease;
  if (int32_t st = lease.acquire(xq_bytes + (size_t)M * sizeof(float), S(stream))) return st;
  int8_t *ws = (int8_t *)lease.ptr;
  float *sx = (float *)(ws + xq_bytes);
  int32_t st = hip_status(mj::launch_quantize_rows_bf16(x, M, K, ws, sx, S(stream)),
                          "quantize_rows_bf16 launch");
  if (st == MJ_OK)
    st = hip_status(mj::launch_linear_w8a8(ws, sx, Q, scales, bias, epilogue, y, M, N, K,
                                           S(stream)),
                    "gemm_w8a8 launch");
  return st;
}

int32_t mj_mlp_w8a16(const uint16_t *x, const int8_t *Wg, const float *sg, const int8_t *Wu,
                     const float *su, const int8_t *Wd, const float *sd, uint16_t *h,
                     uint16_t *y, int64_t M, int64_t K, int64_t I, int64_t H, void *stream) {
  if (int32_t s = check_dims(M, I, K)) return s;
  if (int32_t s = check_dims(M, H, I)) return s;
  if (M == 0 || H == 0) return MJ_OK;
  if (!x || !Wg || !sg || !Wu || !su || !Wd || !sd || !h || !y)
    return fail(MJ_ERR_ARG, "null operand");
  if (K % 16 || I % 16 || !aligned16(x) || !aligned16(Wg) || !aligned16(Wu) || !aligned16(Wd) ||
      !aligned16(h))
    return fail(MJ_ERR_UNSUPPORTED, "MLP needs K, I %% 16 == 0 and 16-byte aligned operands");
  mj::GemmNT gu;
  gu.A = x; gu.lda = K; gu.B = Wg; gu.B2 = Wu; gu.ldb = K; gu.scales = sg; gu.scales2 = su;
  gu.C = h; gu.ldc = I; gu.M = M; gu.N = I; gu.K = K; gu.bkind = mj::B_INT8; gu.gate_up = true;
  mj::GemmNT dn;
  dn.A = h; dn.lda = I; dn.B = Wd; dn.ldb = I; dn.scales = sd; dn.C = y; dn.ldc = H;
  dn.M = M; dn.N = H; dn.K = I; dn.bkind = mj::B_INT8;
  // decode sizes: either projection as a GEMV (no workspace)
  const bool gu_gemv = I > 0 && mj::gemv_gateup_w8a16_takes(M, K);
  const bool down_gemv = mj::gemv_w8a16_takes(M, I);
  if (!gu_gemv) {
    if (int32_t st = check_tile_offsets(gu, "gate/up")) return st;
  }
  if (!down_gemv) {
    if (int32_t st = check_tile_offsets(dn, "down")) return st;
  }
  // both plans first: one workspace of the larger size is acquired before
  // anything is enqueued (the two GEMMs run in order on the stream, so they
  // can share it)
  mj::GemmPlan pgu, pdn;
  size_t ws = 0;
  if (!gu_gemv) {
    pgu = mj::plan_gemm_nt(gu);
    ws = pgu.workspace_bytes(gu);
  }
  if (!down_gemv) {
    pdn = mj::plan_gemm_nt(dn);
    const size_t wd = pdn.workspace_bytes(dn);
    if (wd > ws) ws = wd;
  }
  WorkspaceLease lease;
  if (ws) {
    if (int32_t st = lease.acquire(ws, S(stream))) return st;
  }
  if (gu_gemv) {
    if (int32_t st = hip_status(mj::launch_gemv_gateup_w8a16(x, Wg, sg, Wu, su, h, M, I, K,
                                                             S(stream)),
                                "gate/up gemv launch"))
      return st;
  } else if (int32_t st = launch_planned(gu, pgu, lease.ptr, S(stream), "gate/up")) {
    return st;
  }
  if (down_gemv)
    return hip_status(mj::launch_gemv_w8a16(h, Wd, sd, nullptr, MJ_EPI_NONE, y, M, H, I,
                                            S(stream)),
                      "down gemv launch");
  return launch_planned(dn, pdn, lease.ptr, S(stream), "down");
}

}  // extern "C"
