// Skinny-M W8A16 Linear (decode): y[m,n] = bf16(epi((x[m,:] . Q[n,:]) *
// scales[n] + bias[n])) for M <= 16, int8 weights Q [N,K] streamed once:
// for M = 1 the K-split kernel (gemv_w8a16_ksplit_kernel, further down) at
// K = 4096 and N <= 252 * 64, the persistent streaming kernel
// (gemv_w8a16_stream_kernel) for the other K <= 4096; the streaming kernel
// below for the other M <= 2, the MFMA kernel after it above.
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
#include <atomic>

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
  // uniform wave index: the buffer resource below is then known to be
  // wave-uniform (a divergent one costs a readfirstlane loop per load)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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

// s_waitcnt immediate: vmcnt <= n, lgkmcnt and expcnt unconstrained
constexpr int vmcnt_imm(int n) { return (n & 15) | (((n >> 4) & 3) << 14) | 0x0F70; }

// Skinny-M W8A16 GEMV for 3..48 x rows (MB groups of 16), plain or the FFN's
// gate/up (GATEUP: the workgroup's tiles alternate 16 gate rows and the 16 up
// rows of the same output columns; the epilogue forms bf16(silu(g sg) (u su))
// from the two fp32 tile sums).  With several x rows the streaming GEMV's
// per-lane multiply-adds turn VALU-bound, so the products go to
// v_mfma_f32_16x16x32_bf16 and the lanes only widen the weights (int8 ->
// bf16, exact).  K is taken in NP passes of 1 KB of every row; a step is one
// (pass, 16-row tile), passes outermost, TILES tiles per workgroup.  Eight
// waves split each pass (128 bytes of a row each): per step a wave loads its
// share of the tile's 16 rows into registers (two 1-KB loads of 8 rows x 128
// contiguous bytes), writes them to its own LDS region with chunk p of row r
// at chunk p ^ (r & 7) (the 8 lanes of a 128-byte read phase then hit
// distinct banks) and reads the MFMA fragments back: lane (r, c) takes the 16
// int8 of row r at chunk 4 j + c of 64-deep block j, the first 8 k for one
// MFMA and the other 8 for the second, against x fragments of the same k.
// The x fragments of all MB groups for a pass sit in registers, in two sets:
// the next pass's loads are issued just before its first weight loads (one
// wait then covers both: loads retire in order) while the current pass still
// reads the other set.  DS steps in flight (at most TILES + 1, so that no
// more than two passes are; with one tile per workgroup every step opens a
// pass and DS x sets rotate with the steps); no barrier in the loop (a wave
// reads only its own region).  Past K (K rounded up to 1 KB) the x fragments
// load zero and the weight bytes there (the next row's, or zero past the
// buffer) add exact zeros.  The eight waves' partial tiles are added in K
// order through LDS (deterministic), then scale, bias and the activation.
// Measured on MI355X, 11008 x 4096 weights (graph replay over 8 weight copies,
// alternating runs on one box): M = 3 / 8 / 16 / 17 / 32 10.9-11.1 / 10.8 /
// 12.0 / 13.9 / 16.7 us against 12.0-12.2 / 12.3 / 13.7 / 16.3 / 19.2 for the
// same design with one 4-KB pass (the fill and drain of its three steps were
// a third of a workgroup's life) and 13.3 / 13.7 / 15.1 / 17.6 / 20.5 with the
// weights copied straight into LDS (buffer_load ... lds); M = 33 / 48 / 64
// 20.5-20.9 / 22.6 / 26.1 against 25.4 / 25.7 / 26.3 on the W8A16 tile GEMM
// (every workgroup reads all of x, M K 2 bytes, which sets the time as M
// grows).  The FFN's down projection (4096 x 11008, one tile per workgroup) at
// M = 5 / 8 / 16: 13.1-13.2 / 13.7-13.8 / 16.7 us against 14.0 / 14.5 / 18.2
// with 4-KB passes.
template <int NP, int TILES, int MB, bool GATEUP, int DS = 2>
__global__ __launch_bounds__(512) void gemv_w8a16_skinny_kernel(
    const uint16_t *__restrict__ x, const int8_t *__restrict__ Q, const int8_t *__restrict__ Q2,
    const float *__restrict__ scales, const float *__restrict__ scales2,
    const float *__restrict__ bias, int epi, uint16_t *__restrict__ y, int M, int N, int K) {
  constexpr int NWV = 8;
  constexpr int KQ = 1024 / NWV;  // bytes of a row per wave per pass
  constexpr int NJ = KQ / 64;     // 64-deep blocks per wave per pass
  constexpr int CP = KQ / 64;     // 1-KB loads per wave per step (16 KQ bytes)
  constexpr int SLOT = 16 * KQ;
  constexpr int STEPS = NP * TILES;
  constexpr int XL = 2 * MB * NJ;  // x loads per pass
  constexpr int TP = GATEUP ? TILES / 2 : TILES;  // 16-column output tiles
  static_assert(!GATEUP || TILES % 2 == 0, "gate/up tiles come in pairs");
  // DS steps in flight; more than two only with one tile per workgroup,
  // where every step opens a pass (x sets rotate with the steps)
  static_assert(DS >= 2 && (TILES == 1 || DS <= TILES + 1), "steps in flight");
  constexpr int XS = TILES == 1 ? DS : 2;  // x fragment sets (passes in flight)
  extern __shared__ __attribute__((aligned(16))) uint8_t lds8[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, c = lane >> 4;
  const int n0 = blockIdx.x * 16 * TP;
  const int rows = N - n0 < 16 * TP ? N - n0 : 16 * TP;
  const __amdgpu_buffer_rsrc_t rQ = make_rsrc(Q + (size_t)n0 * K, (int64_t)rows * K);
  const __amdgpu_buffer_rsrc_t rQ2 =
      make_rsrc((GATEUP ? Q2 : Q) + (size_t)n0 * K, (int64_t)rows * K);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (int64_t)M * K * 2);
  uint8_t *mine = lds8 + wave * 2 * SLOT;

  uint4 xa[XS][MB][NJ], xb[XS][MB][NJ];
  // x fragments of pass p into set p & 1: group g, block j: x row 16 g + r,
  // k = 1024 p + KQ wave + 64 j + 16 c .. + 15 (zero past M or K; K % 16 == 0
  // keeps a fragment all in or all out).  Past K the weight bytes (the next
  // row's, or zero past the buffer) then add exact zeros.
  auto load_x = [&](int p) {
#pragma unroll
    for (int g = 0; g < MB; ++g)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int row = 16 * g + r;
        const int k = 1024 * p + wave * KQ + 64 * j + 16 * c;
        const uint32_t xo = row < M && k < K ? (uint32_t)((row * K + k) * 2) : kOobOffset;
        const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);
        const u32x4 b =
            __builtin_amdgcn_raw_buffer_load_b128(rx, xo == kOobOffset ? xo : xo + 16, 0, 0);
        xa[p % XS][g][j] = make_uint4(a[0], a[1], a[2], a[3]);
        xb[p % XS][g][j] = make_uint4(b[0], b[1], b[2], b[3]);
      }
  };
  uint4 R[DS][CP];
  // step st = (pass p, tile t): load i, lane l holds LDS byte e = 1024 i + 16 l
  // of the wave's region, row e / KQ, chunk (e % KQ) / 16 from global chunk
  // chunk ^ (row & 7).  GATEUP: tile 2 j is gate rows 16 j.., tile 2 j + 1
  // the up rows of the same columns.
  auto issue = [&](int st) {
    const int p = st / TILES, t = st % TILES;
    const int tr = GATEUP ? t >> 1 : t;
#pragma unroll
    for (int i = 0; i < CP; ++i) {
      const int e = 1024 * i + 16 * lane;
      const int rr = e / KQ, ch = (e - rr * KQ) >> 4;
      const uint32_t off =
          (uint32_t)((tr * 16 + rr) * K + 1024 * p + wave * KQ + 16 * (ch ^ (rr & 7)));
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128((GATEUP && (t & 1)) ? rQ2 : rQ,
                                                            off, 0, 2 /* nt */);
      R[st % DS][i] = make_uint4(v[0], v[1], v[2], v[3]);
    }
  };
  load_x(0);
  issue(0);
#pragma unroll
  for (int d = 1; d < DS; ++d)
    if (d < STEPS) {
      if (d % TILES == 0) load_x(d / TILES);  // step d opens pass d / TILES
      issue(d);
    }
  f32x4 acc[TILES][MB];
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int g = 0; g < MB; ++g) acc[t][g] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int st = 0; st < STEPS; ++st) {
    const int p = st / TILES, t = st % TILES;
    // step st landed (and its pass's x): at most the loads of the steps
    // after it (and the x loads of the passes they open) still outstanding
    if constexpr (DS == 2) {
      if (st + 1 < STEPS) {
        if ((st + 1) % TILES == 0) __builtin_amdgcn_s_waitcnt(vmcnt_imm(CP + XL));
        else __builtin_amdgcn_s_waitcnt(vmcnt_imm(CP));
      } else {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      }
    } else {
      // the loads of steps st + 1 .. st + DS - 1 (CP each, plus XL x loads
      // for a step that opens a pass); st is a constant once unrolled, so
      // the switch folds to one wait
      int n = 0;
#pragma unroll
      for (int d = 1; d < DS; ++d)
        if (st + d < STEPS) n += CP + ((st + d) % TILES == 0 ? XL : 0);
      switch (n) {
#define MJ_W(c) case c: __builtin_amdgcn_s_waitcnt(vmcnt_imm(c)); break;
        MJ_W(0) MJ_W(1) MJ_W(2) MJ_W(3) MJ_W(4) MJ_W(5) MJ_W(6) MJ_W(7) MJ_W(8) MJ_W(9)
        MJ_W(10) MJ_W(11) MJ_W(12) MJ_W(13) MJ_W(14) MJ_W(15) MJ_W(16) MJ_W(17) MJ_W(18)
        MJ_W(19) MJ_W(20) MJ_W(21) MJ_W(22) MJ_W(23) MJ_W(24) MJ_W(25) MJ_W(26) MJ_W(27)
        MJ_W(28) MJ_W(29) MJ_W(30) MJ_W(31) MJ_W(32)
#undef MJ_W
        default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;
      }
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < CP; ++i)
      *(uint4 *)(mine + (st & 1) * SLOT + 1024 * i + 16 * lane) = R[st % DS][i];
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("" ::: "memory");
    const uint8_t *src = mine + (st & 1) * SLOT + r * KQ;
    uint4 qv[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) qv[j] = *(const uint4 *)(src + 16 * ((4 * j + c) ^ (r & 7)));
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const bf16x8 w0 = i8x8_bf16(qv[j].x, qv[j].y);
      const bf16x8 w1 = i8x8_bf16(qv[j].z, qv[j].w);
#pragma unroll
      for (int g = 0; g < MB; ++g) {
        acc[t][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            w0, __builtin_bit_cast(bf16x8, xa[p % XS][g][j]), acc[t][g], 0, 0, 0);
        acc[t][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            w1, __builtin_bit_cast(bf16x8, xb[p % XS][g][j]), acc[t][g], 0, 0, 0);
      }
    }
    if (st + DS < STEPS) {
      // this wave's fragment reads of the region are done before it is refilled
      __builtin_amdgcn_s_waitcnt(0xC07F);
      asm volatile("" ::: "memory");
      if ((st + DS) % TILES == 0) load_x((st + DS) / TILES);
      issue(st + DS);
    }
  }
  __syncthreads();
  f32x4 *red = (f32x4 *)lds8;
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int g = 0; g < MB; ++g) red[((wave * TILES + t) * MB + g) * 64 + lane] = acc[t][g];
  __syncthreads();
  if (wave >= TP) return;
  // wave w: output columns n0 + 16 w.. (tile w, or gate tile 2 w and up tile 2 w + 1)
  constexpr int TS = GATEUP ? 2 : 1;
#pragma unroll
  for (int g = 0; g < MB; ++g) {
    f32x4 sum = red[((0 * TILES + TS * wave) * MB + g) * 64 + lane];
#pragma unroll
    for (int w = 1; w < NWV; ++w) sum += red[((w * TILES + TS * wave) * MB + g) * 64 + lane];
    f32x4 sum2 = sum;
    if constexpr (GATEUP) {
      sum2 = red[((0 * TILES + 2 * wave + 1) * MB + g) * 64 + lane];
#pragma unroll
      for (int w = 1; w < NWV; ++w) sum2 += red[((w * TILES + 2 * wave + 1) * MB + g) * 64 + lane];
    }
    const int m = 16 * g + r;
    if (m >= M) continue;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n0 + 16 * wave + 4 * c + q;
      if (n >= N) break;
      float v;
      if constexpr (GATEUP) {
        const float gv = epi_scale_bias(sum[q], scales[n], 0.0f, true, false);
        const float uv = epi_scale_bias(sum2[q], scales2[n], 0.0f, true, false);
        {
#pragma clang fp contract(off)
          v = silu_b16(gv) * uv;
        }
      } else {
        {
#pragma clang fp contract(off)
          v = sum[q] * scales[n];
          if (bias) v = v + bias[n];
        }
        v = apply_epi_b16(epi, v);
      }
      y[(size_t)m * N + n] = (uint16_t)f32_to_bf16_bits(v);
    }
  }
}

template <int NP, int TILES, int MB, bool GATEUP, int DS = 2>
static hipError_t launch_skinny_k(const uint16_t *x, const int8_t *Q, const int8_t *Q2,
                               const float *scales, const float *scales2, const float *bias,
                               int epi, uint16_t *y, int64_t M, int64_t N, int64_t K,
                               hipStream_t stream) {
  constexpr size_t slots = size_t(8) * 2 * 16 * 128;
  constexpr size_t red = size_t(8) * TILES * MB * 64 * sizeof(f32x4);
  constexpr size_t lds = slots > red ? slots : red;
  static_assert(lds <= 160 * 1024, "LDS budget");
  auto kern = gemv_w8a16_skinny_kernel<NP, TILES, MB, GATEUP, DS>;
  static std::atomic<uint64_t> attr_set{0};
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
  const uint64_t bit = dev < 64 ? (uint64_t)1 << dev : 0;
  if (!bit || !(attr_set.load(std::memory_order_acquire) & bit)) {
    hipError_t e = hipFuncSetAttribute((const void *)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set.fetch_or(bit, std::memory_order_release);
  }
  constexpr int cols = 16 * (GATEUP ? TILES / 2 : TILES);
  hipLaunchKernelGGL(kern, dim3((unsigned)((N + cols - 1) / cols)), dim3(512), lds, stream, x, Q,
                     Q2, scales, scales2, bias, epi, y, (int)M, (int)N, (int)K);
  return hipGetLastError();
}

// NP = ceil(K / 1024) passes: up to 4 (K <= 4096) for TILES > 1, up to 16
// (K <= 16384) for one tile per workgroup.  Four steps in flight: against two,
// alternating runs on one box on MI355X, the FFN's down projection 4096 x
// 11008 at M = 5 / 8 / 16 13.3 / 13.7 / 16.9 -> 12.6 / 13.1 / 15.8 us (one
// tile; three steps: 13.0 / 13.3 / 16.3), 11008 x 4096 at M = 4 / 16 / 32 /
// 48 11.0-11.1 / 12.3 / 16.8 / 22.3 -> 10.8-10.9 / 12.4-12.6 / 16.1-16.2 /
// 21.4-21.5 us, the decode FFN at M = 4 / 16 30.4 / 35.8-37.1 -> 29.9 /
// 35.1-35.2 us
template <int TILES, int MB, bool GATEUP = false>
static hipError_t launch_skinny(const uint16_t *x, const int8_t *Q, const int8_t *Q2,
                             const float *scales, const float *scales2, const float *bias,
                             int epi, uint16_t *y, int64_t M, int64_t N, int64_t K,
                             hipStream_t stream) {
  const int np = (int)((K + 1023) / 1024);
#define MJ_MK(n)                                                                             \
  case n:                                                                                    \
    return launch_skinny_k<n, TILES, MB, GATEUP, 4>(x, Q, Q2, scales, scales2, bias, epi, y, M, \
                                                    N, K, stream);
  if constexpr (TILES > 1) {
    switch (np) {
      MJ_MK(1) MJ_MK(2) MJ_MK(3) MJ_MK(4)
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (np) {
      MJ_MK(5) MJ_MK(6) MJ_MK(7) MJ_MK(8) MJ_MK(9) MJ_MK(10) MJ_MK(11) MJ_MK(12) MJ_MK(13)
      MJ_MK(14) MJ_MK(15) MJ_MK(16)
      default: return hipErrorInvalidValue;
    }
  }
#undef MJ_MK
}

// Decode GEMV for one x row (M = 1, K = 1024, 2048, 3072 or 4096): persistent
// streaming.
//
// One workgroup per CU (the grid stays below the CU count: a second workgroup
// on a CU doubles that CU's share of the weight stream, and 256 workgroups on
// the 256-CU part measured as slow as 276).  A workgroup owns 4*RW
// consecutive weight rows; wave v takes rows v, v + 4, v + 8, ... so the four
// waves of a CU read neighbouring 4-KB rows at each step.  x is loaded first,
// straight into registers, and converted to fp32 once per wave: lane l owns k
// chunks l, l + 64, ... of 16 elements, for every row.  Each row is four 1-KB
// nontemporal loads (16 bytes per lane); D rows are in flight per wave and the
// loads of row r + D are issued after row r's arithmetic (sched_barrier fences
// keep that order: left free, the scheduler grouped the issues of several rows
// and the stream stalled).  The row dot is 64 widening multiply-adds per lane;
// four rows' lane sums are reduced together (two v_permlane32_swap, one
// v_permlane16_swap and four DPP adds leave row j's total in 16-lane row j),
// then scale, bias and the activation are applied and 16-lane row j stores
// its output.  The row index arithmetic uses a wave index taken through
// readfirstlane: otherwise the compiler treats the per-wave buffer resource as
// divergent and wraps every load in a readfirstlane loop.
//
// Measured on MI355X, 11008 x 4096 (graph replay over 8 weight copies that do
// not fit the MALL, interleaved A/B in one process): 8.43 us against 9.79 us
// for the 2-rows-per-wave kernel above; a pure 45 MB read takes 7.72 us.
constexpr int kGemvStreamMaxWgs = 252;

__device__ __forceinline__ float dpp_row_sum(float v) {
#define MJ_DPP_F(v, ctrl) \
  __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, false))
  v += MJ_DPP_F(v, 0xB1);   // quad_perm [1,0,3,2]
  v += MJ_DPP_F(v, 0x4E);   // quad_perm [2,3,0,1]
  v += MJ_DPP_F(v, 0x124);  // row_ror:4
  v += MJ_DPP_F(v, 0x128);  // row_ror:8
#undef MJ_DPP_F
  return v;
}

// Lane partial sums p0..p3 of four rows -> every lane of 16-lane row j holds
// the 64-lane total of p_j.
__device__ __forceinline__ float reduce4_rows(float p0, float p1, float p2, float p3) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(p0), __float_as_uint(p2), false,
                                                  false);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(p1), __float_as_uint(p3), false,
                                                  false);
  // lanes 0-31: p0 (p1) halves summed, lanes 32-63: p2 (p3)
  const float r02 = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const float r13 = __uint_as_float(b[0]) + __uint_as_float(b[1]);
  const auto c = __builtin_amdgcn_permlane16_swap(__float_as_uint(r02), __float_as_uint(r13),
                                                  false, false);
  return dpp_row_sum(__uint_as_float(c[0]) + __uint_as_float(c[1]));
}

template <int CPL, int RW, int D>
__global__ __launch_bounds__(256) void gemv_w8a16_stream_kernel(
    const uint16_t *__restrict__ x, const int8_t *__restrict__ Q, const float *__restrict__ scales,
    const float *__restrict__ bias, int epi, uint16_t *__restrict__ y, int N, int K) {
  constexpr int NG = (RW + 3) / 4;  // groups of four rows reduced together
  constexpr int NS = D;             // weight register slots
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = blockIdx.x * 4 * RW + wave;  // rows row0 + 4 i
  if (row0 >= N) return;
  const int rows = (N - row0 + 3) / 4 < RW ? (N - row0 + 3) / 4 : RW;

  // lane 16 j + g (g < NG) finishes the wave's row 4 g + j, i.e. weight row
  // row0 + 4 (4 g + j): its scale and bias are loaded first
  const int my_rr = 4 * (lane & 15) + (lane >> 4);
  const bool my_out = (lane & 15) < NG && my_rr < rows;
  const int my_n = row0 + 4 * (my_rr < rows ? my_rr : rows - 1);
  const float my_s = scales[my_n];
  const float my_b = bias ? bias[my_n] : 0.0f;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (int64_t)K * 2);
  uint4 xa[CPL], xb[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)((c * 64 + lane) * 32), 0, 0);
    const u32x4 b =
        __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)((c * 64 + lane) * 32 + 16), 0, 0);
    xa[c] = make_uint4(a[0], a[1], a[2], a[3]);
    xb[c] = make_uint4(b[0], b[1], b[2], b[3]);
  }
  const __amdgpu_buffer_rsrc_t rQ =
      make_rsrc(Q + (size_t)row0 * K, (int64_t)(4 * (rows - 1) + 1) * K);
  uint4 q[NS][CPL];
  // K == 1024 * CPL: every lane chunk lies inside the row, so the only
  // per-load choice is a select on the row (rows past the wave's read zero);
  // a per-chunk test compiled into branches around every load
  auto issue = [&](int r, int slot) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const uint32_t off = r < rows ? (uint32_t)(4 * r * K + (c * 64 + lane) * 16) : kOobOffset;
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rQ, off, 0, 2 /* nt */);
      q[slot][c] = make_uint4(v[0], v[1], v[2], v[3]);
    }
  };
#pragma unroll
  for (int d = 0; d < D; ++d) issue(d, d);
  __builtin_amdgcn_sched_barrier(0);

  float xf[CPL][16];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const uint32_t xw[8] = {xa[c].x, xa[c].y, xa[c].z, xa[c].w, xb[c].x, xb[c].y, xb[c].z, xb[c].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xf[c][2 * e] = __uint_as_float(xw[e] << 16);
      xf[c][2 * e + 1] = __uint_as_float(xw[e] & 0xFFFF0000u);
    }
  }

  float part[4], tot[NG];
#pragma unroll
  for (int r = 0; r < NG * 4; ++r) {
    float a = 0.0f;
    if (r < RW) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const uint32_t qw[4] = {q[r % NS][c].x, q[r % NS][c].y, q[r % NS][c].z, q[r % NS][c].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int32_t v = (int32_t)qw[e];
          a += xf[c][4 * e + 0] * (float)((v << 24) >> 24);
          a += xf[c][4 * e + 1] * (float)((v << 16) >> 24);
          a += xf[c][4 * e + 2] * (float)((v << 8) >> 24);
          a += xf[c][4 * e + 3] * (float)(v >> 24);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (r + D < RW) issue(r + D, r % NS);
      __builtin_amdgcn_sched_barrier(0);
    }
    part[r % 4] = a;
    if (r % 4 == 3) tot[r / 4] = reduce4_rows(part[0], part[1], part[2], part[3]);
  }
  // every lane of 16-lane row j holds tot[g] = row 4 g + j: lane 16 j + g
  // takes tot[g], so one activation evaluation covers all groups (an
  // epilogue per group, with the activation switch, made the kernel 1 us
  // slower: 2370 instructions against ~1900)
  float t = tot[0];
#pragma unroll
  for (int g = 1; g < NG; ++g) t = (lane & 15) == g ? tot[g] : t;
  float v;
  {
#pragma clang fp contract(off)
    v = t * my_s;
    if (bias) v = v + my_b;
  }
  v = apply_epi_b16(epi, v);
  if (my_out) y[my_n] = (uint16_t)f32_to_bf16_bits(v);
}

// Decode GEMV for one x row at K = 4096: the 4 waves of a workgroup split K.
//
// A workgroup owns RW consecutive weight rows; lane l of wave w takes the
// 16-byte chunk 64 w + l of every one of them, so each row is one 1-KB load
// per wave (the four waves of a CU read the four quarters of the same 4-KB
// row), and a wave needs only its 32 bytes of x (16 values, converted once).
// Against the row-per-wave kernel above each CU reads x from L2 once instead
// of four times (2 MB per launch instead of 8) and keeps 16 x values in
// registers instead of 64.  D rows are in flight per wave; the loads of row
// r + D are issued before row r's arithmetic.  Four rows' lane sums are
// reduced together as above (reduce4_rows); lane 16 j + g of each wave then
// holds the wave's partial of row 4 g + j, the four partials of a row meet in
// LDS and wave 0 adds them in wave order, applies scale, bias and the
// activation and stores the workgroup's RW outputs.
//
// Measured on MI355X, 11008 x 4096 (graph replay over 8 weight copies, A/B
// in one process, outputs within the bf16 tolerance of each other): 8.32-8.37
// us against 8.43-8.48 us for the kernel above, in every one of 8 runs; rows
// in flight D = 6..12 within 1 %, 43 rows on all 256 workgroups no faster.
template <int RW, int D>
__global__ __launch_bounds__(256) void gemv_w8a16_ksplit_kernel(
    const uint16_t *__restrict__ x, const int8_t *__restrict__ Q, const float *__restrict__ scales,
    const float *__restrict__ bias, int epi, uint16_t *__restrict__ y, int N) {
  constexpr int K = 4096;
  constexpr int NG = (RW + 3) / 4;  // groups of four rows reduced together
  constexpr int NS = D + 1;         // weight register slots
  __shared__ float part[4][NG * 4];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = blockIdx.x * RW;
  const int rows = N - row0 < RW ? N - row0 : RW;
  const int ch = wave * 64 + lane;  // 16-byte chunk of every row
  const __amdgpu_buffer_rsrc_t rQ = make_rsrc(Q + (size_t)row0 * K, (int64_t)rows * K);
  uint4 q[NS];
  auto issue = [&](int r, int slot) {
    const uint32_t off = r < rows ? (uint32_t)(r * K + ch * 16) : kOobOffset;
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rQ, off, 0, 2 /* nt */);
    q[slot] = make_uint4(v[0], v[1], v[2], v[3]);
  };
  // row 0, then x (its wait then covers row 0 as well: loads retire in
  // order), then rows 1 .. D-1, then wave 0's scale and bias of the output rows
  issue(0, 0);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (int64_t)K * 2);
  const u32x4 xa = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(ch * 32), 0, 0);
  const u32x4 xb = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(ch * 32 + 16), 0, 0);
#pragma unroll
  for (int d = 1; d < D; ++d) issue(d, d);
  float my_s = 1.0f, my_b = 0.0f;
  if (wave == 0) {
    const int t = lane < rows ? lane : rows - 1;
    my_s = scales[row0 + t];
    my_b = (bias ? bias : scales)[row0 + t];
  }
  __builtin_amdgcn_sched_barrier(0);
  float xf[16];
  {
    const uint32_t xw[8] = {xa[0], xa[1], xa[2], xa[3], xb[0], xb[1], xb[2], xb[3]};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xf[2 * e] = __uint_as_float(xw[e] << 16);
      xf[2 * e + 1] = __uint_as_float(xw[e] & 0xFFFF0000u);
    }
  }
  float p4[4], tot[NG];
#pragma unroll
  for (int r = 0; r < NG * 4; ++r) {
    float a = 0.0f;
    if (r < RW) {
      __builtin_amdgcn_sched_barrier(0);
      if (r + D < RW) issue(r + D, (r + D) % NS);
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t qw[4] = {q[r % NS].x, q[r % NS].y, q[r % NS].z, q[r % NS].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int32_t v = (int32_t)qw[e];
        a += xf[4 * e + 0] * (float)((v << 24) >> 24);
        a += xf[4 * e + 1] * (float)((v << 16) >> 24);
        a += xf[4 * e + 2] * (float)((v << 8) >> 24);
        a += xf[4 * e + 3] * (float)(v >> 24);
      }
    }
    p4[r % 4] = a;
    if (r % 4 == 3) tot[r / 4] = reduce4_rows(p4[0], p4[1], p4[2], p4[3]);
  }
  // every lane of 16-lane row j holds tot[g] = the wave's partial of row 4 g + j
  float t = tot[0];
#pragma unroll
  for (int g = 1; g < NG; ++g) t = (lane & 15) == g ? tot[g] : t;
  if ((lane & 15) < NG) part[wave][4 * (lane & 15) + (lane >> 4)] = t;
  __syncthreads();
  if (wave == 0 && lane < rows) {
    float v = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
    {
#pragma clang fp contract(off)
      v = v * my_s;
      if (bias) v = v + my_b;
    }
    y[row0 + lane] = (uint16_t)f32_to_bf16_bits(apply_epi_b16(epi, v));
  }
}

// The K-split GEMV for one x row at other K (K % 16 == 0, K <= 4096 CPL) and
// the FFN's fused gate/up at one x row.  As gemv_w8a16_ksplit_kernel: the 4
// waves split K, lane l of wave w taking 16-byte chunks 64 w + l + 256 c (c <
// CPL) of every row, D rows in flight per wave, four rows' lane sums reduced
// together, the waves' partials added in wave order.  GATEUP: the workgroup's
// rows alternate gate row n and up row n of output column n (weights Q and
// Q2, scales and scales2), and column n gets bf16(silu(g sg[n]) * (u su[n]))
// from the fp32 sums, as the GEMM's gate/up epilogue.
template <int RW, int D, int CPL, bool GATEUP>
__global__ __launch_bounds__(256) void gemv_w8a16_ksplit_g_kernel(
    const uint16_t *__restrict__ x, const int8_t *__restrict__ Q, const int8_t *__restrict__ Q2,
    const float *__restrict__ scales, const float *__restrict__ scales2,
    const float *__restrict__ bias, int epi, uint16_t *__restrict__ y, int N, int K) {
  constexpr int NG = (RW + 3) / 4;  // groups of four rows reduced together
  constexpr int NS = D + 1;         // weight register slots
  constexpr int COLS = GATEUP ? RW / 2 : RW;
  static_assert(!GATEUP || RW % 2 == 0, "gate/up rows come in pairs");
  static_assert(COLS <= 64, "one output per lane of wave 0");
  __shared__ float part[4][NG * 4];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col0 = blockIdx.x * COLS;
  const int cols = N - col0 < COLS ? N - col0 : COLS;
  const int rows = GATEUP ? 2 * cols : cols;
  const int nch = K / 16;
  const int ch0 = wave * 64 + lane;
  const __amdgpu_buffer_rsrc_t rQ = make_rsrc(Q + (size_t)col0 * K, (int64_t)cols * K);
  const __amdgpu_buffer_rsrc_t rQ2 =
      make_rsrc((GATEUP ? Q2 : Q) + (size_t)col0 * K, (int64_t)cols * K);
  uint4 q[NS][CPL];
  auto issue = [&](int r, int slot) {
    const int rr = GATEUP ? r >> 1 : r;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ch = ch0 + 256 * c;
      const uint32_t off = r < rows && ch < nch ? (uint32_t)(rr * K + ch * 16) : kOobOffset;
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128((GATEUP && (r & 1)) ? rQ2 : rQ, off,
                                                            0, 2 /* nt */);
      q[slot][c] = make_uint4(v[0], v[1], v[2], v[3]);
    }
  };
  issue(0, 0);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (int64_t)K * 2);
  u32x4 xa[CPL], xb[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = ch0 + 256 * c;
    const uint32_t xo = ch < nch ? (uint32_t)(ch * 32) : kOobOffset;
    xa[c] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);
    xb[c] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo == kOobOffset ? xo : xo + 16, 0, 0);
  }
#pragma unroll
  for (int d = 1; d < D; ++d) issue(d, d);
  // wave 0's scales (and bias) of its outputs
  float my_s = 1.0f, my_s2 = 1.0f, my_b = 0.0f;
  if (wave == 0) {
    const int t = lane < cols ? lane : cols - 1;
    my_s = scales[col0 + t];
    if (GATEUP) my_s2 = scales2[col0 + t];
    else my_b = (bias ? bias : scales)[col0 + t];
  }
  __builtin_amdgcn_sched_barrier(0);
  float xf[CPL][16];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const uint32_t xw[8] = {xa[c][0], xa[c][1], xa[c][2], xa[c][3],
                            xb[c][0], xb[c][1], xb[c][2], xb[c][3]};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xf[c][2 * e] = __uint_as_float(xw[e] << 16);
      xf[c][2 * e + 1] = __uint_as_float(xw[e] & 0xFFFF0000u);
    }
  }
  float p4[4];
#pragma unroll
  for (int r = 0; r < NG * 4; ++r) {
    float a = 0.0f;
    if (r < RW) {
      __builtin_amdgcn_sched_barrier(0);
      if (r + D < RW) issue(r + D, (r + D) % NS);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const uint32_t qw[4] = {q[r % NS][c].x, q[r % NS][c].y, q[r % NS][c].z, q[r % NS][c].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int32_t v = (int32_t)qw[e];
          a += xf[c][4 * e + 0] * (float)((v << 24) >> 24);
          a += xf[c][4 * e + 1] * (float)((v << 16) >> 24);
          a += xf[c][4 * e + 2] * (float)((v << 8) >> 24);
          a += xf[c][4 * e + 3] * (float)(v >> 24);
        }
      }
    }
    p4[r % 4] = a;
    if (r % 4 == 3) {
      // every lane of 16-lane row j holds the wave's partial of row r - 3 + j;
      // one lane of each row stores it (no partial stays live across the loop)
      const float t = reduce4_rows(p4[0], p4[1], p4[2], p4[3]);
      if ((lane & 15) == ((r / 4) & 15)) part[wave][r - 3 + (lane >> 4)] = t;
    }
  }
  __syncthreads();
  if (wave != 0 || lane >= cols) return;
  const int n = col0 + lane;
  if (GATEUP) {
    const int rg = 2 * lane, ru = 2 * lane + 1;
    const float g = ((part[0][rg] + part[1][rg]) + part[2][rg]) + part[3][rg];
    const float u = ((part[0][ru] + part[1][ru]) + part[2][ru]) + part[3][ru];
    float h;
    {
#pragma clang fp contract(off)
      const float gv = epi_scale_bias(g, my_s, 0.0f, true, false);
      const float uv = epi_scale_bias(u, my_s2, 0.0f, true, false);
      h = silu_b16(gv) * uv;
    }
    y[n] = (uint16_t)f32_to_bf16_bits(h);
  } else {
    float v = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
    {
#pragma clang fp contract(off)
      v = v * my_s;
      if (bias) v = v + my_b;
    }
    y[n] = (uint16_t)f32_to_bf16_bits(apply_epi_b16(epi, v));
  }
}

template <int RW, int CPL, bool GATEUP>
static hipError_t launch_ksplit_g(const uint16_t *x, const int8_t *Q, const int8_t *Q2,
                                  const float *scales, const float *scales2, const float *bias,
                                  int epi, uint16_t *y, int64_t N, int64_t K,
                                  hipStream_t stream) {
  // rows in flight per wave: 8 one-chunk rows, 4 rows of 3 or 4 chunks (the
  // same bytes in flight within registers)
  constexpr int DM = CPL >= 3 ? 4 : 8;
  constexpr int D = RW < DM ? RW : DM;
  constexpr int COLS = GATEUP ? RW / 2 : RW;
  const unsigned grid = (unsigned)((N + COLS - 1) / COLS);
  hipLaunchKernelGGL((gemv_w8a16_ksplit_g_kernel<RW, D, CPL, GATEUP>), dim3(grid), dim3(256), 0,
                     stream, x, Q, Q2, scales, scales2, bias, epi, y, (int)N, (int)K);
  return hipGetLastError();
}

// Rows per workgroup: of 4, 8, 16, 32, 48, 64 and (gate/up) 88, at most 88
// one-chunk rows, 64 of two chunks, 48 of three, 32 of four (beyond those the
// compiler stops unrolling the row loop and the weight slots go to scratch),
// the one with the least ceil(workgroups / 256) * (rows + 2): the rounds of
// workgroups over the 256 CUs times a round's rows and a fixed cost of about
// two rows (the workgroup's x reads, its start and its reduction); ties to
// more rows.  MI355X, one x row: 4096 x 11008 (three chunks) at 8 / 16 / 24 /
// 32 rows 9.3 / 8.8 / 9.9 / 11.0 us; gate/up 2 x 11008 x 4096 at 88 / 64 /
// 48 / 32 rows (250 / 344 / 459 / 688 workgroups): the FFN 25.7 / 28.6 /
// 26.1 / 26.9 us.
template <int CPL, bool GATEUP>
static hipError_t launch_ksplit_g_rw(const uint16_t *x, const int8_t *Q, const int8_t *Q2,
                                     const float *scales, const float *scales2,
                                     const float *bias, int epi, uint16_t *y, int64_t N, int64_t K,
                                     hipStream_t stream) {
  constexpr int kRows[] = {4, 8, 16, 32, 48, 64, 88};
  constexpr int kMaxRows = CPL >= 4 ? 32 : CPL == 3 ? 48 : CPL == 2 ? 64 : GATEUP ? 88 : 64;
  int rw = 4;
  int64_t best = INT64_MAX;
  for (const int r : kRows) {
    if (r > kMaxRows) break;
    const int64_t wgs = (N + (GATEUP ? r / 2 : r) - 1) / (GATEUP ? r / 2 : r);
    const int64_t cost = (wgs + 255) / 256 * (r + 2);
    if (cost <= best) best = cost, rw = r;
  }
#define MJ_KG(r)                                                                        \
  case r:                                                                               \
    if constexpr (r <= kMaxRows)                                                        \
      return launch_ksplit_g<r, CPL, GATEUP>(x, Q, Q2, scales, scales2, bias, epi, y, N, K, \
                                             stream);                                   \
    break;
  switch (rw) {
    MJ_KG(4) MJ_KG(8) MJ_KG(16) MJ_KG(32) MJ_KG(48) MJ_KG(64) MJ_KG(88)
  }
#undef MJ_KG
  return hipErrorInvalidValue;
}

// The K-split GEMV at 2..MR x rows (MR = 2 or 4, K % 16 == 0, K <= 4096 CPL),
// plain or gate/up as gemv_w8a16_ksplit_g_kernel: the same weight stream (lane
// l of wave w takes 16-byte chunks 64 w + l + 256 c of every row, D rows in
// flight), but each weight chunk is widened once to eight bf16 pairs (exact)
// and multiplied against every x row's chunk with v_dot2_f32_bf16 (two exact
// products and the running sum per instruction), x kept as the raw bf16 pairs
// in registers (rows past M load zeros).  Per x row the lane sums go through
// the same four-row reduction into LDS, and the waves' partials are added in
// wave order; thread t of the workgroup then stores x row t / cols.
template <int RW, int D, int CPL, int MR, bool GATEUP>
__global__ __launch_bounds__(256) void gemv_w8a16_ksplit_m_kernel(
    const uint16_t *__restrict__ x, const int8_t *__restrict__ Q, const int8_t *__restrict__ Q2,
    const float *__restrict__ scales, const float *__restrict__ scales2,
    const float *__restrict__ bias, int epi, uint16_t *__restrict__ y, int M, int N, int K) {
  typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
  constexpr int NG = (RW + 3) / 4;
  constexpr int NS = D + 1;
  constexpr int COLS = GATEUP ? RW / 2 : RW;
  static_assert(!GATEUP || RW % 2 == 0, "gate/up rows come in pairs");
  static_assert(MR * COLS <= 256, "one output per thread");
  __shared__ float part[4][MR][NG * 4];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col0 = blockIdx.x * COLS;
  const int cols = N - col0 < COLS ? N - col0 : COLS;
  const int rows = GATEUP ? 2 * cols : cols;
  const int nch = K / 16;
  const int ch0 = wave * 64 + lane;
  const __amdgpu_buffer_rsrc_t rQ = make_rsrc(Q + (size_t)col0 * K, (int64_t)cols * K);
  const __amdgpu_buffer_rsrc_t rQ2 =
      make_rsrc((GATEUP ? Q2 : Q) + (size_t)col0 * K, (int64_t)cols * K);
  uint4 q[NS][CPL];
  auto issue = [&](int r, int slot) {
    const int rr = GATEUP ? r >> 1 : r;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ch = ch0 + 256 * c;
      const uint32_t off = r < rows && ch < nch ? (uint32_t)(rr * K + ch * 16) : kOobOffset;
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128((GATEUP && (r & 1)) ? rQ2 : rQ, off,
                                                            0, 2 /* nt */);
      q[slot][c] = make_uint4(v[0], v[1], v[2], v[3]);
    }
  };
  issue(0, 0);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (int64_t)M * K * 2);
  u32x4 xa[MR][CPL], xb[MR][CPL];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ch = ch0 + 256 * c;
      const uint32_t xo = m < M && ch < nch ? (uint32_t)((m * K + ch * 16) * 2) : kOobOffset;
      xa[m][c] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);
      xb[m][c] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo == kOobOffset ? xo : xo + 16, 0, 0);
    }
#pragma unroll
  for (int d = 1; d < D; ++d) issue(d, d);
  __builtin_amdgcn_sched_barrier(0);
  float p4[MR][4];
#pragma unroll
  for (int r = 0; r < NG * 4; ++r) {
    float a[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) a[m] = 0.0f;
    if (r < RW) {
      __builtin_amdgcn_sched_barrier(0);
      if (r + D < RW) issue(r + D, (r + D) % NS);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const uint4 qc = q[r % NS][c];
        const bf16x8 wl = i8x8_bf16(qc.x, qc.y), wh = i8x8_bf16(qc.z, qc.w);
        const uint4 w0 = __builtin_bit_cast(uint4, wl), w1 = __builtin_bit_cast(uint4, wh);
        const uint32_t wp[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const uint32_t xp[8] = {xa[m][c][0], xa[m][c][1], xa[m][c][2], xa[m][c][3],
                                  xb[m][c][0], xb[m][c][1], xb[m][c][2], xb[m][c][3]};
#pragma unroll
          for (int e = 0; e < 8; ++e)
            a[m] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wp[e]),
                                                   __builtin_bit_cast(bf16x2, xp[e]), a[m],
                                                   false);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) p4[m][r % 4] = a[m];
    if (r % 4 == 3) {
      // every lane of 16-lane row j holds x row m's partial of weight row r - 3 + j
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const float t = reduce4_rows(p4[m][0], p4[m][1], p4[m][2], p4[m][3]);
        if ((lane & 15) == ((r / 4) & 15)) part[wave][m][r - 3 + (lane >> 4)] = t;
      }
    }
  }
  __syncthreads();
  const int m = threadIdx.x / COLS, col = threadIdx.x - m * COLS;
  if (m >= MR || m >= M || col >= cols) return;
  const int n = col0 + col;
  if (GATEUP) {
    const int rg = 2 * col, ru = 2 * col + 1;
    const float g = ((part[0][m][rg] + part[1][m][rg]) + part[2][m][rg]) + part[3][m][rg];
    const float u = ((part[0][m][ru] + part[1][m][ru]) + part[2][m][ru]) + part[3][m][ru];
    float h;
    {
#pragma clang fp contract(off)
      const float gv = epi_scale_bias(g, scales[n], 0.0f, true, false);
      const float uv = epi_scale_bias(u, scales2[n], 0.0f, true, false);
      h = silu_b16(gv) * uv;
    }
    y[(size_t)m * N + n] = (uint16_t)f32_to_bf16_bits(h);
  } else {
    float v = ((part[0][m][col] + part[1][m][col]) + part[2][m][col]) + part[3][m][col];
    {
#pragma clang fp contract(off)
      v = v * scales[n];
      if (bias) v = v + bias[n];
    }
    y[(size_t)m * N + n] = (uint16_t)f32_to_bf16_bits(apply_epi_b16(epi, v));
  }
}

template <int RW, int CPL, int MR, bool GATEUP>
static hipError_t launch_ksplit_m(const uint16_t *x, const int8_t *Q, const int8_t *Q2,
                                  const float *scales, const float *scales2, const float *bias,
                                  int epi, uint16_t *y, int64_t M, int64_t N, int64_t K,
                                  hipStream_t stream) {
  constexpr int DM = CPL >= 3 ? 4 : 8;
  constexpr int D = RW < DM ? RW : DM;
  constexpr int COLS = GATEUP ? RW / 2 : RW;
  const unsigned grid = (unsigned)((N + COLS - 1) / COLS);
  hipLaunchKernelGGL((gemv_w8a16_ksplit_m_kernel<RW, D, CPL, MR, GATEUP>), dim3(grid), dim3(256),
                     0, stream, x, Q, Q2, scales, scales2, bias, epi, y, (int)M, (int)N, (int)K);
  return hipGetLastError();
}

// rows per workgroup by the rule of launch_ksplit_g_rw, at most 64 (two x
// rows) or 48 (four) one-chunk rows, 16 rows of four chunks at four x rows,
// else 32 (past those the row loop is not unrolled and spills)
template <int CPL, int MR, bool GATEUP>
static hipError_t launch_ksplit_m_rw(const uint16_t *x, const int8_t *Q, const int8_t *Q2,
                                     const float *scales, const float *scales2,
                                     const float *bias, int epi, uint16_t *y, int64_t M,
                                     int64_t N, int64_t K, hipStream_t stream) {
  constexpr int kRows[] = {4, 8, 16, 32, 48, 64, 88};
  constexpr int kMaxRows = CPL == 1 ? (MR <= 2 ? 64 : 48) : CPL >= 4 && MR >= 4 ? 16 : 32;
  int rw = 4;
  int64_t best = INT64_MAX;
  for (const int r : kRows) {
    if (r > kMaxRows) break;
    const int64_t wgs = (N + (GATEUP ? r / 2 : r) - 1) / (GATEUP ? r / 2 : r);
    const int64_t cost = (wgs + 255) / 256 * (r + 2);
    if (cost <= best) best = cost, rw = r;
  }
#define MJ_KM(r)                                                                          \
  case r:                                                                                 \
    if constexpr (r <= kMaxRows)                                                          \
      return launch_ksplit_m<r, CPL, MR, GATEUP>(x, Q, Q2, scales, scales2, bias, epi, y, M, \
                                                 N, K, stream);                           \
    break;
  switch (rw) {
    MJ_KM(4) MJ_KM(8) MJ_KM(16) MJ_KM(32) MJ_KM(48) MJ_KM(64) MJ_KM(88)
  }
#undef MJ_KM
  return hipErrorInvalidValue;
}

template <int MR, bool GATEUP>
static hipError_t launch_ksplit_m_k(const uint16_t *x, const int8_t *Q, const int8_t *Q2,
                                    const float *scales, const float *scales2, const float *bias,
                                    int epi, uint16_t *y, int64_t M, int64_t N, int64_t K,
                                    hipStream_t stream) {
  if (K <= 4096)
    return launch_ksplit_m_rw<1, MR, GATEUP>(x, Q, Q2, scales, scales2, bias, epi, y, M, N, K,
                                             stream);
  if (K <= 8192)
    return launch_ksplit_m_rw<2, MR, GATEUP>(x, Q, Q2, scales, scales2, bias, epi, y, M, N, K,
                                             stream);
  if (K <= 12288)
    return launch_ksplit_m_rw<3, MR, GATEUP>(x, Q, Q2, scales, scales2, bias, epi, y, M, N, K,
                                             stream);
  return launch_ksplit_m_rw<4, MR, GATEUP>(x, Q, Q2, scales, scales2, bias, epi, y, M, N, K,
                                           stream);
}

// Rows per workgroup of the K-split GEMV: the fewest of these that keep the
// grid within kGemvStreamMaxWgs workgroups (N <= 252 * 64 rows).
template <int RW>
static void launch_ksplit(const uint16_t *x, const int8_t *Q, const float *scales,
                          const float *bias, int epi, uint16_t *y, int64_t N,
                          hipStream_t stream) {
  constexpr int D = RW < 8 ? RW : 8;
  const unsigned grid = (unsigned)((N + RW - 1) / RW);
  hipLaunchKernelGGL((gemv_w8a16_ksplit_kernel<RW, D>), dim3(grid), dim3(256), 0, stream, x, Q,
                     scales, bias, epi, y, (int)N);
}

static bool launch_ksplit_rw(const uint16_t *x, const int8_t *Q, const float *scales,
                             const float *bias, int epi, uint16_t *y, int64_t N,
                             hipStream_t stream) {
  const int64_t need = (N + kGemvStreamMaxWgs - 1) / kGemvStreamMaxWgs;
  if (need <= 4) launch_ksplit<4>(x, Q, scales, bias, epi, y, N, stream);
  else if (need <= 8) launch_ksplit<8>(x, Q, scales, bias, epi, y, N, stream);
  else if (need <= 12) launch_ksplit<12>(x, Q, scales, bias, epi, y, N, stream);
  else if (need <= 16) launch_ksplit<16>(x, Q, scales, bias, epi, y, N, stream);
  else if (need <= 24) launch_ksplit<24>(x, Q, scales, bias, epi, y, N, stream);
  else if (need <= 32) launch_ksplit<32>(x, Q, scales, bias, epi, y, N, stream);
  else if (need <= 44) launch_ksplit<44>(x, Q, scales, bias, epi, y, N, stream);
  else if (need <= 64) launch_ksplit<64>(x, Q, scales, bias, epi, y, N, stream);
  else return false;
  return true;
}

template <int CPL, int RW>
static void launch_stream(const uint16_t *x, const int8_t *Q, const float *scales,
                          const float *bias, int epi, uint16_t *y, int64_t N, int64_t K,
                          hipStream_t stream) {
  constexpr int D = RW < 3 ? RW : 3;
  const unsigned grid = (unsigned)((N + 4 * RW - 1) / (4 * RW));
  hipLaunchKernelGGL((gemv_w8a16_stream_kernel<CPL, RW, D>), dim3(grid), dim3(256), 0, stream, x,
                     Q, scales, bias, epi, y, (int)N, (int)K);
}

template <int CPL>
static void launch_stream_rw(const uint16_t *x, const int8_t *Q, const float *scales,
                             const float *bias, int epi, uint16_t *y, int64_t N, int64_t K,
                             hipStream_t stream) {
  // fewest rows per wave that keep the grid within kGemvStreamMaxWgs
  // workgroups (larger N: 32 rows per wave and more workgroups)
  const int64_t need = (N + 4 * kGemvStreamMaxWgs - 1) / (4 * kGemvStreamMaxWgs);
  if (need <= 1) return launch_stream<CPL, 1>(x, Q, scales, bias, epi, y, N, K, stream);
  if (need <= 2) return launch_stream<CPL, 2>(x, Q, scales, bias, epi, y, N, K, stream);
  if (need <= 4) return launch_stream<CPL, 4>(x, Q, scales, bias, epi, y, N, K, stream);
  if (need <= 6) return launch_stream<CPL, 6>(x, Q, scales, bias, epi, y, N, K, stream);
  if (need <= 8) return launch_stream<CPL, 8>(x, Q, scales, bias, epi, y, N, K, stream);
  if (need <= 11) return launch_stream<CPL, 11>(x, Q, scales, bias, epi, y, N, K, stream);
  if (need <= 16) return launch_stream<CPL, 16>(x, Q, scales, bias, epi, y, N, K, stream);
  if (need <= 24) return launch_stream<CPL, 24>(x, Q, scales, bias, epi, y, N, K, stream);
  return launch_stream<CPL, 32>(x, Q, scales, bias, epi, y, N, K, stream);
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
  if (M == 2 && K <= 16384)
    // 11008 x 4096: 10.1-10.3 us against 11.6-12.3 on the two-rows-per-wave
    // kernel; 4096 x 11008: 10.1 against 14.4 on the MFMA GEMV
    return launch_ksplit_m_k<2, false>(x, Q, nullptr, scales, nullptr, bias, epi, y, M, N, K,
                                       stream);
  if (M >= kGemvMfmaMinM && M <= 48 && K % 1024 == 0 && K <= 4096) {
    if (M <= 16)
      return launch_skinny<3, 1>(x, Q, nullptr, scales, nullptr, bias, epi, y, M, N, K, stream);
    if (M <= 32)
      return launch_skinny<3, 2>(x, Q, nullptr, scales, nullptr, bias, epi, y, M, N, K, stream);
    return launch_skinny<3, 4>(x, Q, nullptr, scales, nullptr, bias, epi, y, M, N, K, stream);
  }
  if (M >= 3 && M <= 4 && K <= 16384)
    // 4096 x 11008: 11.3-12.6 us against 13.1 (M = 5) on the skinny GEMV
    return launch_ksplit_m_k<4, false>(x, Q, nullptr, scales, nullptr, bias, epi, y, M, N, K,
                                       stream);
  if (M >= 5 && M <= kGemvMaxM && K > 4096 && K <= 16384)
    // one 16-row tile per workgroup (256 workgroups at N = 4096; 2 or 3 tiles
    // measured 2.8 and 6.6 us slower over the decode FFN at M = 16)
    return launch_skinny<1, 1>(x, Q, nullptr, scales, nullptr, bias, epi, y, M, N, K, stream);
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
  if (M == 1 && K % 1024 == 0 && K <= 4096 && K > 0) {
    // (a workgroup's <= 64 rows, or a wave's rows spanning 4 (RW - 1) + 1 <=
    // 125 rows, of K bytes: 32-bit offsets)
    if (K == 4096 && launch_ksplit_rw(x, Q, scales, bias, epi, y, N, stream))
      return hipGetLastError();
    if (K == 1024) launch_stream_rw<1>(x, Q, scales, bias, epi, y, N, K, stream);
    else if (K == 2048) launch_stream_rw<2>(x, Q, scales, bias, epi, y, N, K, stream);
    else if (K == 3072) launch_stream_rw<3>(x, Q, scales, bias, epi, y, N, K, stream);
    else launch_stream_rw<4>(x, Q, scales, bias, epi, y, N, K, stream);
    return hipGetLastError();
  }
  if (M == 1 && K > 4096 && K <= 16384) {
    if (K <= 8192)
      return launch_ksplit_g_rw<2, false>(x, Q, nullptr, scales, nullptr, bias, epi, y, N, K,
                                          stream);
    if (K <= 12288)
      return launch_ksplit_g_rw<3, false>(x, Q, nullptr, scales, nullptr, bias, epi, y, N, K,
                                          stream);
    return launch_ksplit_g_rw<4, false>(x, Q, nullptr, scales, nullptr, bias, epi, y, N, K,
                                        stream);
  }
  if (M <= 1) return launch_mb<1>(x, Q, scales, bias, epi, y, M, N, K, stream);
  if (M <= 2) return launch_mb<2>(x, Q, scales, bias, epi, y, M, N, K, stream);
  return hipErrorInvalidValue;  // M > kGemvMaxM is the GEMM's
}

// The FFN's gate/up at M x rows (gemv_gateup_w8a16_takes): h[m][n] =
// bf16(silu(x[m] . Wg[n] * sg[n]) * (x[m] . Wu[n] * su[n])), 16-byte aligned
// x, Wg, Wu.
hipError_t launch_gemv_gateup_w8a16(const uint16_t *x, const int8_t *Wg, const float *sg,
                                    const int8_t *Wu, const float *su, uint16_t *h, int64_t M,
                                    int64_t N, int64_t K, hipStream_t stream) {
  if (!gemv_gateup_w8a16_takes(M, K)) return hipErrorInvalidValue;
  if (M == 2)  // 2 x 11008 x 4096: 17.3 us against 20.3 on the skinny MFMA GEMV
    return launch_ksplit_m_k<2, true>(x, Wg, Wu, sg, su, nullptr, 0, h, M, N, K, stream);
  if (M <= 4 && (K % 1024 || K > 4096))
    return launch_ksplit_m_k<4, true>(x, Wg, Wu, sg, su, nullptr, 0, h, M, N, K, stream);
  if (M >= 3) {
    // three gate/up tile pairs (48 columns) per workgroup: the decode FFN
    // (2 x 11008 x 4096 gate/up) at M = 4 measured 51.3 / 50.1 / 45.0 / 45.1 us
    // with 1 / 2 / 3 / 4 pairs (688 / 344 / 230 / 172 workgroups) on an
    // earlier form of the kernel; the FFN at M = 8 / 16 / 32 31.4 / 35.4 /
    // 42.5 us with 1-KB passes against 33.4 / 38.5 / 47.9 with one 4-KB pass
    if (M <= 16)
      return launch_skinny<6, 1, true>(x, Wg, Wu, sg, su, nullptr, 0, h, M, N, K, stream);
    return launch_skinny<6, 2, true>(x, Wg, Wu, sg, su, nullptr, 0, h, M, N, K, stream);
  }
  if (K <= 4096)
    return launch_ksplit_g_rw<1, true>(x, Wg, Wu, sg, su, nullptr, 0, h, N, K, stream);
  if (K <= 8192)
    return launch_ksplit_g_rw<2, true>(x, Wg, Wu, sg, su, nullptr, 0, h, N, K, stream);
  if (K <= 12288)
    return launch_ksplit_g_rw<3, true>(x, Wg, Wu, sg, su, nullptr, 0, h, N, K, stream);
  return launch_ksplit_g_rw<4, true>(x, Wg, Wu, sg, su, nullptr, 0, h, N, K, stream);
}

}  // namespace mj
