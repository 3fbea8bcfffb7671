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

// Skinny-M W8A16 GEMV for 3 <= M <= 16 and K = 1024 j (j <= 4): the weights
// stream as whole row pieces and reach the MFMA through LDS.  NWV waves split
// K (KQ = K / NWV bytes of every row each); a workgroup owns 16 TILES weight
// rows.  For each 16-row tile a wave copies its share of the 16 rows straight
// into its own LDS region (buffer_load ... lds, 1 KB per instruction: 1024 /
// KQ rows of KQ contiguous bytes), two tiles in flight, then reads the MFMA
// fragments from there: lane (r, c) takes 16 int8 of row r at 16-byte chunk
// 4 j + c of 64-deep block j, widened exactly to bf16, the first 8 k for one
// v_mfma_f32_16x16x32_bf16 and the other 8 for the second, against x
// fragments of the same k that the wave loaded once, into registers, at the
// start.  Chunk p of row r is stored at LDS chunk p ^ (r & 7), so the 8 lanes
// of a 128-byte read phase hit distinct banks.  No barrier in the loop: a wave
// reads only its own region.  The NWV partial 16 x 16 tiles of a row tile are
// added in K order through LDS (deterministic), then scale, bias and the
// activation.
// Measured on MI355X at 11008 x 4096 (graph replay over 8 weight copies):
// M = 3, 8, 16 13.3, 13.7, 15.1 us against 15.3, 17.3, 19.4 for
// gemv_w8a16_mfma_kernel (16 weight rows per workgroup, x re-read per 16 rows,
// 64 bytes of a row per load instruction); four waves of 1-KB rows 13.5, 14.1,
// 15.6.  The copies alone (no fragment reads, no MFMA) take 9.2 us with four
// waves, 10.8 with eight; the rest is the widening (1.5 VALU per weight).
// Refilling a slot as soon as its fragments are in registers (two tiles in
// flight during the compute) measured slower, and a third slot does not fit
// the LDS.
__device__ __forceinline__ void dma16_lds(__amdgpu_buffer_rsrc_t r, void *lds_dst, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void *)lds_dst, 16, off, 0, 0, 2 /* nt */);
}

// s_waitcnt immediate: vmcnt <= n, lgkmcnt and expcnt unconstrained
constexpr int vmcnt_imm(int n) { return (n & 15) | (((n >> 4) & 3) << 14) | 0x0F70; }

template <int TILES, int KB, int NWV, int MB>
__global__ __launch_bounds__(NWV * 64) void gemv_w8a16_skinny_kernel(const uint16_t *__restrict__ x,
                                                                const int8_t *__restrict__ Q,
                                                                const float *__restrict__ scales,
                                                                const float *__restrict__ bias,
                                                                int epi, uint16_t *__restrict__ y,
                                                                int M, int N, int K) {
  constexpr int NJ = 64 / NWV;         // most 64-deep blocks per wave (K <= 4096)
  constexpr int SLOT = 65536 / NWV;    // bytes of one tile's share at K = 4096
  extern __shared__ __attribute__((aligned(16))) uint8_t lds8[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, c = lane >> 4;
  const int n0 = blockIdx.x * 16 * TILES;
  const int rows = N - n0 < 16 * TILES ? N - n0 : 16 * TILES;
  constexpr int KQ = 512 * KB / NWV;  // bytes of a row per wave (K = 512 KB)
  static_assert(KQ >= 128, "eight 16-byte chunks per row share");
  constexpr int nj = KQ / 64;    // 64-deep blocks per wave
  constexpr int ninst = KQ / 64; // 1-KB copies per tile (16 KQ bytes)
  const int kq0 = wave * KQ;
  const __amdgpu_buffer_rsrc_t rQ = make_rsrc(Q + (size_t)n0 * K, (int64_t)rows * K);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (int64_t)M * K * 2);
  uint8_t *mine = lds8 + wave * 2 * SLOT;

  // x fragments of this wave's share, once: group g holds x rows 16 g + r
  uint4 xa[MB][NJ], xb[MB][NJ];
#pragma unroll
  for (int g = 0; g < MB; ++g)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      xa[g][j] = xb[g][j] = make_uint4(0, 0, 0, 0);
      if (j < nj && 16 * g + r < M) {
        const uint32_t xo = (uint32_t)(((16 * g + r) * K + kq0 + 64 * j + 16 * c) * 2);
        const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);
        const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 16, 0, 0);
        xa[g][j] = make_uint4(a[0], a[1], a[2], a[3]);
        xb[g][j] = make_uint4(b[0], b[1], b[2], b[3]);
      }
    }
  // tile t's share -> slot t & 1: copy i, lane l fills LDS byte e = 1024 i + 16 l
  // of the slot, row e / KQ, chunk p = (e % KQ) / 16, from global chunk p ^ (row & 7)
  auto issue = [&](int t) {
    uint8_t *dst = mine + (t & 1) * SLOT;
#pragma unroll
    for (int i = 0; i < ninst; ++i) {
      const int e = 1024 * i + 16 * lane;
      const int rr = e / KQ, p = (e - rr * KQ) >> 4;
      const uint32_t off = (uint32_t)((t * 16 + rr) * K + kq0 + 16 * (p ^ (rr & 7)));
      dma16_lds(rQ, dst + 1024 * i, off);
    }
  };
  issue(0);
  if (TILES > 1) issue(1);
  f32x4 acc[TILES][MB];
#pragma unroll
  for (int t = 0; t < TILES; ++t) {
    // tile t landed: at most the copies of tile t + 1 still outstanding
    if (t + 1 < TILES) __builtin_amdgcn_s_waitcnt(vmcnt_imm(ninst));
    else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    asm volatile("" ::: "memory");
    const uint8_t *src = mine + (t & 1) * SLOT + r * KQ;
    // two independent accumulator chains per x group (the chunk halves), added
    // in a fixed order at the end
    f32x4 ch[MB][2];
#pragma unroll
    for (int g = 0; g < MB; ++g) ch[g][0] = ch[g][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    uint4 qv[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (j < nj) qv[j] = *(const uint4 *)(src + 16 * ((4 * j + c) ^ (r & 7)));
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (j < nj) {
        const bf16x8 w0 = i8x8_bf16(qv[j].x, qv[j].y);
        const bf16x8 w1 = i8x8_bf16(qv[j].z, qv[j].w);
#pragma unroll
        for (int g = 0; g < MB; ++g) {
          ch[g][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              w0, __builtin_bit_cast(bf16x8, xa[g][j]), ch[g][0], 0, 0, 0);
          ch[g][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              w1, __builtin_bit_cast(bf16x8, xb[g][j]), ch[g][1], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < MB; ++g) acc[t][g] = ch[g][0] + ch[g][1];
    if (t + 2 < TILES) {
      // this wave's fragment reads of the slot are done before it is refilled
      __builtin_amdgcn_s_waitcnt(0xC07F);
      asm volatile("" ::: "memory");
      issue(t + 2);
    }
  }
  // every wave is past its last fragment read (and its copies have landed):
  // the slots become the partials [NWV][TILES][MB][64]
  __syncthreads();
  f32x4 *red = (f32x4 *)lds8;
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int g = 0; g < MB; ++g) red[((wave * TILES + t) * MB + g) * 64 + lane] = acc[t][g];
  __syncthreads();
  if (wave >= TILES) return;
#pragma unroll
  for (int g = 0; g < MB; ++g) {
    f32x4 sum = red[((0 * TILES + wave) * MB + g) * 64 + lane];
#pragma unroll
    for (int w = 1; w < NWV; ++w) sum += red[((w * TILES + wave) * MB + g) * 64 + lane];
    // lane: x row m = 16 g + lane % 16, weight rows n0 + 16 wave + 4 (lane / 16) + q
    const int m = 16 * g + r;
    if (m >= M) continue;
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
}

template <int TILES, int KB, int NWV, int MB>
static hipError_t launch_skinny_k(const uint16_t *x, const int8_t *Q, const float *scales,
                                const float *bias, int epi, uint16_t *y, int64_t M, int64_t N,
                                int64_t K, hipStream_t stream) {
  constexpr size_t lds = 2 * 65536;
  static_assert(NWV * TILES * MB * 64 * sizeof(f32x4) <= lds, "partials fit the slots");
  auto kern = gemv_w8a16_skinny_kernel<TILES, KB, NWV, MB>;
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
  hipLaunchKernelGGL(kern, dim3((unsigned)((N + 16 * TILES - 1) / (16 * TILES))), dim3(NWV * 64), lds,
                     stream, x, Q, scales, bias, epi, y, (int)M, (int)N, (int)K);
  return hipGetLastError();
}

template <int TILES, int NWV, int MB>
static hipError_t launch_skinny(const uint16_t *x, const int8_t *Q, const float *scales,
                                const float *bias, int epi, uint16_t *y, int64_t M, int64_t N,
                                int64_t K, hipStream_t stream) {
  switch (K / 512) {
#define MJ_SK(kb) \
  case kb: return launch_skinny_k<TILES, kb, NWV, MB>(x, Q, scales, bias, epi, y, M, N, K, stream);
    MJ_SK(2) MJ_SK(4) MJ_SK(6) MJ_SK(8)
#undef MJ_SK
    default: return hipErrorInvalidValue;
  }
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
  if (M >= kGemvMfmaMinM && M <= 32 && K % 1024 == 0 && K <= 4096) {
    if (M <= 16) return launch_skinny<3, 8, 1>(x, Q, scales, bias, epi, y, M, N, K, stream);
    return launch_skinny<3, 8, 2>(x, Q, scales, bias, epi, y, M, N, K, stream);
  }
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
  if (M <= 1) return launch_mb<1>(x, Q, scales, bias, epi, y, M, N, K, stream);
  if (M <= 2) return launch_mb<2>(x, Q, scales, bias, epi, y, M, N, K, stream);
  return hipErrorInvalidValue;  // M > kGemvMaxM is the GEMM's
}

}  // namespace mj
