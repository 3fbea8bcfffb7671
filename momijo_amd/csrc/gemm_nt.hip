// NT GEMM on gfx950 bf16 MFMA: C[M,N] = epi((A[M,K] . B[N,K]^T) * s[n] + b[n]).
//
// A is bf16 activations, B is bf16 or int8 (per-output-channel quantized)
// weights; both are K-contiguous, the layout of momijo's Linear weight
// [OutF, InF] (learn/nn/layers.mojo:347-348), so every global load is a
// 16-byte run of K.
//
// One workgroup = 8 waves (2 per SIMD) per BM x BN output tile:
//  * two waves share each SIMD, so one wave's LDS / global waits are covered by
//    the other's MFMAs; waves are laid out 2 (M) x 4 (N), each owning a
//    (BM/2) x (BN/4) sub-tile (128 x 64 for the 256 x 256 tile) of
//    v_mfma_f32_16x16x32_bf16 accumulators (the 16 x 16 shape moves 20 %
//    fewer register-file bytes per flop than 32 x 32 x 16: C and D are 1 KB
//    per 16 K flop instead of 4 KB per 32 K; at 4096^3 the kernel is power
//    limited, so that energy is time);
//  * K advances 64 at a time through two LDS stages; the next stage's bf16
//    tiles go from HBM straight into LDS (buffer_load ... lds: no staging
//    registers, no ds_write), issued before the current stage's MFMAs;
//    int8 weight tiles take the register path and are widened to bf16
//    (exactly, |q| <= 127) on their way into LDS, so the MFMA loop is the
//    same for both weight types;
//  * raw buffer loads return zero for offsets outside their resource: edge
//    tiles (rows >= M, chunks >= K) need no branches;
//  * LDS rows are 64 bf16 (128 B) with an XOR swizzle (see swz) that keeps
//    both the 1-KB direct loads and the 16-byte fragment reads free of bank
//    conflicts;
//  * MFMA operands are swapped (the weight tile feeds the A operand), so each
//    of a lane's 16 x 16 blocks holds 4 consecutive output columns of one
//    output row;
//  * the epilogue (per-column weight scale, bias, activation in fp32 with no
//    FMA contraction, RNE to bf16) is instantiated per activation;
//  * gate/up mode (Llama FFN): each wave's B rows are WN/2 gate rows then the
//    WN/2 up rows of the same output columns, so block j (gate) and block
//    j + TN/2 (up) of a lane hold g and u for the same (m, n), and the lane
//    writes silu(g*sg) * (u*su) directly;
//  * split-K (when the tile grid alone cannot fill the 256 CUs): workgroup
//    (split, tile) accumulates its K slice into an fp32 partial buffer and a
//    second kernel sums the partials in split order and applies the epilogue.
//  * workgroup ids are remapped so the 32 workgroups of one XCD form a
//    compact block of tiles sharing that XCD's L2 (tile_coords).
#include <atomic>
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace mj {

constexpr int kBK = 64;  // K per pipeline stage

// int8 x16 (one 16-byte word) -> 16 bf16 (exact), as two 16-byte words.
__device__ __forceinline__ void i8x16_to_bf16x16(const uint4 &q, uint4 &lo, uint4 &hi) {
  uint32_t w[4] = {q.x, q.y, q.z, q.w};
  uint32_t o[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int32_t v = (int32_t)w[i];
    const float f0 = (float)((v << 24) >> 24);
    const float f1 = (float)((v << 16) >> 24);
    const float f2 = (float)((v << 8) >> 24);
    const float f3 = (float)(v >> 24);
    o[2 * i] = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xFFFF0000u);
    o[2 * i + 1] = (__float_as_uint(f2) >> 16) | (__float_as_uint(f3) & 0xFFFF0000u);
  }
  lo = make_uint4(o[0], o[1], o[2], o[3]);
  hi = make_uint4(o[4], o[5], o[6], o[7]);
}


// LDS is 64 banks x 4 B, and a 16-byte access is served 16 lanes at a time:
// a 256-byte bank window holds two 128-byte rows, so 16 consecutive rows
// read at one logical chunk must land on 16 distinct 16-byte slots.  XOR-ing
// the chunk with (row / 2) % 8 gives the 8 even rows 8 distinct slots in the
// first half of the window and the 8 odd rows 8 in the second half.
__device__ __forceinline__ int swz(int row, int chunk) { return (chunk ^ ((row >> 1) & 7)) * 8; }

// Stores 4 consecutive output columns [nb, nb+4) of row m.
__device__ __forceinline__ void store4_bf16(const GemmNT &p, int m, int nb, const float v[4]) {
  uint16_t *dst = p.C + (size_t)m * p.ldc + nb;
  if (nb + 3 < (int)p.N && (p.ldc & 3) == 0 && ((uintptr_t)p.C & 7) == 0) {
    *(uint2 *)dst = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (nb + q < (int)p.N) dst[q] = (uint16_t)f32_to_bf16_bits(v[q]);
  }
}

// Output staging: after the K loop the LDS is free, so the finished bf16 tile
// is written there (rows padded by 8 elements) and then stored to HBM row by
// row, 16 bytes per lane: every 128-byte line of C is written by one store
// instruction.  Writing straight from the MFMA layout would build each line
// from 8 separate 16-byte stores, and with every workgroup in its epilogue at
// once those lines are evicted half-written (about 5x the output bytes).
template <int BN_OUT>
constexpr int stage_ld() { return BN_OUT + 8; }

template <int BM, int BN_OUT, int NT>
__device__ __forceinline__ void flush_tile(const GemmNT &p, const uint16_t *ct, int m0, int n0) {
  constexpr int LD = stage_ld<BN_OUT>();
  constexpr int CPR = BN_OUT / 8;               // 16-byte chunks per tile row
  constexpr int TOTAL = BM * CPR;
  const int M = (int)p.M, N = (int)p.N;
  const bool vec = (p.ldc & 7) == 0 && ((uintptr_t)p.C & 15) == 0;
#pragma unroll 4
  for (int idx = threadIdx.x; idx < TOTAL; idx += NT) {
    const int r = idx / CPR, ch = idx % CPR;
    const int m = m0 + r, n = n0 + ch * 8;
    if (m >= M || n >= N) continue;
    const uint4 v = *(const uint4 *)(ct + r * LD + ch * 8);
    uint16_t *dst = p.C + (size_t)m * p.ldc + n;
    if (vec && n + 7 < N) {
      *(uint4 *)dst = v;
    } else {
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (n + q < N) dst[q] = (uint16_t)(w[q >> 1] >> (16 * (q & 1)));
    }
  }
}

// Epilogue for one activation E: scale, bias, E, bf16 into the staging tile.
// A lane's block (i, j) holds tile row wm*WM + 16i + (lane & 15) at the 4
// columns wn*WN + 16j + 4*(lane >> 4) + q.
template <int E, int TM, int TN, int WM, int WN, int BN_OUT>
__device__ __forceinline__ void stage_tile(const GemmNT &p, const f32x4 (&acc)[TM][TN],
                                           uint16_t *ct, int n0, int wm, int wn, int lane) {
  constexpr int LD = stage_ld<BN_OUT>();
  const int N = (int)p.N;
  const bool has_s = p.scales != nullptr, has_b = p.bias != nullptr;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int nl = wn * WN + j * 16 + 4 * (lane >> 4);  // column in the tile
    float s[4], b[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n0 + nl + q < N ? n0 + nl + q : N - 1;
      s[q] = has_s ? p.scales[n] : 1.0f;
      b[q] = has_b ? p.bias[n] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int ml = wm * WM + i * 16 + (lane & 15);
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        v[q] = apply_epi_b16(E, epi_scale_bias(acc[i][j][q], s[q], b[q], has_s, has_b));
      *(uint2 *)(ct + ml * LD + nl) = make_uint2(pack_bf16x2(v[0], v[1]),
                                                 pack_bf16x2(v[2], v[3]));
    }
  }
}

// Gate/up epilogue into the staging tile: blocks j < TN/2 are the gate,
// blocks j + TN/2 the up projection of the same output columns;
// h = silu(g*sg) * (u*su) (silu_b16).
template <int TM, int TN, int WM, int WN, int BN_OUT>
__device__ __forceinline__ void stage_gateup(const GemmNT &p, const f32x4 (&acc)[TM][TN],
                                             uint16_t *ct, int n0, int wm, int wn, int lane) {
  constexpr int LD = stage_ld<BN_OUT>();
  const int N = (int)p.N;
#pragma unroll
  for (int j = 0; j < TN / 2; ++j) {
    const int nl = wn * (WN / 2) + j * 16 + 4 * (lane >> 4);
    float sg[4], su[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n0 + nl + q < N ? n0 + nl + q : N - 1;
      sg[q] = p.scales[n];
      su[q] = p.scales2[n];
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int ml = wm * WM + i * 16 + (lane & 15);
      float h[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float gv = epi_scale_bias(acc[i][j][q], sg[q], 0.0f, true, false);
        const float uv = epi_scale_bias(acc[i][j + TN / 2][q], su[q], 0.0f, true, false);
        {
#pragma clang fp contract(off)
          h[q] = silu_b16(gv) * uv;
        }
      }
      *(uint2 *)(ct + ml * LD + nl) = make_uint2(pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3]));
    }
  }
}

// Split-K: raw fp32 sums of this workgroup's K slice.  A lane's block (i, j)
// holds row 16i + (lane & 15), columns 16j + 4*(lane >> 4) + q: one 16-byte
// store covers 64 bytes of 16 rows.  When the wave's whole sub-tile lies
// inside C (N % 4 == 0), blocks j and j+1 are traded between lanes r and r+8
// of each 16-lane row (DPP row_ror:8, bank-masked to the receiving half) so
// that each store covers 128 contiguous bytes of 8 rows, whole lines.
template <int TM, int TN, int WM, int WN>
__device__ __forceinline__ void store_part8(const GemmNT &p, const f32x4 (&acc)[TM][TN], int m0,
                                            int n0, int wm, int wn, int lane, int split) {
  const int M = (int)p.M, N = (int)p.N;
  float *part = p.part + (size_t)split * M * N;
  const bool vec = (N & 3) == 0;
  if constexpr (TN % 2 == 0) {
    const int mw = m0 + wm * WM, nw = n0 + wn * WN;
    if (vec && mw + TM * 16 <= M && nw + TN * 16 <= N) {
      const int fr = lane & 15, fh = lane >> 4;
#pragma unroll
      for (int j = 0; j < TN; j += 2) {
        const int n = nw + (j + (fr >> 3)) * 16 + 4 * fh;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          float r0[4], r1[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int a = __float_as_int(acc[i][j][q]), b = __float_as_int(acc[i][j + 1][q]);
            // rows 0-7 of the block: lanes 8-15 take block j+1 of lane - 8;
            // rows 8-15: lanes 0-7 take block j of lane + 8
            r0[q] = __int_as_float(__builtin_amdgcn_update_dpp(a, b, 0x128, 0xF, 0xC, false));
            r1[q] = __int_as_float(__builtin_amdgcn_update_dpp(b, a, 0x128, 0xF, 0x3, false));
          }
          float *dst = part + (size_t)(mw + i * 16 + (fr & 7)) * N + n;
          *(float4 *)dst = make_float4(r0[0], r0[1], r0[2], r0[3]);
          *(float4 *)(dst + (size_t)8 * N) = make_float4(r1[0], r1[1], r1[2], r1[3]);
        }
      }
      return;
    }
  }
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int nb = n0 + wn * WN + j * 16 + 4 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = m0 + wm * WM + i * 16 + (lane & 15);
      if (m >= M) continue;
      float *dst = part + (size_t)m * N + nb;
      if (vec && nb + 3 < N) {
        *(float4 *)dst = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (nb + q < N) dst[q] = acc[i][j][q];
      }
    }
  }
}

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint16_t *lds_dst, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds_dst, 16, off, 0, 0, 0);
}

// IGLP asks the compiler to interleave the stage's MFMAs with its LDS reads
// and buffer loads (iglp_opt 0) instead of issuing them in source order.
// PF2 selects the K-loop pipeline for bf16 B.  Without it (and always for
// int8 B) a stage has one barrier and stage kt+1 is loaded while stage kt
// multiplies.  With it, all fragments of stage kt are read into registers
// first and an LDS-only barrier then frees the buffer for stage kt+2, so
// every load has a stage more to land (C2: 132 -> 125 us).
//
// NW is the number of waves: 8 (two per SIMD, laid out 2 x 4, each wave a
// BM/2 x BN/4 subtile) or 4 (one per SIMD, 2 x 2, each wave BM/2 x BN/2 with
// its accumulators in the accumulation registers).
//
// Fragments of v_mfma_f32_16x16x32_bf16: lane l supplies row (l & 15) of a
// 16-row block at the 8 consecutive K of logical chunk 4*ks + (l >> 4) of
// the 64-deep stage (ks = 0, 1); both operands use the same chunks, so each
// MFMA adds the products of 32 distinct K of the stage.
template <int BM, int BN, int BKIND, bool GATEUP, bool IGLP, bool PF2, int NW = 8>
__global__ __launch_bounds__(NW * 64) void gemm_nt_kernel(GemmNT p) {
  constexpr int NT = NW * 64;
  constexpr int WGM = 2, WGN = NW / 2;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int BN_OUT = GATEUP ? BN / 2 : BN;
  constexpr int A_DMA = BM / (8 * NW);                   // 1-KB loads per wave per stage
  constexpr int B_DMA = BKIND == B_BF16 ? BN / (8 * NW) : 0;
  constexpr int B_REG = BKIND == B_BF16 ? 0 : BN * 4 / NT;  // int8: 16-B chunks per thread
  static_assert(!GATEUP || TN == 4, "gate/up pairs two gate and two up blocks per wave");
  static_assert(A_DMA >= 1, "tile too small");

  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  uint16_t *As = lds;                    // [2][BM][64]
  uint16_t *Bs = lds + 2 * BM * kBK;     // [2][BN][64]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform: keeps every LDS destination of the direct loads scalar
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;

  const int M = (int)p.M, N = (int)p.N;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN_OUT - 1) / BN_OUT;
  int split, tm, tn;
  split_tile_coords(blockIdx.x, tiles_m, tiles_n, p.splits, 4, split, tm, tn);
  const int m0 = tm * BM;
  const int n0 = tn * BN_OUT;
  // this workgroup's K slice: stages [kt0, kt1); loads stop at K (edge) or at
  // the slice end, whichever is first
  const int nk_all = ((int)p.K + kBK - 1) / kBK;
  const int per = (nk_all + p.splits - 1) / p.splits;
  const int kt0 = split * per;
  const int kt1 = kt0 + per < nk_all ? kt0 + per : nk_all;
  const int K = kt1 * kBK < (int)p.K ? kt1 * kBK : (int)p.K;

  // ---- A: direct loads.  Block b = i*NW + wave covers tile rows [8b, 8b+8).
  const __amdgpu_buffer_rsrc_t rA = make_rsrc(p.A + (size_t)m0 * p.lda,
                                              ((int64_t)(M - m0) * p.lda) * 2);
  uint32_t a_off[A_DMA];
  int a_kc[A_DMA];  // logical chunk (of 8 bf16) this lane fetches
#pragma unroll
  for (int i = 0; i < A_DMA; ++i) {
    const int r = (i * NW + wave) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    a_kc[i] = c;
    a_off[i] = (m0 + r < M) ? (uint32_t)((r * p.lda + c * 8) * 2) : kOobOffset;
  }
  // ---- B
  constexpr int ESZ = BKIND == B_BF16 ? 2 : 1;
  const size_t b_base = (size_t)n0 * p.ldb * ESZ;
  const int64_t b_bytes = (int64_t)(N - n0) * p.ldb * ESZ;
  const __amdgpu_buffer_rsrc_t rB = make_rsrc((const char *)p.B + b_base, b_bytes);
  const __amdgpu_buffer_rsrc_t rB2 =
      make_rsrc((const char *)(GATEUP ? p.B2 : p.B) + b_base, b_bytes);
  auto b_src_row = [&](int r, bool &up) {  // LDS B row -> weight row (and which matrix)
    up = false;
    if (GATEUP) {
      const int w = r / WN, rr = r % WN;
      up = rr >= WN / 2;
      return n0 + w * (WN / 2) + rr % (WN / 2);
    }
    return n0 + r;
  };
  uint32_t b_off[B_DMA > 0 ? B_DMA : 1];
  int b_kc[B_DMA > 0 ? B_DMA : 1];
  bool b_up[B_DMA > 0 ? B_DMA : 1];
#pragma unroll
  for (int i = 0; i < B_DMA; ++i) {
    const int r = (i * NW + wave) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    const int n = b_src_row(r, b_up[i]);
    b_kc[i] = c;
    b_off[i] = n < N ? (uint32_t)(((size_t)(n - n0) * p.ldb + c * 8) * 2) : kOobOffset;
  }
  // int8 register path: 4 chunks of 16 per 64-wide row
  const int q_c = tid & 3, q_r = tid >> 2;
  uint32_t q_off[B_REG > 0 ? B_REG : 1];
  bool q_up[B_REG > 0 ? B_REG : 1];
#pragma unroll
  for (int i = 0; i < B_REG; ++i) {
    const int r = q_r + (NT / 4) * i;
    const int n = b_src_row(r, q_up[i]);
    q_off[i] = n < N ? (uint32_t)((size_t)(n - n0) * p.ldb + q_c * 16) : kOobOffset;
  }
  uint4 rq[B_REG > 0 ? B_REG : 1];

  auto issue_stage = [&](int k0, int buf) {
    uint16_t *as = As + buf * BM * kBK;
#pragma unroll
    for (int i = 0; i < A_DMA; ++i) {
      const bool ok = k0 + a_kc[i] * 8 < K;
      dma16(rA, as + (i * NW + wave) * 8 * kBK, ok ? a_off[i] + k0 * 2 : kOobOffset);
    }
    uint16_t *bs = Bs + buf * BN * kBK;
#pragma unroll
    for (int i = 0; i < B_DMA; ++i) {
      const bool ok = k0 + b_kc[i] * 8 < K;
      const uint32_t off = ok ? b_off[i] + k0 * 2 : kOobOffset;
      if (GATEUP && b_up[i]) dma16(rB2, bs + (i * NW + wave) * 8 * kBK, off);
      else dma16(rB, bs + (i * NW + wave) * 8 * kBK, off);
    }
#pragma unroll
    for (int i = 0; i < B_REG; ++i) {
      const bool ok = k0 + q_c * 16 < K;
      const uint32_t off = ok ? q_off[i] + k0 : kOobOffset;
      rq[i] = (GATEUP && q_up[i]) ? buffer_load16(rB2, off) : buffer_load16(rB, off);
    }
  };
  auto store_int8 = [&](int buf) {
    uint16_t *bs = Bs + buf * BN * kBK;
#pragma unroll
    for (int i = 0; i < B_REG; ++i) {
      const int r = q_r + (NT / 4) * i;
      uint4 lo, hi;
      i8x16_to_bf16x16(rq[i], lo, hi);
      *(uint4 *)(bs + r * kBK + swz(r, 2 * q_c)) = lo;
      *(uint4 *)(bs + r * kBK + swz(r, 2 * q_c + 1)) = hi;
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int fr = lane & 15;       // row within a 16-row block
  const int fh = lane >> 4;       // K chunk within a 32-deep MFMA step
  const int sw = (fr >> 1) & 7;   // the row's swizzle (blocks start at multiples of 16)
  constexpr int KS = kBK / 32;    // MFMA steps per stage

  if constexpr (PF2) {
    static_assert(B_REG == 0, "PF2 takes bf16 B only");
    constexpr int NDMA = A_DMA + B_DMA;  // direct loads per lane per stage
    static_assert(NDMA < 64, "vmcnt range");
    issue_stage(kt0 * kBK, 0);
    issue_stage((kt0 + 1) * kBK, 1);  // past K (or the slice) it reads zeros
    __builtin_amdgcn_s_waitcnt(0x0F70 | (NDMA & 0xF) | ((NDMA >> 4) << 14));  // stage kt0 landed
    asm volatile("s_barrier" ::: "memory");
    for (int kt = kt0; kt < kt1; ++kt) {
      const int buf = (kt - kt0) & 1;
      const uint16_t *as = As + buf * BM * kBK + (wm * WM + fr) * kBK;
      const uint16_t *bs = Bs + buf * BN * kBK + (wn * WN + fr) * kBK;
      bf16x8 fa[KS][TM], fb[KS][TN];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int col = ((ks * 4 + fh) ^ sw) * 8;
#pragma unroll
        for (int i = 0; i < TM; ++i) fa[ks][i] = *(const bf16x8 *)(as + i * 16 * kBK + col);
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[ks][j] = *(const bf16x8 *)(bs + j * 16 * kBK + col);
      }
      // every wave has its fragments of this buffer in registers: free it
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      issue_stage((kt + 2) * kBK, buf);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[ks][j], fa[ks][i], acc[i][j],
                                                                0, 0, 0);
      if constexpr (IGLP) __builtin_amdgcn_iglp_opt(0);
      __builtin_amdgcn_sched_barrier(0);
      // stage kt+1 (issued one stage earlier) has landed in every wave
      __builtin_amdgcn_s_waitcnt(0x0F70 | (NDMA & 0xF) | ((NDMA >> 4) << 14));
      asm volatile("s_barrier" ::: "memory");
    }
    // the zero-filled loads of stages kt1, kt1+1 may still be in flight: they
    // target LDS that the epilogue reuses, so drain them first
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
  } else {
  issue_stage(kt0 * kBK, 0);
  if constexpr (B_REG > 0) store_int8(0);
  __syncthreads();

  for (int kt = kt0; kt < kt1; ++kt) {
    const int buf = (kt - kt0) & 1;
    // the other buffer was last read in stage kt-1, which every wave finished
    // before the barrier that ended it
    issue_stage((kt + 1) * kBK, buf ^ 1);
    const uint16_t *as = As + buf * BM * kBK + (wm * WM + fr) * kBK;
    const uint16_t *bs = Bs + buf * BN * kBK + (wn * WN + fr) * kBK;
    bf16x8 fa[2][TM], fb[2][TN];
    auto read_frags = [&](int slot, int ks) {
      const int col = ((ks * 4 + fh) ^ sw) * 8;
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[slot][i] = *(const bf16x8 *)(as + i * 16 * kBK + col);
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[slot][j] = *(const bf16x8 *)(bs + j * 16 * kBK + col);
    };
    read_frags(0, 0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) read_frags((ks + 1) & 1, ks + 1);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[ks & 1][j], fa[ks & 1][i],
                                                              acc[i][j], 0, 0, 0);
    }
    if constexpr (B_REG > 0) store_int8(buf ^ 1);
    if constexpr (IGLP) __builtin_amdgcn_iglp_opt(0);
    // the direct loads of stage kt+1 must have landed in LDS before anyone
    // reads them: wait for this wave's loads, then the barrier covers all
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
  }
  }

  if (p.part != nullptr) {
    if constexpr (!GATEUP) store_part8<TM, TN, WM, WN>(p, acc, m0, n0, wm, wn, lane, split);
    return;
  }
  // every wave has left the K loop (its last barrier), so the LDS is free
  uint16_t *ct = lds;
  if constexpr (!GATEUP) {
    switch (p.epi) {
#define MJ_STAGE(E) stage_tile<E, TM, TN, WM, WN, BN_OUT>(p, acc, ct, n0, wm, wn, lane); break;
      case EPI_RELU: MJ_STAGE(EPI_RELU)
      case EPI_GELU_TANH: MJ_STAGE(EPI_GELU_TANH)
      case EPI_SILU: MJ_STAGE(EPI_SILU)
      case EPI_GELU_TANH_APPROX: MJ_STAGE(EPI_GELU_TANH_APPROX)
      case EPI_SILU_APPROX: MJ_STAGE(EPI_SILU_APPROX)
      case EPI_RELU_UNARY: MJ_STAGE(EPI_RELU_UNARY)
      default: MJ_STAGE(EPI_NONE)
#undef MJ_STAGE
    }
  } else {
    stage_gateup<TM, TN, WM, WN, BN_OUT>(p, acc, ct, n0, wm, wn, lane);
  }
  __syncthreads();
  flush_tile<BM, BN_OUT, NT>(p, ct, m0, n0);
}

// ---------------------------------------------------------------------------
// The tile kernels below (bf16 256 x 256 with two waves per SIMD; W8A16 and
// int8 with one) share one pipeline:
//
//  * the accumulators are written by inline-asm MFMAs with the accumulator
//    tied ("+a", D = C) so that every block stays in fixed registers (the
//    compiler, left to itself at this pressure, rotates blocks through
//    temporaries every iteration).  Inline asm is opaque to the hazard
//    recognizer, so the two places where other code touches the accumulators
//    (the zero fill before the K loop and the epilogue's reads after it) are
//    separated from the MFMAs by explicit s_nop cover; inside the loop each
//    block is reused only after the rest of its step;
//  * K advances 64 per stage through 128-byte LDS rows (the XOR swizzle of
//    swz()): 2 buffers for A and 3 for B; every direct load fetches 128-byte
//    row segments, half as many L2 requests as 32-deep stages would need;
//  * each stage is two 32-deep MFMA steps, each step one group of MFMAs per
//    B block with the step's fragment reads for the next step spread over
//    the first groups and one direct load per group.  The stage's one
//    barrier sits between its two steps: there every wave holds the stage's
//    fragments, so the stage's A buffer is free and the A loads of stage kt+2
//    go into it during the second step; the third B buffer (stage kt-1's,
//    free since the previous barrier) takes the B loads of stage kt+2 during
//    the first step.  Loads spread over both steps: 16 in one step left the
//    address unit unable to keep up, stalling the wave's MFMA issue;
//  * the K advance of a load is its scalar offset (no per-load VALU); the
//    last stages, whose loads reach past K, take a per-load zero-fill select.
//    The scalar offset stays below 2^31 and an out-of-range row offset plus it
//    cannot wrap for K < 2^30, which the launchers check.
__device__ __forceinline__ void dma16s(__amdgpu_buffer_rsrc_t r, uint16_t *lds_dst,
                                       uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds_dst, 16, voff, soff, 0, 0);
}

// Epilogue of a full, 16-byte aligned tile straight from the accumulators:
// blocks j and j+1 of a lane row are exchanged with v_permlane16_swap so that
// each lane holds 8 consecutive output columns (lane row 0: block j columns
// 0-7, row 1: block j+1 columns 0-7, row 2: block j columns 8-15, row 3:
// block j+1 columns 8-15) and writes them with one 16-byte store; each store
// instruction covers 64 contiguous bytes of 16 output rows.  The stores of
// one row block i go out back to back (j pairs inner), so both halves of a
// 128-byte line of C reach the L2 together: with the j pairs outer the line
// was often written back half full, 1.6 us more per 4096 x 4096 bf16 output
// (MI355X).  SCALES = false: a bf16 B (no per-channel scales; p.scales is
// not read).
template <int E, int TM, int TN, int WM, int WN, bool SCALES = true>
__device__ __forceinline__ void store_tile_direct(const GemmNT &p, const f32x4 (&acc)[TM][TN],
                                                  int m0, int n0, int wm, int wn, int lane) {
  const int fr = lane & 15, fh = lane >> 4;
  const bool has_s = SCALES && p.scales != nullptr, has_b = p.bias != nullptr;
  float s[TN][4], b[TN][4];
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n0 + wn * WN + j * 16 + 4 * fh + q;
      s[j][q] = has_s ? p.scales[n] : 1.0f;
      b[j][q] = has_b ? p.bias[n] : 0.0f;
    }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j + 1 < TN; j += 2) {
      float x[4], y[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        x[q] = apply_epi_b16(E, epi_scale_bias(acc[i][j][q], s[j][q], b[j][q], has_s, has_b));
        y[q] = apply_epi_b16(E, epi_scale_bias(acc[i][j + 1][q], s[j + 1][q], b[j + 1][q],
                                               has_s, has_b));
      }
      const auto w0 = __builtin_amdgcn_permlane16_swap(pack_bf16x2(x[0], x[1]),
                                                       pack_bf16x2(y[0], y[1]), false, false);
      const auto w1 = __builtin_amdgcn_permlane16_swap(pack_bf16x2(x[2], x[3]),
                                                       pack_bf16x2(y[2], y[3]), false, false);
      const int m = m0 + wm * WM + i * 16 + fr;
      const int n = n0 + wn * WN + (j + (fh & 1)) * 16 + 8 * (fh >> 1);
      *(uint4 *)(p.C + (size_t)m * p.ldc + n) = make_uint4(w0[0], w1[0], w0[1], w1[1]);
    }
    if constexpr (TN % 2 == 1) {
      // an odd last block: its 4 columns per lane as one 8-byte store
      float x[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        x[q] = apply_epi_b16(E, epi_scale_bias(acc[i][TN - 1][q], s[TN - 1][q], b[TN - 1][q],
                                               has_s, has_b));
      const int m = m0 + wm * WM + i * 16 + fr;
      const int n = n0 + wn * WN + (TN - 1) * 16 + 4 * fh;
      *(uint2 *)(p.C + (size_t)m * p.ldc + n) = make_uint2(pack_bf16x2(x[0], x[1]),
                                                           pack_bf16x2(x[2], x[3]));
    }
  }
}

// s_waitcnt lgkmcnt(0) as the builtin (vmcnt and expcnt left open): unlike the
// same text in inline asm, the compiler's wait-count pass sees it, so it does
// not add a wait of its own for fragments this one already covered (such a
// wait, placed after the next step's first read, stalled every stage for a
// full LDS round trip).
constexpr int kLgkm0 = 0xC07F;

__device__ __forceinline__ void mfma_16x16x32_tied(f32x4 &acc, const bf16x8 &a, const bf16x8 &b) {
  asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// bf16 256 x 256 tiles with two waves per SIMD: 8 waves laid out 2 x 4, each
// owning 128 x 64 outputs (128 accumulator registers, so two waves fit a
// SIMD), on the pipeline above (the 12 fragment reads of a step 3 per group,
// one direct load per group).  A fragment read holds its wave's instruction
// issue for about half an MFMA's 16 cycles; with one wave per SIMD (4 waves
// of 128 x 128, the fewest reads per flop) the 16 reads of a step delayed its
// 64 MFMAs by ~12 %, with two the other wave issues MFMAs meanwhile: 5 %
// faster at 4096^3 in spite of 1.5x the reads per flop (MI355X, bit-identical
// outputs).
__global__ __launch_bounds__(512) void gemm_nt_w8_kernel(GemmNT p) {
  constexpr int BM = 256, BN = 256, NT = 512;
  constexpr int WM = 128, WN = 64, TM = 8, TN = 4;
  constexpr int DPO = 4;  // 1-KB direct loads per wave per operand per stage
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  uint16_t *As = lds;                    // [2][BM][64]: stage kt in buffer kt % 2
  uint16_t *Bs = lds + 2 * BM * kBK;     // [3][BN][64]: stage kt in buffer kt % 3

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int M = (int)p.M, N = (int)p.N, K = (int)p.K;
  int tm, tn;
  tile_coords(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, 4, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int nk = (K + kBK - 1) / kBK;

  const __amdgpu_buffer_rsrc_t rA = make_rsrc(p.A + (size_t)m0 * p.lda,
                                              ((int64_t)(M - m0) * p.lda) * 2);
  const __amdgpu_buffer_rsrc_t rB = make_rsrc((const uint16_t *)p.B + (size_t)n0 * p.ldb,
                                              ((int64_t)(N - n0) * p.ldb) * 2);
  // 1-KB block b = i*8 + wave covers tile rows [8b, 8b+8)
  uint32_t a_off[DPO], b_off[DPO];
  int kc[DPO];
#pragma unroll
  for (int i = 0; i < DPO; ++i) {
    const int r = (i * 8 + wave) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    kc[i] = c;
    a_off[i] = m0 + r < M ? (uint32_t)((r * p.lda + c * 8) * 2) : kOobOffset;
    b_off[i] = n0 + r < N ? (uint32_t)((r * p.ldb + c * 8) * 2) : kOobOffset;
  }
  // direct load d of stage kt: d < 4 is A block d, else B block d - 4
  auto load = [&](auto fast, int kt, int buf, int d) {
    const int k0 = kt * kBK;
    const int i = d & 3;
    uint16_t *dst = (d < 4 ? As : Bs) + buf * BM * kBK + (i * 8 + wave) * 8 * kBK;
    const __amdgpu_buffer_rsrc_t r = d < 4 ? rA : rB;
    const uint32_t off = d < 4 ? a_off[i] : b_off[i];
    if constexpr (decltype(fast)::value) {
      dma16s(r, dst, off, (uint32_t)(k0 * 2));
    } else {
      const bool ok = k0 + kc[i] * 8 < K;
      dma16s(r, dst, ok ? off + k0 * 2 : kOobOffset, 0u);
    }
  };

  const int fr = lane & 15, fh = lane >> 4;
  const int sw = (fr >> 1) & 7;
  const uint16_t *a_rd[2], *b_rd[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int col = ((ks * 4 + fh) ^ sw) * 8;
    a_rd[ks] = As + (wm * WM + fr) * kBK + col;
    b_rd[ks] = Bs + (wn * WN + fr) * kBK + col;
  }

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  bf16x8 fa[2][TM], fb[2][TN];

#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int d = 0; d < 2 * DPO; ++d) load(std::false_type(), s, s, d);
  __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * DPO));  // stage 0
  asm volatile("s_barrier" ::: "memory");
#pragma unroll
  for (int i = 0; i < TM; ++i) fa[0][i] = *(const bf16x8 *)(a_rd[0] + i * 16 * kBK);
#pragma unroll
  for (int j = 0; j < TN; ++j) fb[0][j] = *(const bf16x8 *)(b_rd[0] + j * 16 * kBK);
  __builtin_amdgcn_s_waitcnt(kLgkm0);
  asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");  // zero fill -> first MFMAs

  auto stage = [&](auto ab_c, auto bb_c, auto fast, int kt) {
    constexpr int AB = decltype(ab_c)::value;
    constexpr int BB = decltype(bb_c)::value;
    // the 12 fragment reads of a step (read t < 8: A block t, else B block
    // t - 8) go 3 per group into groups 0-3
    auto read_frag = [&](int t, int dst, int abuf, int bbuf) {
      if (t < 8) fa[dst][t] = *(const bf16x8 *)(a_rd[dst] + abuf * BM * kBK + t * 16 * kBK);
      else fb[dst][t - 8] = *(const bf16x8 *)(b_rd[dst] + bbuf * BN * kBK + (t - 8) * 16 * kBK);
    };
    auto group = [&](int j, int src, int dst, int abuf, int bbuf, int load_d, int load_buf) {
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        __builtin_amdgcn_sched_barrier(0);
        read_frag(3 * j + u, dst, abuf, bbuf);
        __builtin_amdgcn_sched_barrier(0);
        mfma_16x16x32_tied(acc[u][j], fb[src][j], fa[src][u]);
      }
      __builtin_amdgcn_sched_barrier(0);
      load(fast, kt + 2, load_buf, load_d);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 3; i < TM; ++i) mfma_16x16x32_tied(acc[i][j], fb[src][j], fa[src][i]);
    };
    // step 0; B loads of stage kt+2 into B buffer (BB + 2) % 3
#pragma unroll
    for (int j = 0; j < TN; ++j) group(j, 0, 1, AB, BB, DPO + j, (BB + 2) % 3);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kLgkm0);
    __builtin_amdgcn_s_waitcnt(0x0F70 | DPO);  // vmcnt(DPO): all but this step's B loads
    asm volatile("s_barrier" ::: "memory");
    // step 1; A loads of stage kt+2 into A buffer AB
#pragma unroll
    for (int j = 0; j < TN; ++j) group(j, 1, 0, AB ^ 1, (BB + 1) % 3, j, AB);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kLgkm0);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using F = std::true_type;
  using S = std::false_type;
  const int nk_full = K / kBK;
  int kt = 0;
  for (; kt + 8 <= nk_full; kt += 6) {
    stage(I0(), I0(), F(), kt);
    stage(I1(), I1(), F(), kt + 1);
    stage(I0(), I2(), F(), kt + 2);
    stage(I1(), I0(), F(), kt + 3);
    stage(I0(), I1(), F(), kt + 4);
    stage(I1(), I2(), F(), kt + 5);
  }
  for (; kt < nk; kt += 6) {
    stage(I0(), I0(), S(), kt);
    if (kt + 1 < nk) stage(I1(), I1(), S(), kt + 1);
    if (kt + 2 < nk) stage(I0(), I2(), S(), kt + 2);
    if (kt + 3 < nk) stage(I1(), I0(), S(), kt + 3);
    if (kt + 4 < nk) stage(I0(), I1(), S(), kt + 4);
    if (kt + 5 < nk) stage(I1(), I2(), S(), kt + 5);
  }
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();

  if (m0 + BM <= M && n0 + BN <= N && (p.ldc & 7) == 0 && ((uintptr_t)p.C & 15) == 0) {
    switch (p.epi) {
#define MJ_DIRECT(E) store_tile_direct<E, TM, TN, WM, WN, false>(p, acc, m0, n0, wm, wn, lane); break;
      case EPI_RELU: MJ_DIRECT(EPI_RELU)
      case EPI_GELU_TANH: MJ_DIRECT(EPI_GELU_TANH)
      case EPI_SILU: MJ_DIRECT(EPI_SILU)
      case EPI_GELU_TANH_APPROX: MJ_DIRECT(EPI_GELU_TANH_APPROX)
      case EPI_SILU_APPROX: MJ_DIRECT(EPI_SILU_APPROX)
      case EPI_RELU_UNARY: MJ_DIRECT(EPI_RELU_UNARY)
      default: MJ_DIRECT(EPI_NONE)
#undef MJ_DIRECT
    }
    return;
  }
  uint16_t *ct = lds;
  switch (p.epi) {
#define MJ_STAGE(E) stage_tile<E, TM, TN, WM, WN, BN>(p, acc, ct, n0, wm, wn, lane); break;
    case EPI_RELU: MJ_STAGE(EPI_RELU)
    case EPI_GELU_TANH: MJ_STAGE(EPI_GELU_TANH)
    case EPI_SILU: MJ_STAGE(EPI_SILU)
    case EPI_GELU_TANH_APPROX: MJ_STAGE(EPI_GELU_TANH_APPROX)
    case EPI_SILU_APPROX: MJ_STAGE(EPI_SILU_APPROX)
    case EPI_RELU_UNARY: MJ_STAGE(EPI_RELU_UNARY)
    default: MJ_STAGE(EPI_NONE)
#undef MJ_STAGE
  }
  __syncthreads();
  flush_tile<BM, BN, NT>(p, ct, m0, n0);
}

static hipError_t launch_w8(const GemmNT &p, hipStream_t stream) {
  constexpr size_t lds_loop = size_t(2 * 256 + 3 * 256) * kBK * sizeof(uint16_t);  // 160 KB
  constexpr size_t lds_out = size_t(256) * stage_ld<256>() * sizeof(uint16_t);
  constexpr size_t lds = lds_loop > lds_out ? lds_loop : lds_out;
  if (p.K >= ((int64_t)1 << 30) || p.bkind != B_BF16 || p.gate_up || p.splits != 1 ||
      256 * p.lda * 2 >= ((int64_t)1 << 31) || 256 * p.ldb * 2 >= ((int64_t)1 << 31))
    return hipErrorInvalidValue;
  static std::atomic<uint64_t> attr_set{0};
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
  const uint64_t bit = dev < 64 ? (uint64_t)1 << dev : 0;
  if (!bit || !(attr_set.load(std::memory_order_acquire) & bit)) {
    hipError_t e = hipFuncSetAttribute((const void *)gemm_nt_w8_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set.fetch_or(bit, std::memory_order_release);
  }
  const int64_t grid = ((p.M + 255) / 256) * ((p.N + 255) / 256);
  if (grid > INT32_MAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL(gemm_nt_w8_kernel, dim3((unsigned)grid), dim3(512), lds, stream, p);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// int8 x int8 -> int32 on 256 x BN tiles (BN = 256 or 128) with one wave per
// SIMD: matmul_i8_i8_to_i32 (learn/api/functional.mojo:249-279), QuantLinear's
// dequantize (learn/nn/layers.mojo:1681-1685, functional.mojo:281-302) fused
// into the epilogue, and the W8A8 Linear with per-row activation and
// per-channel weight scales, for problems large enough to fill the CUs.  It is
// the bf16 tile pipeline on int8 data: a 128-deep int8 stage is 128
// bytes per row, the same LDS bytes as a 64-deep bf16 stage, so the buffers,
// the XOR swizzle, the direct loads and the fragment reads are byte for byte
// the same; a lane's 16-byte fragment of a 64-deep step is the 16 consecutive
// k at 16 (lane / 16) of its row, which is the operand layout of
// v_mfma_i32_16x16x64_i8 (16 x 16 x 64 per instruction, twice the work of the
// bf16 16 x 16 x 32 in the same issue slot).  Integer sums are exact, so the
// sums are the reference's in any order.  BN = 128 (waves of 128 x 64) gives
// twice the workgroups where 256 x 256 tiles would leave CUs idle; its step 1
// issues two A loads per MFMA group instead of one.
//
// Epilogue (MODE): 0 = the int32 sums C[m, n]; 1 = QuantLinear's
// y[m, n] = float(acc) * sf + b[n] in fp32; 2 = the W8A8 Linear's
// y[m, n] = bf16(epi(float(acc) * (sx[m] * sw[n]) + b[n])) (no FMA contraction
// in either; epi as the bf16-output epilogues of the W8A16 kernels).
struct GemmI8 {
  const int8_t *A = nullptr;  // [M, K], leading dimension lda
  int64_t lda = 0;
  const int8_t *B = nullptr;  // [N, K] (the stored w_q layout), leading dimension ldb
  int64_t ldb = 0;
  int32_t *C = nullptr;       // MODE 0: [M, N] int32, leading dimension ldc
  float *Y = nullptr;         // MODE 1: [M, N] fp32, leading dimension ldc
  uint16_t *Yb = nullptr;     // MODE 2: [M, N] bf16, leading dimension ldc
  int64_t ldc = 0;
  float sf = 1.0f;            // MODE 1: s_x * s_w
  const float *sx = nullptr;  // MODE 2: per-row activation scales [M]
  const float *sw = nullptr;  // MODE 2: per-channel weight scales [N]
  const float *bias = nullptr;  // MODES 1, 2: [N] (may be null in MODE 2)
  int epi = 0;                // MODE 2
  int64_t M = 0, N = 0, K = 0;
};

__device__ __forceinline__ void mfma_i8_16x16x64_tied(i32x4 &acc, const bf16x8 &a,
                                                      const bf16x8 &b) {
  asm("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// MODE 2 epilogue for activation E: a lane's block (i, j) holds output row
// m0 + wm*128 + 16 i + (lane & 15) at the 4 columns nb_j .. nb_j + 3.
template <int E, int TM, int TN, int WN>
__device__ __forceinline__ void store_w8a8(const GemmI8 &p, const i32x4 (&acc)[TM][TN], int m0,
                                           int n0, int wm, int wn, int lane) {
  const int M = (int)p.M, N = (int)p.N;
  const int fr = lane & 15, fh = lane >> 4;
  const bool vec = (p.ldc & 3) == 0 && ((uintptr_t)p.Yb & 7) == 0;
  float sxm[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm * 128 + i * 16 + fr;
    sxm[i] = p.sx[m < M ? m : M - 1];
  }
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int nb = n0 + wn * WN + j * 16 + 4 * fh;
    float swq[4], bq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = nb + q < N ? nb + q : N - 1;
      swq[q] = p.sw[n];
      bq[q] = p.bias ? p.bias[n] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = m0 + wm * 128 + i * 16 + fr;
      if (m >= M) continue;
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float t;
        {
#pragma clang fp contract(off)
          const float sf = sxm[i] * swq[q];
          t = (float)acc[i][j][q] * sf;
          if (p.bias) t = t + bq[q];
        }
        v[q] = apply_epi_b16(E, t);
      }
      uint16_t *dst = p.Yb + (size_t)m * p.ldc + nb;
      if (vec && nb + 3 < N) {
        *(uint2 *)dst = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (nb + q < N) dst[q] = (uint16_t)f32_to_bf16_bits(v[q]);
      }
    }
  }
}

// The W8A8 epilogue for a tile wholly inside the output with 16-byte aligned
// rows: the values of store_w8a8 (same operations, same order), with blocks
// j, j+1 exchanged through v_permlane16_swap so each lane stores 8
// consecutive bf16 columns in one 16-byte store, the j pairs inner so both
// halves of a 128-byte output line are written together (as
// store_tile_direct does for the W8A16 kernels).
template <int E, int TM, int TN, int WN>
__device__ __forceinline__ void store_w8a8_direct(const GemmI8 &p, const i32x4 (&acc)[TM][TN],
                                                  int m0, int n0, int wm, int wn, int lane) {
  static_assert(TN % 2 == 0, "column blocks in pairs");
  const int fr = lane & 15, fh = lane >> 4;
  const bool has_b = p.bias != nullptr;
  float swq[TN][4], bq[TN][4];
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n0 + wn * WN + j * 16 + 4 * fh + q;
      swq[j][q] = p.sw[n];
      bq[j][q] = has_b ? p.bias[n] : 0.0f;
    }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm * 128 + i * 16 + fr;
    const float sxm = p.sx[m];
#pragma unroll
    for (int j = 0; j < TN; j += 2) {
      float x[4], y[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float t0, t1;
        {
#pragma clang fp contract(off)
          const float sf0 = sxm * swq[j][q], sf1 = sxm * swq[j + 1][q];
          t0 = (float)acc[i][j][q] * sf0;
          t1 = (float)acc[i][j + 1][q] * sf1;
          if (has_b) {
            t0 = t0 + bq[j][q];
            t1 = t1 + bq[j + 1][q];
          }
        }
        x[q] = apply_epi_b16(E, t0);
        y[q] = apply_epi_b16(E, t1);
      }
      const auto w0 = __builtin_amdgcn_permlane16_swap(pack_bf16x2(x[0], x[1]),
                                                       pack_bf16x2(y[0], y[1]), false, false);
      const auto w1 = __builtin_amdgcn_permlane16_swap(pack_bf16x2(x[2], x[3]),
                                                       pack_bf16x2(y[2], y[3]), false, false);
      const int n = n0 + wn * WN + (j + (fh & 1)) * 16 + 8 * (fh >> 1);
      *(uint4 *)(p.Yb + (size_t)m * p.ldc + n) = make_uint4(w0[0], w1[0], w0[1], w1[1]);
    }
  }
}

template <int BN, int MODE>
__global__ __launch_bounds__(256) void gemm_i8_w4_kernel(GemmI8 p) {
  constexpr int BM = 256;
  constexpr int WM = 128, WN = BN / 2, TM = 8, TN = WN / 16;
  constexpr int DPA = 8;       // 1-KB direct loads of A per wave per stage
  constexpr int DPB = BN / 32;  // of B
  constexpr int A_PER_GROUP = DPA / TN;  // A loads per MFMA group of step 1
  constexpr int KS = 128;      // int8 k per stage (128 bytes per row, as kBK bf16)
  static_assert(BN == 128 || BN == 256, "tile width");
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  uint16_t *As = lds;                    // [2][BM][128 B]: stage kt in buffer kt % 2
  uint16_t *Bs = lds + 2 * BM * kBK;     // [3][BN][128 B]: stage kt in buffer kt % 3

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int M = (int)p.M, N = (int)p.N, K = (int)p.K;
  int tm, tn;
  tile_coords(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, 4, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int nk = (K + KS - 1) / KS;

  const __amdgpu_buffer_rsrc_t rA = make_rsrc(p.A + (size_t)m0 * p.lda, (int64_t)(M - m0) * p.lda);
  const __amdgpu_buffer_rsrc_t rB = make_rsrc(p.B + (size_t)n0 * p.ldb, (int64_t)(N - n0) * p.ldb);
  // 1-KB block b = i*4 + wave covers tile rows [8b, 8b+8): row 8b + lane/8,
  // stored chunk lane%8, which holds logical 16-byte chunk c of the row
  uint32_t a_off[DPA], b_off[DPB];
  int kc[DPA];
#pragma unroll
  for (int i = 0; i < DPA; ++i) {
    const int r = (i * 4 + wave) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    kc[i] = c;
    a_off[i] = m0 + r < M ? (uint32_t)(r * p.lda + c * 16) : kOobOffset;
    if (i < DPB) b_off[i] = n0 + r < N ? (uint32_t)(r * p.ldb + c * 16) : kOobOffset;
  }
  // direct load d of stage kt into buffer buf: d < 8 is A block d, else B
  // block d - 8 (< DPB)
  auto load = [&](auto fast, int kt, int buf, int d) {
    const int k0 = kt * KS;
    const int i = d & 7;
    uint16_t *dst = d < 8 ? As + buf * BM * kBK + (i * 4 + wave) * 8 * kBK
                          : Bs + buf * BN * kBK + (i * 4 + wave) * 8 * kBK;
    const __amdgpu_buffer_rsrc_t r = d < 8 ? rA : rB;
    const uint32_t off = d < 8 ? a_off[i] : b_off[i];
    if constexpr (decltype(fast)::value) {
      dma16s(r, dst, off, (uint32_t)k0);
    } else {
      const bool ok = k0 + kc[i] * 16 < K;
      dma16s(r, dst, ok ? off + k0 : kOobOffset, 0u);
    }
  };

  const int fr = lane & 15, fh = lane >> 4;
  const int sw = (fr >> 1) & 7;
  const uint16_t *a_rd[2], *b_rd[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int col = ((ks * 4 + fh) ^ sw) * 8;
    a_rd[ks] = As + (wm * WM + fr) * kBK + col;
    b_rd[ks] = Bs + (wn * WN + fr) * kBK + col;
  }

  i32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = i32x4{0, 0, 0, 0};
  bf16x8 fa[2][TM], fb[2][TN];

#pragma unroll
  for (int s = 0; s < 2; ++s) {
#pragma unroll
    for (int d = 0; d < DPA; ++d) load(std::false_type(), s, s, d);
#pragma unroll
    for (int d = 0; d < DPB; ++d) load(std::false_type(), s, s, 8 + d);
  }
  constexpr int kStage = DPA + DPB;  // loads per stage: wait for stage 0
  __builtin_amdgcn_s_waitcnt(0x0F70 | (kStage & 0xF) | ((kStage >> 4) << 14));
  asm volatile("s_barrier" ::: "memory");
#pragma unroll
  for (int i = 0; i < TM; ++i) fa[0][i] = *(const bf16x8 *)(a_rd[0] + i * 16 * kBK);
#pragma unroll
  for (int j = 0; j < TN; ++j) fb[0][j] = *(const bf16x8 *)(b_rd[0] + j * 16 * kBK);
  __builtin_amdgcn_s_waitcnt(kLgkm0);
  asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");  // zero fill -> first MFMAs

  auto stage = [&](auto ab_c, auto bb_c, auto fast, int kt) {
    constexpr int AB = decltype(ab_c)::value;
    constexpr int BB = decltype(bb_c)::value;
    // read t < 8: A block t, else B block t - 8
    auto read_frag = [&](int t, int dst, int abuf, int bbuf) {
      if (t < 8) fa[dst][t] = *(const bf16x8 *)(a_rd[dst] + abuf * BM * kBK + t * 16 * kBK);
      else fb[dst][t - 8] = *(const bf16x8 *)(b_rd[dst] + bbuf * BN * kBK + (t - 8) * 16 * kBK);
    };
    // the 8 + TN fragment reads of a step go 3 per group into groups 0-3,
    // then (TN = 8) 2, 2 into groups 4-5; a group's loads go after its third
    // MFMA and (a second one) after its sixth
    auto group = [&](int j, int src, int dst, int abuf, int bbuf, int load_d, int nld,
                     int load_buf) {
      const int t0 = j < 4 ? 3 * j : 12 + 2 * (j - 4);
      const int nt = j < 4 ? 3 : (j < 6 ? 2 : 0);
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        __builtin_amdgcn_sched_barrier(0);
        if (u < nt) read_frag(t0 + u, dst, abuf, bbuf);
        __builtin_amdgcn_sched_barrier(0);
        mfma_i8_16x16x64_tied(acc[u][j], fb[src][j], fa[src][u]);
      }
      __builtin_amdgcn_sched_barrier(0);
      load(fast, kt + 2, load_buf, load_d);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 3; i < TM; ++i) {
        mfma_i8_16x16x64_tied(acc[i][j], fb[src][j], fa[src][i]);
        if (i == 5 && nld > 1) {
          __builtin_amdgcn_sched_barrier(0);
          load(fast, kt + 2, load_buf, load_d + 1);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };
    // step 0; B loads of stage kt+2 into B buffer (BB + 2) % 3
#pragma unroll
    for (int j = 0; j < TN; ++j) group(j, 0, 1, AB, BB, 8 + j, 1, (BB + 2) % 3);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kLgkm0);
    __builtin_amdgcn_s_waitcnt(0x0F70 | DPB);  // vmcnt(DPB): all but this step's B loads
    asm volatile("s_barrier" ::: "memory");
    // step 1; A loads of stage kt+2 into A buffer AB
#pragma unroll
    for (int j = 0; j < TN; ++j)
      group(j, 1, 0, AB ^ 1, (BB + 1) % 3, A_PER_GROUP * j, A_PER_GROUP, AB);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kLgkm0);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using F = std::true_type;
  using S = std::false_type;
  const int nk_full = K / KS;
  int kt = 0;
  for (; kt + 8 <= nk_full; kt += 6) {
    stage(I0(), I0(), F(), kt);
    stage(I1(), I1(), F(), kt + 1);
    stage(I0(), I2(), F(), kt + 2);
    stage(I1(), I0(), F(), kt + 3);
    stage(I0(), I1(), F(), kt + 4);
    stage(I1(), I2(), F(), kt + 5);
  }
  for (; kt < nk; kt += 6) {
    stage(I0(), I0(), S(), kt);
    if (kt + 1 < nk) stage(I1(), I1(), S(), kt + 1);
    if (kt + 2 < nk) stage(I0(), I2(), S(), kt + 2);
    if (kt + 3 < nk) stage(I1(), I0(), S(), kt + 3);
    if (kt + 4 < nk) stage(I0(), I1(), S(), kt + 4);
    if (kt + 5 < nk) stage(I1(), I2(), S(), kt + 5);
  }
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();

  if constexpr (MODE == 2) {
    const bool full = m0 + BM <= M && n0 + BN <= N && (p.ldc & 7) == 0 &&
                      ((uintptr_t)p.Yb & 15) == 0;
    if (full) {
      switch (p.epi) {
#define MJ_W8A8D(E) store_w8a8_direct<E, TM, TN, WN>(p, acc, m0, n0, wm, wn, lane); break;
        case EPI_RELU: MJ_W8A8D(EPI_RELU)
        case EPI_GELU_TANH: MJ_W8A8D(EPI_GELU_TANH)
        case EPI_SILU: MJ_W8A8D(EPI_SILU)
        case EPI_GELU_TANH_APPROX: MJ_W8A8D(EPI_GELU_TANH_APPROX)
        case EPI_SILU_APPROX: MJ_W8A8D(EPI_SILU_APPROX)
        case EPI_RELU_UNARY: MJ_W8A8D(EPI_RELU_UNARY)
        default: MJ_W8A8D(EPI_NONE)
#undef MJ_W8A8D
      }
      return;
    }
    switch (p.epi) {
#define MJ_W8A8(E) store_w8a8<E, TM, TN, WN>(p, acc, m0, n0, wm, wn, lane); break;
      case EPI_RELU: MJ_W8A8(EPI_RELU)
      case EPI_GELU_TANH: MJ_W8A8(EPI_GELU_TANH)
      case EPI_SILU: MJ_W8A8(EPI_SILU)
      case EPI_GELU_TANH_APPROX: MJ_W8A8(EPI_GELU_TANH_APPROX)
      case EPI_SILU_APPROX: MJ_W8A8(EPI_SILU_APPROX)
      case EPI_RELU_UNARY: MJ_W8A8(EPI_RELU_UNARY)
      default: MJ_W8A8(EPI_NONE)
#undef MJ_W8A8
    }
    return;
  }
  // a lane's block (i, j) holds output row m0 + wm*WM + 16 i + (lane & 15) at
  // the 4 columns n0 + wn*WN + 16 j + 4 (lane >> 4) + q.  Blocks j of one
  // row block go out back to back (j inner): consecutive 64-byte pieces of
  // the same output rows, so whole 128-byte lines reach the L2 together.
  const bool vec = (p.ldc & 3) == 0 && ((uintptr_t)(MODE == 0 ? (void *)p.C : (void *)p.Y) & 15) == 0;
  float bq[TN][4];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int nb = n0 + wn * WN + j * 16 + 4 * fh;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      bq[j][q] = MODE == 1 && p.bias ? p.bias[nb + q < N ? nb + q : N - 1] : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm * WM + i * 16 + fr;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int nb = n0 + wn * WN + j * 16 + 4 * fh;
      if constexpr (MODE == 0) {
        int32_t *dst = p.C + (size_t)m * p.ldc + nb;
        if (vec && nb + 3 < N) {
          *(i32x4 *)dst = acc[i][j];
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (nb + q < N) dst[q] = acc[i][j][q];
        }
      } else {
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
#pragma clang fp contract(off)
          v[q] = (float)acc[i][j][q] * p.sf + bq[j][q];
        }
        float *dst = p.Y + (size_t)m * p.ldc + nb;
        if (vec && nb + 3 < N) {
          *(f32x4 *)dst = f32x4{v[0], v[1], v[2], v[3]};
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (nb + q < N) dst[q] = v[q];
        }
      }
    }
  }
}

// Launches gemm_i8_w4_kernel<BN, MODE> for p: 256 x 256 tiles when they
// cover at least 192 CUs' worth of workgroups, else 256 x 128.
template <int MODE>
static hipError_t launch_i8_w4(const GemmI8 &p, hipStream_t stream) {
  constexpr size_t lds256 = size_t(2 * 256 + 3 * 256) * kBK * sizeof(uint16_t);  // 160 KB
  constexpr size_t lds128 = size_t(2 * 256 + 3 * 128) * kBK * sizeof(uint16_t);  // 112 KB
  // a tile's 256 rows of K bytes in 32-bit buffer offsets; the scalar K
  // offset of a stage below 2^31; whole 16-byte chunks of K (a chunk must not
  // straddle two rows) from 16-byte aligned rows
  if (256 * p.lda >= ((int64_t)1 << 31) || 256 * p.ldb >= ((int64_t)1 << 31) ||
      p.K >= ((int64_t)1 << 30) || p.K % 16 != 0 || p.lda % 16 != 0 || p.ldb % 16 != 0 ||
      (((uintptr_t)p.A | (uintptr_t)p.B) & 15) != 0)
    return hipErrorInvalidValue;
  static std::atomic<uint64_t> attr_set{0};
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
  const uint64_t bit = dev < 64 ? (uint64_t)1 << dev : 0;
  if (!bit || !(attr_set.load(std::memory_order_acquire) & bit)) {
    hipError_t e = hipFuncSetAttribute((const void *)gemm_i8_w4_kernel<256, MODE>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds256);
    if (e == hipSuccess)
      e = hipFuncSetAttribute((const void *)gemm_i8_w4_kernel<128, MODE>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds128);
    if (e != hipSuccess) return e;
    attr_set.fetch_or(bit, std::memory_order_release);
  }
  const int64_t tiles256 = ((p.M + 255) / 256) * ((p.N + 255) / 256);
  const int64_t tiles128 = ((p.M + 255) / 256) * ((p.N + 127) / 128);
  if (tiles128 > INT32_MAX) return hipErrorInvalidValue;
  if (tiles256 >= 192)
    hipLaunchKernelGGL((gemm_i8_w4_kernel<256, MODE>), dim3((unsigned)tiles256), dim3(256), lds256,
                       stream, p);
  else
    hipLaunchKernelGGL((gemm_i8_w4_kernel<128, MODE>), dim3((unsigned)tiles128), dim3(256), lds128,
                       stream, p);
  return hipGetLastError();
}

hipError_t launch_gemm_i8_w4(const int8_t *A, const int8_t *B, int32_t *C, float *y, float sf,
                             const float *b, int64_t M, int64_t N, int64_t K,
                             hipStream_t stream) {
  GemmI8 p;
  p.A = A; p.lda = K; p.B = B; p.ldb = K; p.C = C; p.Y = y; p.ldc = N;
  p.sf = sf; p.bias = b; p.M = M; p.N = N; p.K = K;
  return y ? launch_i8_w4<1>(p, stream) : launch_i8_w4<0>(p, stream);
}

hipError_t launch_linear_w8a8(const int8_t *xq, const float *sx, const int8_t *Wq,
                              const float *sw, const float *bias, int epi, uint16_t *y,
                              int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  GemmI8 p;
  p.A = xq; p.lda = K; p.B = Wq; p.ldb = K; p.Yb = y; p.ldc = N;
  p.sx = sx; p.sw = sw; p.bias = bias; p.epi = epi; p.M = M; p.N = N; p.K = K;
  return launch_i8_w4<2>(p, stream);
}

// ---------------------------------------------------------------------------
// W8A16 tiles with one wave per SIMD: A bf16, B int8 per-channel weights.
// The bf16 tile pipeline (2 A buffers of 128-byte rows, 3 B
// buffers, one barrier between the two 32-deep steps of a 64-deep stage, the
// stage's direct loads spread one per MFMA group), with the weights kept int8
// all the way into registers:
//  * B rows are 64 bytes per stage in LDS, filled by direct loads (16 rows per
//    1-KB load); the 16-byte chunk c of row r is stored at c ^ ((r >> 2) & 3);
//  * a lane's B fragment of a 32-deep step is 8 int8 (one ds_read_b64 at
//    8-byte unit (4 ks + fh) ^ 2 ((r >> 2) & 3)), widened exactly to bf16 in
//    registers (i8x8_quarter: |q| <= 127 is exact in bf16) two MFMA groups
//    before its MFMAs use it, beside the group's last 8 MFMAs (at most two
//    VALU ops beside each);
//  * the widening costs one v_cvt_f32_i32 per int8, and a convert holds the
//    wave's issue for about half of an MFMA's 16 cycles, so the wave tile is
//    as tall as the tile: a fragment widened once feeds TM = WM / 16 MFMAs.
//    Plain GEMMs run BM x BN = 256 x 128 with 1 x 4 waves of 256 x 32 (WMT =
//    256: half a convert per MFMA, 18 fragment reads per 32 MFMAs); the
//    gate/up GEMM runs 256 x 192 or 256 x 256 with 1 x 4 waves of 256 x 48 or
//    256 x 64, waves 0-1 on the tile's gate rows and waves 2-3 on the up rows
//    of the same output columns, paired through LDS in the epilogue
//    (gateup_split_epilogue).  WMT = 128 (2 x 2 or 1 x 4 waves of 128 rows,
//    one convert per MFMA) is the plain-GEMM layout these replaced;
//  * the B fragment reads are inline asm (ds_read8_asm): as C++ reads the
//    compiler put a full vmcnt(0) before each of them, which took away the
//    load pipelining and doubled the kernel's time;
//  * split-K: workgroup (split, tile) runs its K slice into fp32 partials,
//    reduced by splitk_reduce_kernel.
template <int V>
using IC = std::integral_constant<int, V>;

typedef __attribute__((address_space(3))) const uint8_t lds_u8;

// LDS read of 8 bytes as inline asm.  The compiler's wait-count pass cannot
// tell such a read from the direct loads still in flight into other LDS
// buffers and, for a C++ read, waits for all of them (vmcnt(0)) before it;
// the kernel's own waits (the per-stage vmcnt and barrier) already order every
// read after the loads it needs.  The result is not tracked by the compiler,
// which treats the register as written at once: the caller waits (lgkmcnt)
// and then marks the register landed().
__device__ __forceinline__ uint2 ds_read8_asm(uint32_t addr) {
  uint2 r;
  asm volatile("ds_read_b64 %0, %1" : "=v"(r) : "v"(addr) : "memory");
  return r;
}
// Placed after the wait for an asm read: an empty asm that takes the register
// as read-written, so no use of the value (and no reuse of the register) can
// be moved ahead of the wait, not even by IR passes, which see the wait as an
// unrelated call.
__device__ __forceinline__ void landed(uint2 &r) { asm volatile("" : "+v"(r)); }

// Quarter p of an int8x8 fragment widened to bf16: int8 2p and 2p+1 of the
// 8 in q as bf16x2.
// An integer of magnitude <= 128 has at most 8 significant bits, so its bf16
// is exactly the upper half of its fp32: one byte permute packs two (an
// integer op, cheaper beside the MFMAs than the float convert-and-pack).
__device__ __forceinline__ uint32_t i8x8_quarter(uint2 q, int p) {
  const int32_t v = (int32_t)(p < 2 ? q.x : q.y);
  const float lo = (p & 1) ? (float)((v << 8) >> 24) : (float)((v << 24) >> 24);
  const float hi = (p & 1) ? (float)(v >> 24) : (float)((v << 16) >> 24);
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}
// The two halves of i8x8_quarter, so that the pack can be issued an MFMA
// after the converts it consumes (their latency then hides under the MFMA).
__device__ __forceinline__ void i8x8_quarter_cvt(uint2 q, int p, float &lo, float &hi) {
  const int32_t v = (int32_t)(p < 2 ? q.x : q.y);
  lo = (p & 1) ? (float)((v << 8) >> 24) : (float)((v << 24) >> 24);
  hi = (p & 1) ? (float)(v >> 24) : (float)((v << 16) >> 24);
}
__device__ __forceinline__ uint32_t i8x8_quarter_pack(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// Gate/up epilogue of the split layout (1 x 4 waves of 256 x WN): wave wn < 2
// holds the gate sums of output columns [wn WN, wn WN + WN) of the tile, wave
// wn + 2 the up sums of the same columns, for all 256 rows.  Each side scales
// its sums (g = acc * sg, u = acc * su, as the paired layout) and hands one
// half of the rows to its partner through its own LDS region (the gate waves
// rows 0-127 into xs[0], the up waves rows 128-255 into xs[1], each 128 rows
// of the tile's 2 WN columns in fp32); then the up waves finish rows 0-127 and
// the gate waves rows 128-255: h = silu_b16(g) * u in bf16, the same
// arithmetic as the paired layout.  Full tiles are stored from registers;
// partial ones are staged through LDS (after every wave has read xs) and
// written by flush_tile.  The LDS is free on entry (every wave has passed the
// K loop's last barrier).
template <int TM, int TN, int WN>
__device__ __forceinline__ void gateup_split_epilogue(const GemmNT &p, const f32x4 (&acc)[TM][TN],
                                                      float *xs, int m0, int n0, int wn, int lane,
                                                      bool full) {
  constexpr int HM = TM / 2;            // row blocks handed over / kept
  constexpr int HR = HM * 16;           // rows of one exchange region
  constexpr int LDX = 2 * WN + 4;       // fp32 row stride of the exchange regions
  const int N = (int)p.N;
  const int fr = lane & 15, fh = lane >> 4;
  const bool up = wn >= 2;
  const int cw = (up ? wn - 2 : wn) * WN;  // the wave's first output column in the tile
  float sc[TN][4];
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n0 + cw + j * 16 + 4 * fh + q;
      const int nc = n < N ? n : N - 1;
      sc[j][q] = up ? p.scales2[nc] : p.scales[nc];
    }
  // the accumulator row block indices must be compile-time constants (a
  // runtime index would move the accumulators to scratch), hence one body
  // per side
  auto run = [&](auto up_c) {
    constexpr bool UP = decltype(up_c)::value;
    constexpr int send0 = UP ? HM : 0, keep0 = UP ? 0 : HM;
#pragma unroll
    for (int i = 0; i < HM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        f32x4 v;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
#pragma clang fp contract(off)
          v[q] = acc[send0 + i][j][q] * sc[j][q];
        }
        *(f32x4 *)(xs + ((UP ? HR : 0) + i * 16 + fr) * LDX + cw + j * 16 + 4 * fh) = v;
      }
    __syncthreads();
    // h of row block keep0 + i, column block j (4 values of one lane), the
    // partner's half from the other region
    auto h4 = [&](int i, int j, float (&h)[4]) {
      const f32x4 o =
          *(const f32x4 *)(xs + ((UP ? 0 : HR) + i * 16 + fr) * LDX + cw + j * 16 + 4 * fh);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
#pragma clang fp contract(off)
        const float own = acc[keep0 + i][j][q] * sc[j][q];
        const float g = UP ? o[q] : own;
        const float u = UP ? own : o[q];
        h[q] = silu_b16(g) * u;
      }
    };
    if (full) {
#pragma unroll
      for (int i = 0; i < HM; ++i) {
        const int m = m0 + (keep0 + i) * 16 + fr;
#pragma unroll
        for (int j = 0; j + 1 < TN; j += 2) {
          float x[4], y[4];
          h4(i, j, x);
          h4(i, j + 1, y);
          const auto w0 = __builtin_amdgcn_permlane16_swap(pack_bf16x2(x[0], x[1]),
                                                           pack_bf16x2(y[0], y[1]), false, false);
          const auto w1 = __builtin_amdgcn_permlane16_swap(pack_bf16x2(x[2], x[3]),
                                                           pack_bf16x2(y[2], y[3]), false, false);
          const int n = n0 + cw + (j + (fh & 1)) * 16 + 8 * (fh >> 1);
          *(uint4 *)(p.C + (size_t)m * p.ldc + n) = make_uint4(w0[0], w1[0], w0[1], w1[1]);
        }
        if constexpr (TN % 2 == 1) {
          float h[4];
          h4(i, TN - 1, h);
          const int n = n0 + cw + (TN - 1) * 16 + 4 * fh;
          *(uint2 *)(p.C + (size_t)m * p.ldc + n) = make_uint2(pack_bf16x2(h[0], h[1]),
                                                               pack_bf16x2(h[2], h[3]));
        }
      }
      return;
    }
    // partial tile: h as bf16 in registers, then (once every wave has read
    // xs) into the staging tile over it
    uint32_t hp[HM][TN][2];
#pragma unroll
    for (int i = 0; i < HM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        float h[4];
        h4(i, j, h);
        hp[i][j][0] = pack_bf16x2(h[0], h[1]);
        hp[i][j][1] = pack_bf16x2(h[2], h[3]);
      }
    __syncthreads();
    constexpr int LD = stage_ld<2 * WN>();
    uint16_t *ct = (uint16_t *)xs;
#pragma unroll
    for (int i = 0; i < HM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        *(uint2 *)(ct + ((keep0 + i) * 16 + fr) * LD + cw + j * 16 + 4 * fh) =
            make_uint2(hp[i][j][0], hp[i][j][1]);
    __syncthreads();
    flush_tile<TM * 16, 2 * WN, 256>(p, ct, m0, n0);
  };
  if (up) run(std::true_type());
  else run(std::false_type());
}

template <int BM, int BN, bool GATEUP, int WMT = 128, int DEPTH = 2>
__global__ __launch_bounds__(256) void gemm_nt_w4i8_kernel(GemmNT p) {
  constexpr int NT = 256;
  // DEPTH 2: stage kt + 2's B loads go out in stage kt's first step (three B
  // buffers), its A loads in the second (two A buffers).  DEPTH > 2: a ring
  // of DEPTH stages for A and B alike; stage kt + DEPTH's loads all go out in
  // stage kt's second step into stage kt's slot (free once the stage's
  // barrier is passed: its second-step fragments were read in its first
  // step), so every load has about DEPTH - 1/2 stages to land before the
  // wait that covers it (loads retire in order: issuing B earlier than A
  // would not give B more time, since the wait for the A loads issued after
  // it covers it too).  The weights of a short-M GEMM stream from HBM once,
  // and two stages in flight left that stream latency-bound; a ring of six
  // (128 x 128 tiles, 144 KB of LDS) measured between two and three.
  static_assert(DEPTH == 2 || DEPTH == 3 || DEPTH == 6, "ring depth divides the 6-stage round");
  constexpr int NA = DEPTH == 2 ? 2 : DEPTH;  // A slots
  constexpr int NB = DEPTH == 2 ? 3 : DEPTH;  // B slots
  // waves: WMS x WNS, each owning WM x WN (WMT = 128: 2 x 2 on 256-row tiles,
  // 1 x 4 on 128-row ones; WMT = 256: 1 x 4 on 256-row tiles)
  constexpr int WM = WMT, WMS = BM / WM, WNS = 4 / WMS;
  constexpr int WN = BN / WNS, TM = WM / 16, TN = WN / 16;
  static_assert(WMT == 128 || (WMT == 256 && BM == 256), "wave tile height");
  // gate/up (WMT = 256 only): the tile's B rows are BN/2 gate rows then the
  // BN/2 up rows of the same output columns, so waves 0-1 hold gate sums and
  // waves 2-3 the up sums of the same columns (paired in the epilogue through
  // LDS)
  static_assert(!GATEUP || WMS == 1, "gate/up runs the split layout (1 x 4 waves)");
  static_assert(TN >= 2, "the widened-fragment rotation needs two blocks per step");
  // the B widening of a group sits beside its last 8 MFMAs
  constexpr int CU0 = TM - 8;
  constexpr int BN_OUT = GATEUP ? BN / 2 : BN;
  constexpr int A_DPW = BM / 32;             // 1-KB A loads per wave per stage
  constexpr int B_DPW = BN / 64;             // 1-KB B loads per wave per stage (16 rows each)
  constexpr int BROW = 64;                   // int8 B row bytes per stage
  static_assert(BM == 256 || BM == 128, "tile height");
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  uint16_t *As = lds;                                        // [NA][BM][64] bf16
  int8_t *Bs = (int8_t *)(lds + NA * BM * kBK);              // [NB][BN][64] int8

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WNS, wn = wave % WNS;
  const int M = (int)p.M, N = (int)p.N, K = (int)p.K;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN_OUT - 1) / BN_OUT;
  int split, tm, tn;
  split_tile_coords(blockIdx.x, tiles_m, tiles_n, p.splits, 4, split, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN_OUT;
  const int nk_all = (K + kBK - 1) / kBK;
  const int per = (nk_all + p.splits - 1) / p.splits;
  const int kt0 = split * per;
  const int kt1 = kt0 + per < nk_all ? kt0 + per : nk_all;
  const int Kend = kt1 * kBK < K ? kt1 * kBK : K;  // loads stop here (zero fill beyond)

  const __amdgpu_buffer_rsrc_t rA = make_rsrc(p.A + (size_t)m0 * p.lda,
                                              ((int64_t)(M - m0) * p.lda) * 2);
  const __amdgpu_buffer_rsrc_t rB = make_rsrc(p.B, (int64_t)N * p.ldb);
  const __amdgpu_buffer_rsrc_t rB2 = make_rsrc(GATEUP ? p.B2 : p.B, (int64_t)N * p.ldb);
  uint32_t a_off[A_DPW];
  int a_kc[A_DPW];
#pragma unroll
  for (int i = 0; i < A_DPW; ++i) {
    const int r = (i * 4 + wave) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    a_kc[i] = c;
    a_off[i] = m0 + r < M ? (uint32_t)((r * p.lda + c * 8) * 2) : kOobOffset;
  }
  // B block b = i*4 + wave covers LDS rows [16b, 16b+16): row 16b + lane/4,
  // stored chunk lane%4 holds logical chunk c of the weight row
  uint32_t b_off[B_DPW];
  int b_kc[B_DPW];
  bool b_up[B_DPW];
#pragma unroll
  for (int i = 0; i < B_DPW; ++i) {
    const int r = (i * 4 + wave) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 2) & 3);
    int n = n0 + r;
    b_up[i] = false;
    if (GATEUP) {
      b_up[i] = r >= BN / 2;
      n = n0 + (b_up[i] ? r - BN / 2 : r);
    }
    b_kc[i] = c;
    b_off[i] = n < N ? (uint32_t)((size_t)n * p.ldb + c * 16) : kOobOffset;
  }
  // direct load d of stage kt: d < 8 is A block d into A buffer abuf, else B
  // block d - 8 into B buffer bbuf.  FAST: the stage lies inside the K slice.
  auto load = [&](auto fast, int kt, int buf, int d) __attribute__((always_inline)) {
    const int k0 = kt * kBK;
    if (d < A_DPW) {
      uint16_t *dst = As + buf * BM * kBK + (d * 4 + wave) * 8 * kBK;
      if constexpr (decltype(fast)::value) {
        dma16s(rA, dst, a_off[d], (uint32_t)(k0 * 2));
      } else {
        const bool ok = k0 + a_kc[d] * 8 < Kend;
        dma16s(rA, dst, ok ? a_off[d] + k0 * 2 : kOobOffset, 0u);
      }
    } else {
      const int i = d - A_DPW;
      uint16_t *dst = (uint16_t *)(Bs + buf * BN * BROW + (i * 4 + wave) * 16 * BROW);
      const __amdgpu_buffer_rsrc_t r = (GATEUP && b_up[i]) ? rB2 : rB;
      if constexpr (decltype(fast)::value) {
        dma16s(r, dst, b_off[i], (uint32_t)k0);
      } else {
        const bool ok = k0 + b_kc[i] * 16 < Kend;
        dma16s(r, dst, ok ? b_off[i] + k0 : kOobOffset, 0u);
      }
    }
  };

  const int fr = lane & 15, fh = lane >> 4;
  const int sw = (fr >> 1) & 7;
  const uint16_t *a_rd[2];
  uint32_t b_rd[2];  // LDS byte addresses
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    a_rd[ks] = As + (wm * WM + fr) * kBK + ((ks * 4 + fh) ^ sw) * 8;
    // rows of a wave's B blocks start at multiples of 16, so (r >> 2) & 3 is
    // (fr >> 2) & 3
    b_rd[ks] = (uint32_t)(uintptr_t)(lds_u8 *)(Bs + (wn * WN + fr) * BROW +
                                               (((ks * 4 + fh) ^ (2 * ((fr >> 2) & 3)))) * 8);
  }

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  bf16x8 fa[2][TM];
  uint2 fbr[2][TN];      // raw int8 B fragments
  // widened B fragments (bf16x2 words): group g of the kernel's sequence uses
  // fbc[g % 3] while the fragment of group g + 2 is built in fbc[(g + 2) % 3]
  uint32_t fbc[3][4];
  float cvt_lo[4], cvt_hi[4];  // converted int8 pairs awaiting their pack

  constexpr int NDMA = A_DPW + B_DPW;
  constexpr int PRO = DEPTH;  // stages loaded before the loop
#pragma unroll
  for (int s2 = 0; s2 < PRO; ++s2)
#pragma unroll
    for (int d = 0; d < NDMA; ++d) load(std::false_type(), kt0 + s2, s2, d);
  constexpr int PW = (PRO - 1) * NDMA;  // loads after stage kt0's
  static_assert(PW < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (PW & 0xF) | ((PW >> 4) << 14));  // stage kt0
  asm volatile("s_barrier" ::: "memory");
#pragma unroll
  for (int j = 0; j < TN; ++j) fbr[0][j] = ds_read8_asm(b_rd[0] + j * 16 * BROW);
#pragma unroll
  for (int i = 0; i < TM; ++i) fa[0][i] = *(const bf16x8 *)(a_rd[0] + i * 16 * kBK);
  __builtin_amdgcn_s_waitcnt(kLgkm0);
#pragma unroll
  for (int j = 0; j < TN; ++j) landed(fbr[0][j]);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    fbc[0][q] = i8x8_quarter(fbr[0][0], q);
    fbc[1][q] = i8x8_quarter(fbr[0][TN > 1 ? 1 : 0], q);
  }
  asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");  // zero fill -> first MFMAs

  // one 32-deep step: MFMAs on fa[src] and the widened fbr[src]; the step's
  // TN + TM fragment reads for the next step (B first, into fbr/fa[dst], from
  // B buffer bbuf and A buffer abuf) are spread over its groups, and its nload
  // direct loads (load_d, load_d + 1, ...) into buffer load_buf over its first
  // groups.  Group j widens the B fragment of group j + 1 (the last group: the
  // next step's first, read at the start of this step) in four quarters: the
  // two converts of quarter u follow MFMA u and their pack follows MFMA u + 1,
  // so the convert latency hides under an MFMA instead of stalling issue, and
  // three MFMAs separate the last VALU write from the first MFMA that reads
  // it (the asm MFMAs are invisible to the compiler's hazard recognizer; that
  // distance covers the VALU -> MFMA operand hazard).  Every index argument is a compile-time
  // constant, so the fragment arrays stay in registers and the LDS pointers
  // keep their address space.
  auto step = [&](auto src_c, auto dst_c, auto abuf_c, auto bbuf_c, auto fast, int kt,
                  auto load_d_c, auto nload_c, auto load_buf_c,
                  auto g0_c) __attribute__((always_inline)) {
    constexpr int src = decltype(src_c)::value, dst = decltype(dst_c)::value;
    constexpr int g0 = decltype(g0_c)::value;  // sequence number of the step's group 0
    constexpr int abuf = decltype(abuf_c)::value, bbuf = decltype(bbuf_c)::value;
    constexpr int load_d = decltype(load_d_c)::value, nload = decltype(nload_c)::value;
    constexpr int load_buf = decltype(load_buf_c)::value;
    constexpr int NR = TM + TN;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int t0 = (j * NR + TN - 1) / TN;
      const int t1 = ((j + 1) * NR + TN - 1) / TN;
#pragma unroll
      for (int u = 0; u < TM; ++u) {
        __builtin_amdgcn_sched_barrier(0);
        const int t = t0 + u;
        if (t < t1) {
          if (t < TN) fbr[dst][t] = ds_read8_asm(b_rd[dst] + bbuf * BN * BROW + t * 16 * BROW);
          else fa[dst][t - TN] = *(const bf16x8 *)(a_rd[dst] + abuf * BM * kBK + (t - TN) * 16 * kBK);
        }
        __builtin_amdgcn_sched_barrier(0);
        const int cur = (g0 + j) % 3, nxt = (g0 + j + 2) % 3;
        mfma_16x16x32_tied(acc[u][j],
                           __builtin_bit_cast(bf16x8, make_uint4(fbc[cur][0], fbc[cur][1],
                                                                 fbc[cur][2], fbc[cur][3])),
                           fa[src][u]);
        {
          // loads per group: ceil(nload / TN), at u = 1, 2, ...
          constexpr int lpg = (nload + TN - 1) / TN;
          static_assert(lpg < TM, "loads per group");
          const int l = j * lpg + (u - 1);
          if (u == 1 || u == 2 || (u >= 1 && u <= lpg)) {
            __builtin_amdgcn_sched_barrier(0);
            if (u <= lpg && l < nload) load(fast, kt + DEPTH, load_buf, load_d + l);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        if (u >= CU0) {
          // the fragment of group j + 2 (past the step's end: block
          // j + 2 - TN of the next step, read in this step): quarter q's two
          // converts after MFMA CU0 + 2q, its pack after MFMA CU0 + 2q + 1
          __builtin_amdgcn_sched_barrier(0);
          const int q = (u - CU0) >> 1;
          if ((u - CU0) & 1) {
            fbc[nxt][q] = i8x8_quarter_pack(cvt_lo[q], cvt_hi[q]);
          } else if (j + 2 < TN) {
            i8x8_quarter_cvt(fbr[src][j + 2], q, cvt_lo[q], cvt_hi[q]);
          } else {
            const int b = j + 2 - TN;
            if (u == CU0) {
              // fbr[dst][b] is this step's read t = b; the reads issued after
              // it up to this slot (t < min(t0 + CU0 + 1, t1)) may still be
              // in flight (LDS reads complete in order; beyond 15 of them
              // the wait is for a few more than needed)
              constexpr auto k_after = [](int jj) {
                const int tn = (jj * NR + TN - 1) / TN + CU0 + 1;
                const int t1c = ((jj + 1) * NR + TN - 1) / TN;
                const int after = (tn < t1c ? tn : t1c) - (jj + 2 - TN + 1);
                return after < 15 ? after : 15;
              };
              static_assert(k_after(TN - 2) >= 0 && k_after(TN - 1) >= 0, "read order");
              if (j == TN - 2) __builtin_amdgcn_s_waitcnt(kLgkm0 | (k_after(TN - 2) << 8));
              else __builtin_amdgcn_s_waitcnt(kLgkm0 | (k_after(TN - 1) << 8));
              landed(fbr[dst][b]);
            }
            i8x8_quarter_cvt(fbr[dst][b], q, cvt_lo[q], cvt_hi[q]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  };
  // stage kt in A buffer AB = (kt - kt0) % NA and B buffer BB = (kt - kt0) % NB
  auto stage = [&](auto ab_c, auto bb_c, auto pos_c, auto fast, int kt)
      __attribute__((always_inline)) {
    constexpr int AB = decltype(ab_c)::value;
    constexpr int BB = decltype(bb_c)::value;
    constexpr int G0 = decltype(pos_c)::value * 2 * TN;  // groups before this stage
    if constexpr (DEPTH == 2) {
      // step 0; loads of B for stage kt+2 go into B buffer (BB + 2) % 3
      step(IC<0>(), IC<1>(), IC<AB>(), IC<BB>(), fast, kt, IC<A_DPW>(), IC<B_DPW>(),
           IC<(BB + 2) % 3>(), IC<G0 % 3>());
    } else {
      step(IC<0>(), IC<1>(), IC<AB>(), IC<BB>(), fast, kt, IC<0>(), IC<0>(), IC<AB>(),
           IC<G0 % 3>());
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kLgkm0);
#pragma unroll
    for (int j = 1; j < TN; ++j) landed(fbr[1][j]);
    if constexpr (DEPTH == 2) {
      // only this stage's B loads may be in flight (loads retire in order)
      __builtin_amdgcn_s_waitcnt(0x0F70 | B_DPW);
    } else {
      // stage kt + 1 landed: the loads of stages kt + 2 .. kt + DEPTH - 1 may
      // be in flight
      constexpr int W = (DEPTH - 2) * NDMA;
      __builtin_amdgcn_s_waitcnt(0x0F70 | (W & 0xF) | ((W >> 4) << 14));
    }
    asm volatile("s_barrier" ::: "memory");
    if constexpr (DEPTH == 2) {
      // step 1; loads of A for stage kt+2 go into A buffer AB
      step(IC<1>(), IC<0>(), IC<AB ^ 1>(), IC<(BB + 1) % 3>(), fast, kt, IC<0>(), IC<A_DPW>(),
           IC<AB>(), IC<(G0 + TN) % 3>());
    } else {
      // step 1; all loads of stage kt + DEPTH go into this stage's slot
      step(IC<1>(), IC<0>(), IC<(AB + 1) % NA>(), IC<(BB + 1) % NB>(), fast, kt, IC<0>(),
           IC<NDMA>(), IC<AB>(), IC<(G0 + TN) % 3>());
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kLgkm0);
#pragma unroll
    for (int j = 1; j < TN; ++j) landed(fbr[0][j]);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using F = std::true_type;
  using S = std::false_type;
  // stages kt .. kt+5 load stages kt+DEPTH .. kt+5+DEPTH: fast while those lie inside K
  const int full_end = kt0 + (Kend - kt0 * kBK) / kBK;  // stages wholly inside the slice
  int kt = kt0;
  // (the third argument is the stage's position in the 6-stage round, which
  // fixes the rotation of the widened-fragment registers)
  if constexpr (DEPTH == 2) {
    for (; kt + 8 <= full_end; kt += 6) {
      stage(I0(), I0(), IC<0>(), F(), kt);
      stage(I1(), I1(), IC<1>(), F(), kt + 1);
      stage(I0(), I2(), IC<2>(), F(), kt + 2);
      stage(I1(), I0(), IC<3>(), F(), kt + 3);
      stage(I0(), I1(), IC<4>(), F(), kt + 4);
      stage(I1(), I2(), IC<5>(), F(), kt + 5);
    }
    for (; kt < kt1; kt += 6) {
      stage(I0(), I0(), IC<0>(), S(), kt);
      if (kt + 1 < kt1) stage(I1(), I1(), IC<1>(), S(), kt + 1);
      if (kt + 2 < kt1) stage(I0(), I2(), IC<2>(), S(), kt + 2);
      if (kt + 3 < kt1) stage(I1(), I0(), IC<3>(), S(), kt + 3);
      if (kt + 4 < kt1) stage(I0(), I1(), IC<4>(), S(), kt + 4);
      if (kt + 5 < kt1) stage(I1(), I2(), IC<5>(), S(), kt + 5);
    }
  } else {
    // slot (kt - kt0) % DEPTH; DEPTH divides the 6-stage round
    constexpr int R = DEPTH;
    for (; kt + 6 + DEPTH <= full_end; kt += 6) {
      stage(IC<0 % R>(), IC<0 % R>(), IC<0>(), F(), kt);
      stage(IC<1 % R>(), IC<1 % R>(), IC<1>(), F(), kt + 1);
      stage(IC<2 % R>(), IC<2 % R>(), IC<2>(), F(), kt + 2);
      stage(IC<3 % R>(), IC<3 % R>(), IC<3>(), F(), kt + 3);
      stage(IC<4 % R>(), IC<4 % R>(), IC<4>(), F(), kt + 4);
      stage(IC<5 % R>(), IC<5 % R>(), IC<5>(), F(), kt + 5);
    }
    for (; kt < kt1; kt += 6) {
      stage(IC<0 % R>(), IC<0 % R>(), IC<0>(), S(), kt);
      if (kt + 1 < kt1) stage(IC<1 % R>(), IC<1 % R>(), IC<1>(), S(), kt + 1);
      if (kt + 2 < kt1) stage(IC<2 % R>(), IC<2 % R>(), IC<2>(), S(), kt + 2);
      if (kt + 3 < kt1) stage(IC<3 % R>(), IC<3 % R>(), IC<3>(), S(), kt + 3);
      if (kt + 4 < kt1) stage(IC<4 % R>(), IC<4 % R>(), IC<4>(), S(), kt + 4);
      if (kt + 5 < kt1) stage(IC<5 % R>(), IC<5 % R>(), IC<5>(), S(), kt + 5);
    }
  }
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();

  if (p.part != nullptr) {
    if constexpr (!GATEUP) store_part8<TM, TN, WM, WN>(p, acc, m0, n0, wm, wn, lane, split);
    return;
  }
  const bool full = m0 + BM <= M && n0 + BN_OUT <= N && (p.ldc & 7) == 0 &&
                    ((uintptr_t)p.C & 15) == 0;
  if constexpr (GATEUP) {
    gateup_split_epilogue<TM, TN, WN>(p, acc, (float *)lds, m0, n0, wn, lane, full);
    return;
  } else {
    if (full) {
      switch (p.epi) {
#define MJ_DIRECT(E) store_tile_direct<E, TM, TN, WM, WN>(p, acc, m0, n0, wm, wn, lane); break;
        case EPI_RELU: MJ_DIRECT(EPI_RELU)
        case EPI_GELU_TANH: MJ_DIRECT(EPI_GELU_TANH)
        case EPI_SILU: MJ_DIRECT(EPI_SILU)
        case EPI_GELU_TANH_APPROX: MJ_DIRECT(EPI_GELU_TANH_APPROX)
        case EPI_SILU_APPROX: MJ_DIRECT(EPI_SILU_APPROX)
        case EPI_RELU_UNARY: MJ_DIRECT(EPI_RELU_UNARY)
        default: MJ_DIRECT(EPI_NONE)
#undef MJ_DIRECT
      }
      return;
    }
    switch (p.epi) {
#define MJ_STAGE(E) stage_tile<E, TM, TN, WM, WN, BN_OUT>(p, acc, lds, n0, wm, wn, lane); break;
      case EPI_RELU: MJ_STAGE(EPI_RELU)
      case EPI_GELU_TANH: MJ_STAGE(EPI_GELU_TANH)
      case EPI_SILU: MJ_STAGE(EPI_SILU)
      case EPI_GELU_TANH_APPROX: MJ_STAGE(EPI_GELU_TANH_APPROX)
      case EPI_SILU_APPROX: MJ_STAGE(EPI_SILU_APPROX)
      case EPI_RELU_UNARY: MJ_STAGE(EPI_RELU_UNARY)
      default: MJ_STAGE(EPI_NONE)
#undef MJ_STAGE
    }
  }
  __syncthreads();
  flush_tile<BM, BN_OUT, NT>(p, lds, m0, n0);
}

// Sums the split-K partials in split order and applies scale, bias, the
// activation and the bf16 rounding.  Rows of a multiple of 8 columns with a
// 16-byte aligned output, scales and bias take 8 columns per thread: the
// thread's scales and biases and all of its partial loads (two 16-byte
// loads per split) are issued before the sums, and the result is one 16-byte
// store; anything else takes 4 columns per thread.  The partials were written
// by the GEMM just before: plain loads read them 6 % faster than nontemporal
// ones (C5's down projection, 8.33 -> 7.86 us on MI355X).
template <int E>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmNT p) {
  const int M = (int)p.M, N = (int)p.N;
  const size_t plane = (size_t)M * N;
  const bool has_s = p.scales != nullptr, has_b = p.bias != nullptr;
  if ((N & 7) == 0 && (p.ldc & 7) == 0 && ((uintptr_t)p.C & 15) == 0 && p.splits <= 8 &&
      (((uintptr_t)p.scales | (uintptr_t)p.bias) & 15) == 0) {
    const int n8 = N / 8;
    const int64_t total8 = (int64_t)M * n8;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total8;
         t += (int64_t)gridDim.x * blockDim.x) {
      const int m = (int)(t / n8);
      const int nb = (int)(t - (int64_t)m * n8) * 8;
      // the 8 columns' scales and biases first, as two 16-byte loads each:
      // fetched per element after the partials they were a second round trip
      // at the end of every thread (C5's down projection: 10.7 -> 8.7 us)
      float sc[8], bi[8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const f32x4 s4 = has_s ? *(const f32x4 *)(p.scales + nb + 4 * h) : f32x4{1.f, 1.f, 1.f, 1.f};
        const f32x4 b4 = has_b ? *(const f32x4 *)(p.bias + nb + 4 * h) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          sc[4 * h + q] = s4[q];
          bi[4 * h + q] = b4[q];
        }
      }
      const float *src = p.part + (size_t)m * N + nb;
      f32x4 part[8][2];
#pragma unroll
      for (int sp = 0; sp < 8; ++sp) {
        if (sp < p.splits) {
          part[sp][0] = *(const f32x4 *)(src + sp * plane);
          part[sp][1] = *(const f32x4 *)(src + sp * plane + 4);
        }
      }
      float v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        float acc = 0.0f;
#pragma unroll
        for (int sp = 0; sp < 8; ++sp)
          if (sp < p.splits) acc += part[sp][q >> 2][q & 3];
        v[q] = apply_epi_b16(E, epi_scale_bias(acc, sc[q], bi[q], has_s, has_b));
      }
      *(uint4 *)(p.C + (size_t)m * p.ldc + nb) =
          make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                     pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
    }
    return;
  }
  const int n4 = (N + 3) / 4;
  const int64_t total = (int64_t)M * n4;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int m = (int)(t / n4);
    const int nb = (int)(t - (int64_t)m * n4) * 4;
    float v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = nb + q < N ? nb + q : N - 1;
      float acc = 0.0f;
      for (int s = 0; s < p.splits; ++s) acc += p.part[s * plane + (size_t)m * N + n];
      v[q] = apply_epi_b16(E, epi_scale_bias(acc, has_s ? p.scales[n] : 1.0f,
                                         has_b ? p.bias[n] : 0.0f, has_s, has_b));
    }
    store4_bf16(p, m, nb, v);
  }
}

static hipError_t launch_reduce(const GemmNT &p, hipStream_t stream) {
  // 8 columns per thread on the 16-byte path of the kernel, else 4
  const bool vec8 = (p.N & 7) == 0 && (p.ldc & 7) == 0 && ((uintptr_t)p.C & 15) == 0 &&
                    p.splits <= 8 && (((uintptr_t)p.scales | (uintptr_t)p.bias) & 15) == 0;
  const int64_t total = vec8 ? p.M * (p.N / 8) : p.M * ((p.N + 3) / 4);
  int64_t blocks = (total + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  const dim3 g((unsigned)blocks), b(256);
  switch (p.epi) {
    case EPI_RELU: hipLaunchKernelGGL(splitk_reduce_kernel<EPI_RELU>, g, b, 0, stream, p); break;
    case EPI_GELU_TANH:
      hipLaunchKernelGGL(splitk_reduce_kernel<EPI_GELU_TANH>, g, b, 0, stream, p); break;
    case EPI_SILU: hipLaunchKernelGGL(splitk_reduce_kernel<EPI_SILU>, g, b, 0, stream, p); break;
    case EPI_GELU_TANH_APPROX:
      hipLaunchKernelGGL(splitk_reduce_kernel<EPI_GELU_TANH_APPROX>, g, b, 0, stream, p); break;
    case EPI_SILU_APPROX:
      hipLaunchKernelGGL(splitk_reduce_kernel<EPI_SILU_APPROX>, g, b, 0, stream, p); break;
    case EPI_RELU_UNARY:
      hipLaunchKernelGGL(splitk_reduce_kernel<EPI_RELU_UNARY>, g, b, 0, stream, p); break;
    default: hipLaunchKernelGGL(splitk_reduce_kernel<EPI_NONE>, g, b, 0, stream, p); break;
  }
  return hipGetLastError();
}

template <int BM, int BN, int BKIND, bool GATEUP, bool IGLP, bool PF2 = false, int NW = 8>
static hipError_t launch_tile(const GemmNT &p, hipStream_t stream) {
  constexpr int BN_OUT = GATEUP ? BN / 2 : BN;
  constexpr size_t lds_loop = size_t(2) * (BM + BN) * kBK * sizeof(uint16_t);
  constexpr size_t lds_out = size_t(BM) * stage_ld<BN_OUT>() * sizeof(uint16_t);
  constexpr size_t lds = lds_loop > lds_out ? lds_loop : lds_out;
  static_assert(lds <= 160 * 1024, "LDS budget");
  auto kern = gemm_nt_kernel<BM, BN, BKIND, GATEUP, IGLP, PF2, NW>;
  // the dynamic-LDS limit is raised once per device this kernel runs on
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
  const int64_t grid = ((p.M + BM - 1) / BM) * ((p.N + BN_OUT - 1) / BN_OUT) * p.splits;
  if (grid > INT32_MAX) return hipErrorInvalidValue;  // grid.x limit
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(NW * 64), lds, stream, p);
  return hipGetLastError();
}

template <int BM, int BN, bool GATEUP, int WMT = 128, int DEPTH = 2>
static hipError_t launch_w4i8(const GemmNT &p, hipStream_t stream) {
  constexpr int BN_OUT = GATEUP ? BN / 2 : BN;
  constexpr int NA = DEPTH == 2 ? 2 : DEPTH, NB = DEPTH == 2 ? 3 : DEPTH;
  constexpr size_t lds_loop = size_t(NA) * BM * kBK * sizeof(uint16_t) + size_t(NB) * BN * 64;
  constexpr size_t lds_out = size_t(BM) * stage_ld<BN_OUT>() * sizeof(uint16_t);
  // the split gate/up epilogue's two fp32 exchange regions (128 rows each)
  constexpr size_t lds_x = GATEUP ? size_t(2) * (WMT / 2) * (BN_OUT + 4) * 4 : 0;
  constexpr size_t lds_lo = lds_loop > lds_out ? lds_loop : lds_out;
  constexpr size_t lds = lds_lo > lds_x ? lds_lo : lds_x;
  static_assert(lds <= 160 * 1024, "LDS budget");
  // buffer offsets: A rows of the tile and every weight row must stay within
  // 31-bit offsets, K advances in the scalar offset
  if (p.K >= ((int64_t)1 << 30) || p.bkind != B_INT8 || p.gate_up != GATEUP ||
      p.N * p.ldb >= ((int64_t)1 << 31) || BM * p.lda * 2 >= ((int64_t)1 << 31))
    return hipErrorInvalidValue;
  auto kern = gemm_nt_w4i8_kernel<BM, BN, GATEUP, WMT, DEPTH>;
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
  const int64_t grid = ((p.M + BM - 1) / BM) * ((p.N + BN_OUT - 1) / BN_OUT) * p.splits;
  if (grid > INT32_MAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(256), lds, stream, p);
  return hipGetLastError();
}

// The W8A16 tile kernel with the plan's load depth (2, or the 3-stage ring).
template <int BM, int BN, bool GATEUP, int WMT>
static hipError_t launch_w4i8_d(const GemmNT &p, int depth, hipStream_t stream) {
  if (depth == 3) return launch_w4i8<BM, BN, GATEUP, WMT, 3>(p, stream);
  if (depth != 2) return hipErrorInvalidValue;
  return launch_w4i8<BM, BN, GATEUP, WMT>(p, stream);
}

template <int BKIND, bool IGLP, bool PF2>
static hipError_t launch_plain(int bm, int bn, const GemmNT &p, hipStream_t stream) {
  if (bm == 256 && bn == 256) return launch_tile<256, 256, BKIND, false, IGLP, PF2>(p, stream);
  if (bm == 256 && bn == 128) return launch_tile<256, 128, BKIND, false, IGLP, PF2>(p, stream);
  if (bm == 128 && bn == 256) return launch_tile<128, 256, BKIND, false, IGLP, PF2>(p, stream);
  return launch_tile<128, 128, BKIND, false, IGLP, PF2>(p, stream);
}

// Chooses the tile shape, K split and schedule by predicted time.
//
// A launch of W workgroups runs in rounds of (256 CUs x resident workgroups
// per CU); a 128 x 128 tile needs 64 KB of LDS so two share a CU, the larger
// tiles take one CU each.  A round costs (K stages per workgroup) x (time of
// one 64-deep K stage at that shape and occupancy), and a K split adds the
// fp32 partial round trip (8 B per output and split, plus the bf16 result)
// at ~5 TB/s and one extra launch.  The per-stage times are measured on
// MI355X at the BASELINE shapes (4096^3 bf16, 2048x4096x4096 and
// 512x4096x11008 W8A16) with the schedule the plan selects; a 256 x 256
// tile is never split (its short-K slices measured well below the model).
namespace {
struct StageCost {
  int bm, bn, per_cu;
  double us_full[2];  // per stage, CU holding per_cu workgroups: [bf16 B, int8 B]
  double us_one[2];   // per stage, CU holding one workgroup
};
constexpr StageCost kStageCost[4] = {
    {256, 256, 1, {1.74, 2.17}, {1.74, 2.17}},  // bf16: the 4-wave kernel
    {256, 128, 1, {1.15, 1.48}, {1.15, 1.48}},
    {128, 256, 1, {1.17, 1.45}, {1.17, 1.45}},
    {128, 128, 2, {1.14, 1.54}, {0.80, 0.88}},
};
constexpr int kCUs = 256;
constexpr double kPartialBytesPerUs = 5.0e6;  // 5 TB/s
constexpr double kLaunchUs = 3.0;
}  // namespace

// Schedules: bf16 tiles run the distance-2 pipeline with the compiler's
// MFMA interleave (iglp), except 128 x 128, where two resident workgroups
// per CU already cover the loads and the one-barrier pipeline is 4 % faster;
// int8 tiles run the one-barrier pipeline with iglp
// (measured C4 -10 %, C5 down -6 %) except the 256 x 256 tile, whose register
// budget the interleave exceeds; the paired gate/up tiles measured faster
// without it.

static double plan_time_us(const GemmNT &p, int bm, int bn, int splits) {
  for (const StageCost &c : kStageCost) {
    if (c.bm != bm || c.bn != bn) continue;
    const int kind = p.bkind == B_BF16 ? 0 : 1;
    const int64_t tiles = ((p.M + bm - 1) / bm) * ((p.N + bn - 1) / bn);
    const int64_t wgs = tiles * splits;
    const int64_t nk = (p.K + kBK - 1) / kBK;
    const int64_t stages = (nk + splits - 1) / splits;
    const bool full = c.per_cu > 1 && wgs > kCUs;
    const int64_t slots = (int64_t)kCUs * (full ? c.per_cu : 1);
    const int64_t rounds = (wgs + slots - 1) / slots;
    double t = (double)rounds * (double)stages * (full ? c.us_full[kind] : c.us_one[kind]);
    if (splits > 1)
      t += ((double)splits * 8.0 + 2.0) * (double)p.M * (double)p.N / kPartialBytesPerUs +
           kLaunchUs;
    return t;
  }
  return 1e30;
}

GemmPlan plan_gemm_nt(const GemmNT &p) {
  GemmPlan pl;
  // the one-wave-per-SIMD int8 kernel needs 31-bit weight offsets and K < 2^30
  const bool w4i8_ok = p.bkind == B_INT8 && p.K < ((int64_t)1 << 30) &&
                       p.N * p.ldb < ((int64_t)1 << 31) && 256 * p.lda * 2 < ((int64_t)1 << 31);
  // Up to 256 x rows (one row tile) every weight tile streams from HBM once,
  // and with two stages of loads in flight that stream was latency-bound: a
  // ring of three stages (all of a stage's loads in the second step of the
  // stage three earlier) took, on MI355X, the W8A16 GEMM 11008 x 4096 at M =
  // 64 / 128 / 192 / 256 from 26.7 / 29.1 / 35.3 / 37.8 to 24.5 / 27.0 / 34.8
  // / 36.5 us and the FFN 4096 -> 11008 -> 4096 at M = 64 / 128 / 256 from
  // 66.1 / 68.8 / 88.5 to 60.3 / 61.9 / 86.0 us (bit-identical sums).  Where
  // the weight tiles are re-read by several row tiles (C4, C5) it was 0.5-1 %
  // slower (C4 1245-1248 -> 1236-1241 TFLOP/s, C5 1154-1158 -> 1146-1151,
  // alternating bench runs on one box), so those keep two stages.
  const int depth = p.M <= 256 ? 3 : 2;
  if (p.gate_up) {
    // The one-wave-per-SIMD int8 kernel in its split layout: 1 x 4 waves of
    // BM x BN/4, gate rows in waves 0-1 and the up rows of the same columns
    // in waves 2-3, paired through LDS in the epilogue (a widened fragment
    // feeds 16 MFMAs; against 2 x 2 waves each pairing its own gate and up
    // blocks C5's gate/up 78.6 -> 68.1 us; against the 8-wave kernel, which
    // remains the fallback for weights past 31-bit offsets or K >= 2^30, 20
    // us faster).  Tiles of 256 rows, 128 up to 128 rows (half the MFMAs on
    // zero rows: the FFN 4096 -> 11008 -> 4096 at M = 33 / 64 / 128 73.9-75.2
    // / 72.5-72.8 / 76.4-76.5 -> 63.5-63.7 / 63.6-63.8 / 68.0-68.2 us), rows
    // past M loading zeros.  Output columns per tile (BN/2): 64, 96 or 128,
    // the fewest columns per CU (rounds of 256 workgroups times columns), ties
    // to the wider tile: 64 (172 workgroups) at I = 11008 up to 256 rows, 96
    // (230) at 512.  The 64-column tiles against 96 / 128 took the FFN at M =
    // 192 / 256 from 98.1 / 103.5 to 86.2-86.7 / 90.8-91.1 us.
    pl.bm = p.M > 128 || w4i8_ok ? 256 : 128;
    pl.bn = 256;
    pl.tile_kernel = w4i8_ok;
    if (pl.tile_kernel) {
      pl.wm = p.M <= 128 ? 128 : 256;
      pl.bm = pl.wm;
      pl.depth = depth;
      const int64_t tm = (p.M + 255) / 256;
      const int64_t r256 = (tm * ((p.N + 127) / 128) + 255) / 256;
      const int64_t r192 = (tm * ((p.N + 95) / 96) + 255) / 256;
      const int64_t r128 = (tm * ((p.N + 63) / 64) + 255) / 256;
      int64_t best = r256 * 128;
      if (r192 * 96 < best) pl.bn = 192, best = r192 * 96;
      if (r128 * 64 < best) pl.bn = 128;
    }
    return pl;
  }
  if (w4i8_ok && p.M > kGemvMaxM && p.M < 256) {
    // batched decode and short prefill: the same kernel on 128-row tiles for
    // M <= 128, else on 256-row tiles (rows past M load zeros), the K split
    // as below.  Against the eight-wave tiles the cost model picks, on MI355X
    // (11008 x 4096 weights, M x 4096 x): M = 17 28.3 -> 25.3 us, M = 128
    // 36.5 -> 29.2, M = 192 54.7 -> 36.0, M = 255 55.8 -> 39.1
    pl.bm = p.M <= 128 ? 128 : 256;
    pl.bn = 128;
    pl.wm = pl.bm;
    pl.depth = depth;
    pl.tile_kernel = true;
    const int64_t nk = (p.K + kBK - 1) / kBK;
    // K split until the grid covers the CUs; the share of the CU rounds the
    // grid keeps busy
    auto fill = [&](int bn, int &splits) {
      const int64_t tiles = ((p.M + pl.bm - 1) / pl.bm) * ((p.N + bn - 1) / bn);
      splits = 1;
      while (splits < 8 && tiles * splits * 2 <= 256 && nk / (splits * 2) >= 8) splits *= 2;
      const int64_t wgs = tiles * splits;
      return (double)wgs / (256.0 * (double)((wgs + 255) / 256));
    };
    int s128 = 1, s192 = 1;
    const double f128 = fill(128, s128);
    pl.splits = s128;
    // 128-row tiles 192 columns wide where they fill more of the chip
    // (waves of 128 x 48): 11008 x 4096 at M = 64 / 128 on 58 tiles x 4 K
    // slices (232 workgroups) 22.6-22.7 / 26.1-26.3 us against 24.2-24.4 /
    // 26.5-26.7 on 86 x 2 (172), MI355X, alternating runs on one box; at
    // 4096 x 11008 the 128-column tiles' 32 x 8 (256) stay (21.4 / 25.0
    // against 23.6 / 27.1 us on 22 x 8)
    if (pl.bm == 128 && fill(192, s192) > f128 + 0.05) {
      pl.bn = 192;
      pl.splits = s192;
    }
    return pl;
  }
  if (w4i8_ok && p.M >= 256) {
    // the one-wave-per-SIMD int8 kernel on 256 x 128 tiles with 1 x 4 waves of
    // 256 x 32, K split until the grid covers the 256 CUs (>= 8 stages per
    // split).  A widened B fragment feeds 16 MFMAs instead of 8, which halves
    // the int8 -> bf16 converts per MFMA (a v_cvt_f32_i32 holds a wave's issue
    // for about half an MFMA); the cost is 18 fragment reads per 32 MFMAs
    // instead of 12.  Bit-identical outputs, 5.5 % faster at 2048x4096x4096,
    // 2.9 % at the 4-way split 512 x 4096 x 11008 down projection and 5.2 % at
    // 4096^3 than 128 x 256 tiles of 1 x 4 waves of 128 x 64 (MI355X, settled
    // A/B in one process).
    // Earlier measurements: 256 x 256 tiles, which leave half the CUs idle
    // at 2048x4096x4096: 126 us, split in two: 102 us; the 8-wave 128 x 256
    // kernel 83 us; the down projection's 4-way split beats 2- and 8-way
    pl.bm = 256;
    pl.bn = 128;
    pl.wm = 256;
    pl.depth = depth;
    pl.tile_kernel = true;
    const int64_t tiles = ((p.M + 255) / 256) * ((p.N + 127) / 128);
    const int64_t nk = (p.K + kBK - 1) / kBK;
    while (pl.splits < 8 && tiles * pl.splits * 2 <= 256 && nk / (pl.splits * 2) >= 8)
      pl.splits *= 2;
    return pl;
  }
  const int64_t nk = (p.K + kBK - 1) / kBK;
  double best = 1e30;
  for (const StageCost &c : kStageCost) {
    const int max_split = (c.bm == 256 && c.bn == 256) ? 1 : 8;
    for (int sk = 1; sk <= max_split; sk *= 2) {
      if (sk > 1 && nk / sk < 8) break;  // keep >= 8 stages per split
      const double t = plan_time_us(p, c.bm, c.bn, sk);
      if (t < best * 0.999) {
        best = t;
        pl.bm = c.bm;
        pl.bn = c.bn;
        pl.splits = sk;
      }
    }
  }
  if (p.bkind == B_BF16) {
    pl.iglp = true;
    pl.pf2 = !(pl.bm == 128 && pl.bn == 128);
    // 256 x 256 runs gemm_nt_w8_kernel, two waves per SIMD (its scalar K
    // offsets need K < 2^30; beyond that the generic gemm_nt_kernel takes the tile)
    pl.tile_kernel = pl.bm == 256 && pl.bn == 256 && pl.splits == 1 && p.K < ((int64_t)1 << 30);
  } else {
    pl.iglp = !(pl.bm == 256 && pl.bn == 256);
  }
  return pl;
}

hipError_t launch_gemm_nt(const GemmNT &p_in, const GemmPlan &pl, hipStream_t stream) {
  GemmNT p = p_in;
  p.splits = pl.splits;
  if (p.gate_up) {
    p.splits = 1;
    p.part = nullptr;
    if (pl.iglp || pl.pf2) return hipErrorInvalidValue;
    if (pl.tile_kernel) {
      if (pl.bm == 128 && pl.wm == 128) {
        if (pl.bn == 128) return launch_w4i8_d<128, 128, true, 128>(p, pl.depth, stream);
        if (pl.bn == 192) return launch_w4i8_d<128, 192, true, 128>(p, pl.depth, stream);
        return launch_w4i8_d<128, 256, true, 128>(p, pl.depth, stream);
      }
      if (pl.bm != 256 || pl.wm != 256) return hipErrorInvalidValue;
      if (pl.bn == 128) return launch_w4i8_d<256, 128, true, 256>(p, pl.depth, stream);
      if (pl.bn == 192) return launch_w4i8_d<256, 192, true, 256>(p, pl.depth, stream);
      if (pl.bn == 256) return launch_w4i8_d<256, 256, true, 256>(p, pl.depth, stream);
      return hipErrorInvalidValue;
    }
    if (pl.bm == 256) return launch_tile<256, 256, B_INT8, true, false>(p, stream);
    return launch_tile<128, 256, B_INT8, true, false>(p, stream);
  }
  if (pl.splits > 1 && p.part == nullptr) return hipErrorInvalidValue;
  if (pl.splits == 1) p.part = nullptr;
  hipError_t e;
  if (p.bkind == B_BF16) {
    // the bf16 schedules built: iglp with PF2 for the large tiles, iglp alone
    // for 128 x 128
    const bool small = pl.bm == 128 && pl.bn == 128;
    if (pl.tile_kernel) {
      if (pl.bm != 256 || pl.bn != 256 || pl.splits != 1) return hipErrorInvalidValue;
      return launch_w8(p, stream);
    }
    if (!pl.iglp || pl.pf2 == small) return hipErrorInvalidValue;
    if (small)
      e = launch_tile<128, 128, B_BF16, false, true, false>(p, stream);
    else if (pl.bm == 256 && pl.bn == 256)
      e = launch_tile<256, 256, B_BF16, false, true, true>(p, stream);
    else if (pl.bm == 256)
      e = launch_tile<256, 128, B_BF16, false, true, true>(p, stream);
    else
      e = launch_tile<128, 256, B_BF16, false, true, true>(p, stream);
  } else if (pl.tile_kernel) {
    if (pl.bm == 128 && pl.bn == 128 && pl.wm == 128) {
      e = launch_w4i8_d<128, 128, false, 128>(p, pl.depth, stream);
    } else if (pl.bm == 128 && pl.bn == 192 && pl.wm == 128) {
      e = launch_w4i8_d<128, 192, false, 128>(p, pl.depth, stream);
    } else {
      if (pl.bm != 256 || pl.bn != 128 || pl.wm != 256) return hipErrorInvalidValue;
      e = launch_w4i8_d<256, 128, false, 256>(p, pl.depth, stream);
    }
  } else {
    if (pl.pf2) return hipErrorInvalidValue;
    e = pl.iglp ? launch_plain<B_INT8, true, false>(pl.bm, pl.bn, p, stream)
                : launch_plain<B_INT8, false, false>(pl.bm, pl.bn, p, stream);
  }
  if (e != hipSuccess || pl.splits == 1) return e;
  return launch_reduce(p, stream);
}

}  // namespace mj
