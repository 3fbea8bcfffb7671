// NT GEMM on gfx950 bf16 MFMA: C[M,N] = epi((A[M,K] . B[N,K]^T) * s[n] + b[n]).
//
// A is bf16, B is bf16 or int8 (per-output-channel quantized weights); both
// are K-contiguous, the layout of momijo's Linear weight [OutF, InF]
// (learn/nn/layers.mojo:347-348), so every global load is a 16-byte run of K.
//
// Structure (one workgroup = 4 waves = 256 threads per BM x BN tile):
//  * global -> registers -> LDS, double-buffered with one barrier per 64-wide
//    K step: the next K step's loads are in flight while the current one is
//    multiplied.  int8 weights are converted to bf16 (exactly: |q| <= 127) on
//    their way into LDS, so the MFMA loop is the same for both weight types.
//  * LDS rows are padded to 72 bf16 (144 B): the 16-byte fragment reads of 16
//    consecutive lanes then fall into distinct banks.
//  * each wave owns a (BM/2) x (BN/2) quarter of the tile and runs
//    v_mfma_f32_32x32x16_bf16 over it: lane l feeds row (l%32) of A and row
//    (l%32) of B with 8 consecutive K values, and receives 16 accumulators
//    at rows 8*(r/4) + 4*(l/32) + r%4, column l%32.
//  * the epilogue applies the per-column weight scale, the bias and the
//    activation in fp32 (no FMA contraction, as in the reference), rounds to
//    bf16 (RNE) and stores.
//  * gate/up mode (the Llama-style FFN): each wave's B rows hold 64 gate rows
//    followed by the 64 up rows of the same output columns, so one lane holds
//    g and u for the same (m, n) and writes silu(g*sg)*(u*su) directly.
#include "common.h"
#include "launch.h"

namespace mj {

constexpr int kBK = 64;        // K per pipeline stage
constexpr int kLds = kBK + 8;  // LDS row stride in bf16 elements (144 B)

template <int BM, int BN>
constexpr size_t gemm_nt_lds_bytes() {
  return size_t(2) * (BM + BN) * kLds * sizeof(uint16_t);
}

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

__device__ __forceinline__ float epi_scale_bias(float acc, float s, float b, bool has_s,
                                                bool has_b) {
#pragma clang fp contract(off)
  float v = acc;
  if (has_s) v = v * s;
  if (has_b) v = v + b;
  return v;
}

template <int BM, int BN, int BKIND, bool GATEUP>
__global__ __launch_bounds__(256, 1) void gemm_nt_kernel(GemmNT p) {
  constexpr int WM = BM / 2, WN = BN / 2;  // per-wave tile
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int BN_OUT = GATEUP ? BN / 2 : BN;  // output columns per tile
  constexpr int A_LOADS = BM / 32;              // 16-B chunks per thread
  constexpr int B_LOADS = BKIND == B_BF16 ? BN / 32 : BN / 64;
  static_assert(!GATEUP || TN % 2 == 0, "gate/up needs an even number of N subtiles");

  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  uint16_t *As = lds;                          // [2][BM][kLds]
  uint16_t *Bs = lds + 2 * BM * kLds;          // [2][BN][kLds]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int M = (int)p.M, N = (int)p.N, K = (int)p.K;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN_OUT - 1) / BN_OUT;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, 4, tm, tn);
  const int m0 = tm * BM;
  const int n0 = tn * BN_OUT;

  // ---- global load addressing ------------------------------------------
  // A: 8 chunks of 8 bf16 per 64-wide row; thread -> (row t/8 + 32 i, chunk t%8)
  const int a_c = tid & 7;
  const int a_r = tid >> 3;
  const uint16_t *a_ptr[A_LOADS];
  bool a_ok[A_LOADS];
#pragma unroll
  for (int i = 0; i < A_LOADS; ++i) {
    const int m = m0 + a_r + 32 * i;
    a_ok[i] = m < M;
    a_ptr[i] = p.A + (size_t)(a_ok[i] ? m : 0) * p.lda + a_c * 8;
  }
  // B rows: bf16 -> 8 chunks/row like A; int8 -> 4 chunks of 16 per row.
  constexpr int B_CPR = BKIND == B_BF16 ? 8 : 4;  // chunks per row
  constexpr int B_RPP = 256 / B_CPR;              // rows per pass
  const int b_c = tid % B_CPR;
  const int b_r = tid / B_CPR;
  const char *b_ptr[B_LOADS];
  bool b_ok[B_LOADS];
  constexpr int ESZ = BKIND == B_BF16 ? 2 : 1;
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i) {
    const int r = b_r + B_RPP * i;  // row of the LDS B tile
    int n;
    const void *base = p.B;
    if (GATEUP) {
      // wave half wn = r / (BN/2); inside it 32*TN/2 gate rows then up rows
      const int half = r / (BN / 2);
      const int rr = r % (BN / 2);
      const int up = rr / (BN / 4);
      n = n0 + half * (BN / 4) + rr % (BN / 4);
      base = up ? p.B2 : p.B;
    } else {
      n = n0 + r;
    }
    b_ok[i] = n < N;
    b_ptr[i] = (const char *)base + ((size_t)(b_ok[i] ? n : 0) * p.ldb + b_c * (16 / ESZ)) * ESZ;
  }

  uint4 ra[A_LOADS];
  uint4 rb[B_LOADS];
  auto load_stage = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const bool ok = a_ok[i] && (k0 + a_c * 8 < K);
      ra[i] = ok ? *(const uint4 *)(a_ptr[i] + k0) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const bool ok = b_ok[i] && (k0 + b_c * (16 / ESZ) < K);
      rb[i] = ok ? *(const uint4 *)(b_ptr[i] + (size_t)k0 * ESZ) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_stage = [&](int buf) {
    uint16_t *as = As + buf * BM * kLds;
    uint16_t *bs = Bs + buf * BN * kLds;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i)
      *(uint4 *)(as + (a_r + 32 * i) * kLds + a_c * 8) = ra[i];
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int r = b_r + B_RPP * i;
      if (BKIND == B_BF16) {
        *(uint4 *)(bs + r * kLds + b_c * 8) = rb[i];
      } else {
        uint4 lo, hi;
        i8x16_to_bf16x16(rb[i], lo, hi);
        *(uint4 *)(bs + r * kLds + b_c * 16) = lo;
        *(uint4 *)(bs + r * kLds + b_c * 16 + 8) = hi;
      }
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int nk = (K + kBK - 1) / kBK;
  load_stage(0);
  store_stage(0);
  __syncthreads();

  const int frag_row = lane & 31;
  const int frag_k = (lane >> 5) * 8;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load_stage((kt + 1) * kBK);
    const uint16_t *as = As + buf * BM * kLds + (wm * WM + frag_row) * kLds + frag_k;
    const uint16_t *bs = Bs + buf * BN * kLds + (wn * WN + frag_row) * kLds + frag_k;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      bf16x8 a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = *(const bf16x8 *)(as + i * 32 * kLds + ks * 16);
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j] = *(const bf16x8 *)(bs + j * 32 * kLds + ks * 16);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store_stage(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue ---------------------------------------------------------
  const int row_base = m0 + wm * WM + 4 * (lane >> 5);
  if (!GATEUP) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * WN + j * 32 + (lane & 31);
      if (n >= N) continue;
      const float s = p.scales ? p.scales[n] : 1.0f;
      const float b = p.bias ? p.bias[n] : 0.0f;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = row_base + i * 32 + 8 * (r >> 2) + (r & 3);
          if (m < M) {
            float v = epi_scale_bias(acc[i][j][r], s, b, p.scales != nullptr, p.bias != nullptr);
            v = apply_epi(p.epi, v);
            p.C[(size_t)m * p.ldc + n] = (uint16_t)f32_to_bf16_bits(v);
          }
        }
    }
  } else {
#pragma unroll
    for (int j = 0; j < TN / 2; ++j) {
      const int n = n0 + wn * (WN / 2) + j * 32 + (lane & 31);
      if (n >= N) continue;
      const float sg = p.scales[n];
      const float su = p.scales2[n];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = row_base + i * 32 + 8 * (r >> 2) + (r & 3);
          if (m < M) {
            const float g = epi_scale_bias(acc[i][j][r], sg, 0.0f, true, false);
            const float u = epi_scale_bias(acc[i][j + TN / 2][r], su, 0.0f, true, false);
            float h;
            {
#pragma clang fp contract(off)
              h = silu32(g) * u;
            }
            p.C[(size_t)m * p.ldc + n] = (uint16_t)f32_to_bf16_bits(h);
          }
        }
    }
  }
}

template <int BM, int BN, int BKIND, bool GATEUP>
static hipError_t launch_cfg(const GemmNT &p, hipStream_t stream) {
  constexpr size_t lds = gemm_nt_lds_bytes<BM, BN>();
  auto kern = gemm_nt_kernel<BM, BN, BKIND, GATEUP>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void *)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  constexpr int BN_OUT = GATEUP ? BN / 2 : BN;
  const int tiles = (int)((p.M + BM - 1) / BM) * (int)((p.N + BN_OUT - 1) / BN_OUT);
  hipLaunchKernelGGL(kern, dim3(tiles), dim3(256), lds, stream, p);
  return hipGetLastError();
}

// Picks the tile that keeps the 256 CUs busiest: the largest tile whose
// grid still covers about one full wave of workgroups.
hipError_t launch_gemm_nt(const GemmNT &p, hipStream_t stream) {
  auto tiles = [&](int bm, int bn) {
    return ((p.M + bm - 1) / bm) * ((p.N + bn - 1) / bn);
  };
  if (p.gate_up) {
    // output columns per tile are BN/2
    if (tiles(128, 128) >= 200 || p.M > 128)
      return launch_cfg<128, 256, B_INT8, true>(p, stream);
    return launch_cfg<128, 128, B_INT8, true>(p, stream);
  }
  if (p.bkind == B_BF16) {
    if (tiles(256, 256) >= 224) return launch_cfg<256, 256, B_BF16, false>(p, stream);
    if (tiles(128, 256) >= 224) return launch_cfg<128, 256, B_BF16, false>(p, stream);
    return launch_cfg<128, 128, B_BF16, false>(p, stream);
  }
  if (tiles(256, 256) >= 224) return launch_cfg<256, 256, B_INT8, false>(p, stream);
  if (tiles(128, 256) >= 224) return launch_cfg<128, 256, B_INT8, false>(p, stream);
  return launch_cfg<128, 128, B_INT8, false>(p, stream);
}

}  // namespace mj
