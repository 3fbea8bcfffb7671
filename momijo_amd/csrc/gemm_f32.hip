// fp32 / fp64 engine on gfx950: the matmul / Linear / tensordot of momijo's
// Float32 and Float64 tensor engine (tensor/broadcast.mojo:1397-1900,
// tensor/math.mojo:7838-7880, learn/nn/layers.mojo:383-433).
//
// gemm_fx_kernel<T, TB>: C = epi(A @ B + bias) on v_mfma_f32_16x16x4f32 (T =
// float, full fp32 products) or v_mfma_f64_16x16x4f64 (T = double), a TB x TB
// tile per 256-thread workgroup (64; 128 for problems with enough tiles, where
// each wave then runs 4 x 4 MFMA blocks per LDS fragment read instead of
// 2 x 2; 32 for tiny latency-bound problems, one block per wave; the 128 and
// 64 tiles run eight waves, two per SIMD, of TB/2 x TB/4), K stages
// staged through LDS (k-major, padded; 16 deep, 64 (fp32) or 32 (fp64) on the
// 32 x 32 tiles).  Neither the tile size nor the stage depth changes any
// output's summation order.  Tiny fp32 products whose operands are both
// k-contiguous skip LDS (gemm_f32_direct_kernel, same MFMA sequence).  Operands come as (pointer, row stride, column stride), which
// covers the reference's zero-copy transpose views; the loader walks
// whichever dimension has unit stride with consecutive lanes so global reads
// stay coalesced.  A grid dimension over broadcast batch indices serves
// tensordot's batched paths.
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace mj {

constexpr int kFBK = 16;

typedef __attribute__((__vector_size__(4 * sizeof(double)))) double f64x4;

template <typename T> struct Acc;
// Both instructions read A[i][k] from lane i + 16 k and B[k][j] from lane
// j + 16 k.  Accumulator item r of lane l holds column l % 16 and row
// 4 (l / 16) + r for fp32, but row 4 r + l / 16 for fp64.
template <> struct Acc<float> {
  typedef f32x4 V;
  static __device__ __forceinline__ V mfma(float a, float b, V c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ int row(int lane, int r) { return 4 * (lane >> 4) + r; }
};
template <> struct Acc<double> {
  typedef f64x4 V;
  static __device__ __forceinline__ V mfma(double a, double b, V c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ int row(int lane, int r) { return 4 * r + (lane >> 4); }
};

// Implicit-GEMM view of an NCHW conv2d (the CONV instantiations): B[k][p] of
// a batch (image) is x[c][iy][ix] with k = (c kH + ky) kW + kx (the flattened
// weight index of w[oc][c][ky][kx]), p = oy OW + ox, iy = oy sH - pH + ky,
// ix = ox sW - pW + kx, and zero where (iy, ix) lies outside the H x W image;
// the bias is per output row (channel).  One K stage of BK advances (c, ky,
// kx) by (dc, dky, dkx) with BK = (dc kH + dky) kW + dkx.
struct ConvDesc {
  int H = 0, W = 0, OW = 0, kH = 1, kW = 1, sH = 1, sW = 1, pH = 0, pW = 0;
  int dc = 0, dky = 0, dkx = 0;
};

// One (batch, 64 x 64 tile) per workgroup: C[b] = epi(A[b] @ B[b] + bias),
// or with accum set C[b] = C[b] + A[b] @ B[b] (gradient accumulation: the old
// value plus the finished product, one rounding).
// The batch index (batch0 + blockIdx.y) is decomposed over up to 5 broadcast
// batch dimensions into element offsets of A and B; C is contiguous per batch.
// CONV: B is the image gathered by cv (above) instead of a strided view.
template <typename T, int TB, int BK = kFBK, bool CONV = false, int NW = 4>
__global__ __launch_bounds__(NW * 64) void gemm_fx_kernel(int M, int N, int K, const T *__restrict__ A,
                                                      int64_t sAm, int64_t sAk,
                                                      const T *__restrict__ B, int64_t sBk,
                                                      int64_t sBn, const T *__restrict__ bias,
                                                      int epi, int accum, T *__restrict__ C,
                                                      int64_t ldc, BatchDesc bd, int64_t batch0,
                                                      ConvDesc cv) {
  constexpr int kFBM = TB, kFBN = TB;
  constexpr int NT = NW * 64;
  constexpr int WGN = NW / 2;        // waves 2 x WGN
  constexpr int NBM = TB / 32;       // 16 x 16 blocks per wave along M
  constexpr int NBN = TB / (16 * WGN);  // and along N
  constexpr int EPT = TB * BK / NT;  // elements of each operand per thread per stage
  constexpr int MF = NT / TB;        // m-fast / n-fast loader: k rows per pass
  constexpr int KF = NT / BK;        // k-fast loader: m (n) columns per pass
  static_assert(EPT >= 1 && BK % 4 == 0 && NBN >= 1, "stage shape");
  __shared__ T As[2][BK][kFBM + 4];
  __shared__ T Bs[2][BK][kFBN + 4];

  {
    const int64_t bi = batch0 + blockIdx.y;
    int64_t b = bi, oa = 0, ob = 0;
    for (int d = bd.rank - 1; d >= 0; --d) {
      const int64_t i = b % bd.shape[d];
      b /= bd.shape[d];
      oa += i * bd.a_stride[d];
      ob += i * bd.b_stride[d];
    }
    A += oa;
    B += ob;
    C += bi * M * ldc;
  }

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int tiles_n = (N + kFBN - 1) / kFBN;
  const int m0 = (blockIdx.x / tiles_n) * kFBM;
  const int n0 = (blockIdx.x % tiles_n) * kFBN;

  const bool a_k_fast = (sAk == 1);
  const bool b_n_fast = CONV || (sBn == 1) || (sBk != 1);

  // CONV: a thread's output pixel p = n0 + tid % TB is fixed; element i of
  // its B loads walks k = k0 + tid / TB + MF i, kept as (c, ky, kx) and
  // advanced by one stage after each load
  int cy0 = 0, cx0 = 0, cc[EPT], cky[EPT], ckx[EPT];
  bool cp_ok = false;
  if constexpr (CONV) {
    const int pix = n0 + tid % TB;
    cp_ok = pix < N;
    const int oy = cp_ok ? pix / cv.OW : 0;
    cy0 = oy * cv.sH - cv.pH;
    cx0 = (pix - oy * cv.OW) * cv.sW - cv.pW;
    const int khw = cv.kH * cv.kW;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int k = tid / TB + MF * i;
      cc[i] = k / khw;
      cky[i] = (k - cc[i] * khw) / cv.kW;
      ckx[i] = k - cc[i] * khw - cky[i] * cv.kW;
    }
  }

  T ra[EPT], rb[EPT];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      int m, k;
      if (a_k_fast) { k = tid % BK; m = tid / BK + KF * i; }
      else          { m = tid % TB; k = tid / TB + MF * i; }
      const int gm = m0 + m, gk = k0 + k;
      ra[i] = (gm < M && gk < K) ? A[(int64_t)gm * sAm + (int64_t)gk * sAk] : T(0);
    }
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      if constexpr (CONV) {
        const int iy = cy0 + cky[i], ix = cx0 + ckx[i];
        const bool in = cp_ok && k0 + tid / TB + MF * i < K && (unsigned)iy < (unsigned)cv.H &&
                        (unsigned)ix < (unsigned)cv.W;
        rb[i] = in ? B[((int64_t)cc[i] * cv.H + iy) * cv.W + ix] : T(0);
        // advance (c, ky, kx) by BK: each digit carries at most once
        ckx[i] += cv.dkx;
        const int cx = ckx[i] >= cv.kW;
        ckx[i] -= cx ? cv.kW : 0;
        cky[i] += cv.dky + cx;
        const int cyc = cky[i] >= cv.kH;
        cky[i] -= cyc ? cv.kH : 0;
        cc[i] += cv.dc + cyc;
      } else {
        int n, k;
        if (b_n_fast) { n = tid % TB; k = tid / TB + MF * i; }
        else          { k = tid % BK; n = tid / BK + KF * i; }
        const int gn = n0 + n, gk = k0 + k;
        rb[i] = (gn < N && gk < K) ? B[(int64_t)gk * sBk + (int64_t)gn * sBn] : T(0);
      }
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      int m, k;
      if (a_k_fast) { k = tid % BK; m = tid / BK + KF * i; }
      else          { m = tid % TB; k = tid / TB + MF * i; }
      As[buf][k][m] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      int n, k;
      if (b_n_fast) { n = tid % TB; k = tid / TB + MF * i; }
      else          { k = tid % BK; n = tid / BK + KF * i; }
      Bs[buf][k][n] = rb[i];
    }
  };

  typename Acc<T>::V acc[NBM][NBN];
#pragma unroll
  for (int i = 0; i < NBM; ++i)
#pragma unroll
    for (int j = 0; j < NBN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = T(0);

  const int nk = (K + BK - 1) / BK;
  load(0);
  store(0);
  __syncthreads();
  const int fr = lane & 15, fk = lane >> 4;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load((kt + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 4) {
      T a[NBM], b[NBN];
#pragma unroll
      for (int i = 0; i < NBM; ++i) a[i] = As[buf][kk + fk][wm * (TB / 2) + i * 16 + fr];
#pragma unroll
      for (int j = 0; j < NBN; ++j) b[j] = Bs[buf][kk + fk][wn * (TB / WGN) + j * 16 + fr];
#pragma unroll
      for (int i = 0; i < NBM; ++i)
#pragma unroll
        for (int j = 0; j < NBN; ++j) acc[i][j] = Acc<T>::mfma(a[i], b[j], acc[i][j]);
    }
    if (kt + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < NBN; ++j) {
    const int n = n0 + wn * (TB / WGN) + j * 16 + (lane & 15);
    if (n >= N) continue;
    const T bb = (bias && !CONV) ? bias[n] : T(0);
#pragma unroll
    for (int i = 0; i < NBM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * (TB / 2) + i * 16 + Acc<T>::row(lane, r);
        if (m < M) {
          T v = acc[i][j][r];
          if (bias) {
#pragma clang fp contract(off)
            v = v + (CONV ? bias[m] : bb);
          }
          if constexpr (sizeof(T) == sizeof(float)) v = apply_epi(epi, v);  // fp64: none
          T *dst = C + (int64_t)m * ldc + n;
          if (accum) {
#pragma clang fp contract(off)
            v = *dst + v;
          }
          *dst = v;
        }
      }
  }
}

// 16 x 16 outputs per 64-thread workgroup for tiny fp32 products whose
// operands are both k-contiguous (x . W^T: the Linear forward, and matmul
// with a transposed right operand), without LDS: lane l = fr + 16 j loads
// A[fr][16 u + 4 j .. + 3] and B^T[fr][16 u + 4 j .. + 3] of each 16-deep
// chunk u as one 16-byte load, and a 4 x 4 transpose across the four 16-lane
// rows (two v_permlane32_swap, then two v_permlane16_swap) leaves in register
// c of lane fr + 16 j the element k = 16 u + 4 c + j, the operand that the
// MFMA t = 4 u + c takes from that lane.  So the outputs see the MFMA
// sequence of gemm_fx_kernel in the same k order, bit for bit (chunks past K
// are zero, as the staged kernel's padding is).  Loads run two batches of CB
// chunks ahead of the MFMAs; needs K % 4 == 0 and 16-byte aligned rows.
__device__ __forceinline__ void transpose4_rows(f32x4 &v) {
  const auto s0 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[0]), __float_as_uint(v[2]),
                                                   false, false);
  const auto s1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[1]), __float_as_uint(v[3]),
                                                   false, false);
  const auto t0 = __builtin_amdgcn_permlane16_swap(s0[0], s1[0], false, false);
  const auto t1 = __builtin_amdgcn_permlane16_swap(s0[1], s1[1], false, false);
  v = f32x4{__uint_as_float(t0[0]), __uint_as_float(t0[1]), __uint_as_float(t1[0]),
            __uint_as_float(t1[1])};
}

template <int CB>
__global__ __launch_bounds__(64) void gemm_f32_direct_kernel(int M, int N, int K,
                                                             const float *__restrict__ A,
                                                             int64_t sAm,
                                                             const float *__restrict__ Bt,
                                                             int64_t sBn,
                                                             const float *__restrict__ bias,
                                                             int epi, float *__restrict__ C,
                                                             int64_t ldc) {
  const int lane = threadIdx.x;
  const int fr = lane & 15, j = lane >> 4;
  const int tiles_n = (N + 15) / 16;
  const int m0 = (blockIdx.x / tiles_n) * 16, n0 = (blockIdx.x % tiles_n) * 16;
  const bool am = m0 + fr < M, bn = n0 + fr < N;
  const float *pa = A + (am ? (int64_t)(m0 + fr) * sAm : 0) + 4 * j;
  const float *pb = Bt + (bn ? (int64_t)(n0 + fr) * sBn : 0) + 4 * j;
  const int nc = (K + 15) / 16;
  f32x4 xa[CB], xb[CB], ya[CB], yb[CB];
  auto load = [&](f32x4 (&ra)[CB], f32x4 (&rb)[CB], int c0) {
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      const bool ok = (c0 + c) * 16 + 4 * j < K;  // K % 4 == 0: wholly in or out
      ra[c] = am && ok ? *(const f32x4 *)(pa + (int64_t)(c0 + c) * 16) : f32x4{0.f, 0.f, 0.f, 0.f};
      rb[c] = bn && ok ? *(const f32x4 *)(pb + (int64_t)(c0 + c) * 16) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  auto compute = [&](f32x4 (&ra)[CB], f32x4 (&rb)[CB], int c0) {
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      if (c0 + c >= nc) break;
      transpose4_rows(ra[c]);
      transpose4_rows(rb[c]);
#pragma unroll
      for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ra[c][q], rb[c][q], acc, 0, 0, 0);
    }
  };
  load(xa, xb, 0);
  for (int c0 = 0;;) {
    if (c0 + CB < nc) load(ya, yb, c0 + CB);
    compute(xa, xb, c0);
    c0 += CB;
    if (c0 >= nc) break;
    if (c0 + CB < nc) load(xa, xb, c0 + CB);
    compute(ya, yb, c0);
    c0 += CB;
    if (c0 >= nc) break;
  }
  const int n = n0 + fr;
  if (!bn) return;
  const float bb = bias ? bias[n] : 0.0f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = m0 + Acc<float>::row(lane, r);
    if (m < M) {
      float v = acc[r];
      if (bias) {
#pragma clang fp contract(off)
        v = v + bb;
      }
      C[(int64_t)m * ldc + n] = apply_epi(epi, v);
    }
  }
}

// K per stage of the 32 x 32 tiles: each stage costs a global-load round
// trip that its MFMAs (BK / 4 per wave) cannot cover, so the latency-bound
// tiny problems take deep stages (fp32: 64, 37 KB of LDS; fp64: 32, the
// static LDS limit); per output the k order is the same at any depth
template <typename T>
constexpr int kTinyBK = sizeof(T) == 4 ? 64 : 32;

template <typename T>
static hipError_t launch_fx(int64_t M, int64_t N, int64_t K, const T *A, int64_t sAm,
                            int64_t sAk, const T *B, int64_t sBk, int64_t sBn, const T *bias,
                            int epi, int accum, T *C, int64_t ldc, const BatchDesc &bd,
                            int64_t batches, hipStream_t stream) {
  // 128 x 128 tiles for matrices of at least 256 x 256 once they still give
  // every CU two workgroups; problems of fewer than 64 tiles of 64 x 64 take
  // 32 x 32 tiles (a latency-bound launch: a quarter of the MFMA chain per
  // wave and four times the workgroups; 256^3 Linear 17.4 -> 8.4 us); the
  // rest 64 x 64
  const int64_t tiles128 = ((M + 127) / 128) * ((N + 127) / 128);
  const bool big = M >= 256 && N >= 256 && tiles128 * batches >= 512;
  const bool tiny = !big && ((M + 63) / 64) * ((N + 63) / 64) * batches < 64;
  if constexpr (sizeof(T) == sizeof(float)) {
    const bool direct = tiny && batches == 1 && bd.rank == 0 && !accum && sAk == 1 && sBk == 1 &&
                        K % 4 == 0 && (M == 1 || sAm % 4 == 0) && (N == 1 || sBn % 4 == 0) &&
                        (((uintptr_t)A | (uintptr_t)B) & 15) == 0;
    if (direct) {
      const int64_t tiles16 = ((M + 15) / 16) * ((N + 15) / 16);
      hipLaunchKernelGGL(gemm_f32_direct_kernel<8>, dim3((unsigned)tiles16), dim3(64), 0, stream,
                         (int)M, (int)N, (int)K, A, sAm, B, sBn, bias, epi, C, ldc);
      return hipGetLastError();
    }
  }
  const int TBs = big ? 128 : (tiny ? 32 : 64);
  const int64_t tiles64 = ((M + TBs - 1) / TBs) * ((N + TBs - 1) / TBs);
  if (tiles64 > INT32_MAX) return hipErrorInvalidValue;  // grid.x limit
  const int tiles = (int)tiles64;
  constexpr int64_t kMaxGridY = 65535;
  for (int64_t b0 = 0; b0 < batches; b0 += kMaxGridY) {
    const int64_t nb = batches - b0 < kMaxGridY ? batches - b0 : kMaxGridY;
    // eight waves (two per SIMD) on the 128 x 128 and 64 x 64 tiles, four on
    // the tiny 32 x 32 ones (measured on MI355X against four waves on the same
    // tiles: fp32 Linear.backward 4096 2857 -> 2694 us, fp32 2048^3 220 ->
    // 207 us, 1536^3 130 -> 119 us, fp64 4096^3 3293 -> 2657 us, fp64 2048^3
    // 411 -> 326 us)
    if (big)
      hipLaunchKernelGGL((gemm_fx_kernel<T, 128, kFBK, false, 8>), dim3(tiles, (unsigned)nb),
                         dim3(512), 0, stream, (int)M, (int)N, (int)K, A, sAm, sAk, B, sBk, sBn,
                         bias, epi, accum, C, ldc, bd, b0, ConvDesc{});
    else if (tiny)
      hipLaunchKernelGGL((gemm_fx_kernel<T, 32, kTinyBK<T>>), dim3(tiles, (unsigned)nb),
                         dim3(256), 0, stream, (int)M, (int)N, (int)K, A, sAm, sAk, B, sBk, sBn,
                         bias, epi, accum, C, ldc, bd, b0, ConvDesc{});
    else
      hipLaunchKernelGGL((gemm_fx_kernel<T, 64, kFBK, false, 8>), dim3(tiles, (unsigned)nb),
                         dim3(512), 0, stream, (int)M, (int)N, (int)K, A, sAm, sAk, B, sBk, sBn,
                         bias, epi, accum, C, ldc, bd, b0, ConvDesc{});
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_gemm_f32(int64_t M, int64_t N, int64_t K, const float *A, int64_t sAm,
                           int64_t sAk, const float *B, int64_t sBk, int64_t sBn,
                           const float *bias, int epi, float *C, int64_t ldc,
                           hipStream_t stream) {
  return launch_fx<float>(M, N, K, A, sAm, sAk, B, sBk, sBn, bias, epi, 0, C, ldc, BatchDesc{},
                          1, stream);
}

hipError_t launch_gemm_f32_accum(int64_t M, int64_t N, int64_t K, const float *A, int64_t sAm,
                                 int64_t sAk, const float *B, int64_t sBk, int64_t sBn, float *C,
                                 int64_t ldc, int accum, hipStream_t stream) {
  return launch_fx<float>(M, N, K, A, sAm, sAk, B, sBk, sBn, nullptr, 0, accum, C, ldc,
                          BatchDesc{}, 1, stream);
}

hipError_t launch_gemm_f32_batched(int64_t M, int64_t N, int64_t K, const float *A, int64_t sAm,
                                   int64_t sAk, const float *B, int64_t sBk, int64_t sBn,
                                   float *C, const BatchDesc &bd, int64_t batches,
                                   hipStream_t stream) {
  return launch_fx<float>(M, N, K, A, sAm, sAk, B, sBk, sBn, nullptr, 0, 0, C, N, bd, batches,
                          stream);
}

hipError_t launch_gemm_f64(int64_t M, int64_t N, int64_t K, const double *A, int64_t sAm,
                           int64_t sAk, const double *B, int64_t sBk, int64_t sBn, double *C,
                           int64_t ldc, int accum, hipStream_t stream) {
  return launch_fx<double>(M, N, K, A, sAm, sAk, B, sBk, sBn, nullptr, 0, accum, C, ldc,
                           BatchDesc{}, 1, stream);
}

// Conv2d.forward with OC >= 64 (conv2d_fx_kernel<NBN>): 64 x TBN tiles of
// (output channel, output pixel of one image), TBN = 32 NBN, eight waves
// 4 x 2 of 16 x 16 NBN, 16-deep K stages through LDS, with the MFMA of
// gemm_fx_kernel in the same k order (k ascending by 4, lane group fk
// supplying k = 4 t + fk): the outputs are bit-identical to it.
// The gather: thread t owns pixel n0 + t % 256 of the tile (t % 256 < TBN)
// and loads 8 k of each stage, waves 0-3 the first 8, waves 4-7 the last 8.
// Element k = (c kH + ky) kW + kx sits at (pixel base) + c H W + ky W + kx in
// the image, pixel base = (oy sH - pH) W + ox sW - pW; the (c, ky, kx) walk
// is the same for every lane of a wave (scalar registers), and an out-of-range
// buffer offset (a tap in the padding, k >= K, a pixel past the image) loads
// zero.  Two stages are in flight in registers while one multiplies from LDS.
// The LDS rows are padded to 16 mod 32 words, so the fragment reads of four
// consecutive k rows (16 lanes each) hit distinct banks.  Against one wave
// per SIMD (four waves of 32 x 16 NBN) the eight waves ran the bench layer
// (32 x 64 x 56 x 56, 3 x 3, pad 1) 116.5 us against 126.8 (MI355X, same
// tile).  Needs C H W and OC C kH kW below 2^29 (32-bit byte offsets).
template <int NBN>
__global__ __launch_bounds__(512) void conv2d_fx_kernel(int M, int Ng, int K,
                                                        const float *__restrict__ w,
                                                        const float *__restrict__ x,
                                                        const float *__restrict__ bias, int epi,
                                                        float *__restrict__ y, int64_t img0,
                                                        int C, ConvDesc cv) {
  constexpr int TBM = 64, TBN = 32 * NBN, BK = 16;
  constexpr int LDA = TBM + 16, LDB = TBN + 16;
  __shared__ float As[2][BK][LDA];
  __shared__ float Bs[2][BK][LDB];
  const int64_t img = img0 + blockIdx.y;
  const int hw = cv.H * cv.W;
  const int64_t chw = (int64_t)C * hw;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + img * chw, chw * 4);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (int64_t)M * K * 4);
  y += img * (int64_t)M * Ng;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_n = (Ng + TBN - 1) / TBN;
  const int m0 = (blockIdx.x / tiles_n) * TBM;
  const int n0 = (blockIdx.x % tiles_n) * TBN;

  const int kg = wave >> 2;      // k group of the B gather (wave-uniform)
  const int px = tid & 255;
  int iy0 = -(1 << 28), ix0 = 0, pbase = 0;
  if (px < TBN && n0 + px < Ng) {
    const int pix = n0 + px;
    const int oy = pix / cv.OW;
    iy0 = oy * cv.sH - cv.pH;
    ix0 = (pix - oy * cv.OW) * cv.sW - cv.pW;
    pbase = iy0 * cv.W + ix0;
  }
  // walk state: the (c, ky, kx) of k = 8 kg of the next stage to load
  const int khw = cv.kH * cv.kW;
  int wc = (8 * kg) / khw;
  int wky = (8 * kg - wc * khw) / cv.kW;
  int wkx = 8 * kg - wc * khw - wky * cv.kW;
  const int ak = tid & 15, am = tid >> 4;

  float ra[2][2], rb[2][8];
  auto step = [&]() {
    if (++wkx == cv.kW) {
      wkx = 0;
      if (++wky == cv.kH) {
        wky = 0;
        ++wc;
      }
    }
  };
  auto load = [&](int k0, auto slot_c) {
    constexpr int SL = decltype(slot_c)::value;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int m = m0 + am + 32 * i, k = k0 + ak;
      const uint32_t off = (m < M && k < K) ? (uint32_t)(m * K + k) * 4u : kOobOffset;
      ra[SL][i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rw, off, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int iy = iy0 + wky, ix = ix0 + wkx;
      const bool in = (unsigned)iy < (unsigned)cv.H && (unsigned)ix < (unsigned)cv.W &&
                      k0 + 8 * kg + i < K;
      const uint32_t off = in ? (uint32_t)(pbase + wc * hw + wky * cv.W + wkx) * 4u : kOobOffset;
      rb[SL][i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rx, off, 0, 0));
      step();
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) step();
  };
  auto store = [&](int buf, auto slot_c) {
    constexpr int SL = decltype(slot_c)::value;
#pragma unroll
    for (int i = 0; i < 2; ++i) As[buf][ak][am + 32 * i] = ra[SL][i];
    if (px < TBN) {
#pragma unroll
      for (int i = 0; i < 8; ++i) Bs[buf][8 * kg + i][px] = rb[SL][i];
    }
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;

  f32x4 acc[NBN];
#pragma unroll
  for (int j = 0; j < NBN; ++j) acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const int nk = (K + BK - 1) / BK;
  const int fr = lane & 15, fk = lane >> 4;
  auto mma = [&](int buf) {
#pragma unroll
    for (int kk = 0; kk < BK; kk += 4) {
      const float a = As[buf][kk + fk][wm * 16 + fr];
      float b[NBN];
#pragma unroll
      for (int j = 0; j < NBN; ++j) b[j] = Bs[buf][kk + fk][wn * 16 * NBN + j * 16 + fr];
#pragma unroll
      for (int j = 0; j < NBN; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b[j], acc[j], 0, 0, 0);
    }
  };
  load(0, S0());
  if (nk > 1) load(BK, S1());
  store(0, S0());
  __syncthreads();
  int kt = 0;
  for (; kt + 1 < nk; kt += 2) {
    if (kt + 2 < nk) load((kt + 2) * BK, S0());
    mma(0);
    store(1, S1());
    __syncthreads();
    if (kt + 3 < nk) load((kt + 3) * BK, S1());
    mma(1);
    if (kt + 2 < nk) store(0, S0());
    __syncthreads();
  }
  if (kt < nk) mma(0);

#pragma unroll
  for (int j = 0; j < NBN; ++j) {
    const int n = n0 + wn * 16 * NBN + j * 16 + fr;
    if (n >= Ng) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + wm * 16 + 4 * fk + r;
      if (m < M) {
        float v = acc[j][r];
        if (bias) {
#pragma clang fp contract(off)
          v = v + bias[m];
        }
        y[(int64_t)m * Ng + n] = apply_epi(epi, v);
      }
    }
  }
}

// Conv2d.forward (NCHW) as one implicit GEMM per image: y[n] [OC, OH OW] =
// w [OC, C kH kW] @ im2col(x[n]) [C kH kW, OH OW] + b[oc], the image index
// on the grid's second dimension: conv2d_fx_kernel's 64 x 224 or 64 x 256
// tiles when they apply (below), else the matmul engine's square tiles as
// the matmul picks them (64 x 64, 128 x 128 for large problems, 32 x 32 for
// tiny ones).  Both sum each output in the same k order.
hipError_t launch_conv2d_f32(const float *x, const float *w, const float *b, float *y, int64_t N,
                             int64_t C, int64_t H, int64_t W, int64_t OC, int64_t kH,
                             int64_t kW, int64_t sH, int64_t sW, int64_t pH, int64_t pW,
                             int64_t OH, int64_t OW, int epi, hipStream_t stream) {
  const int64_t M = OC, Ng = OH * OW, K = C * kH * kW;
  constexpr int64_t kMaxGridY = 65535;
  ConvDesc cv;
  cv.H = (int)H; cv.W = (int)W; cv.OW = (int)OW; cv.kH = (int)kH; cv.kW = (int)kW;
  cv.sH = (int)sH; cv.sW = (int)sW; cv.pH = (int)pH; cv.pW = (int)pW;
  // OC >= 64 and a grid of at least 192 workgroups: conv2d_fx_kernel with
  // 224- or 256-pixel tiles, whichever leaves fewer pixel columns on the
  // busiest CU (workgroups of all images dealt over 256 CUs; 256 on a tie).
  // Against the square tiles below (eight waves), MI355X: 32 x 64 x 56^2 ->
  // 64 (448 workgroups) 126 against 145 us, 16 x 64 x 56^2 -> 64 (224) 79.5
  // against 87.5, but 8 x 64 x 56^2 -> 64 (112) 74.5 against 49.1 and
  // 16 x 128 x 28^2 -> 128 (128) 139 against 90.  Narrower tiles of that
  // kernel were slower than the square ones (128 pixels: 158.6 us on the
  // bench layer).
  if (M >= 64 && C * H * W < ((int64_t)1 << 29) && M * K < ((int64_t)1 << 29)) {
    int nbn = 0;
    int64_t best = INT64_MAX, wgs_best = 0;
    for (int c : {8, 7}) {
      const int64_t tbn = 32 * c;
      const int64_t wgs = ((M + 63) / 64) * ((Ng + tbn - 1) / tbn) * N;
      const int64_t cost = (wgs + 255) / 256 * tbn;
      if (cost < best) {
        best = cost;
        nbn = c;
        wgs_best = wgs;
      }
    }
    if (wgs_best >= 192) {
      const int64_t tiles_c = ((M + 63) / 64) * ((Ng + 32 * nbn - 1) / (32 * nbn));
      if (tiles_c > INT32_MAX) return hipErrorInvalidValue;
      for (int64_t b0 = 0; b0 < N; b0 += kMaxGridY) {
        const int64_t nb = N - b0 < kMaxGridY ? N - b0 : kMaxGridY;
        const dim3 g((unsigned)tiles_c, (unsigned)nb);
        if (nbn == 8)
          hipLaunchKernelGGL((conv2d_fx_kernel<8>), g, dim3(512), 0, stream, (int)M, (int)Ng,
                             (int)K, w, x, b, epi, y, b0, (int)C, cv);
        else
          hipLaunchKernelGGL((conv2d_fx_kernel<7>), g, dim3(512), 0, stream, (int)M, (int)Ng,
                             (int)K, w, x, b, epi, y, b0, (int)C, cv);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
      }
      return hipSuccess;
    }
  }
  BatchDesc bd;
  bd.rank = 1;
  bd.shape[0] = N;
  bd.a_stride[0] = 0;
  bd.b_stride[0] = C * H * W;
  const int64_t tiles128 = ((M + 127) / 128) * ((Ng + 127) / 128);
  const bool big = M >= 256 && Ng >= 256 && tiles128 * N >= 512;
  const bool tiny = !big && ((M + 63) / 64) * ((Ng + 63) / 64) * N < 64;
  const int TBs = big ? 128 : (tiny ? 32 : 64);
  const int BKs = tiny ? kTinyBK<float> : kFBK;
  cv.dc = (int)(BKs / (kH * kW));
  cv.dky = (int)((BKs % (kH * kW)) / kW);
  cv.dkx = (int)(BKs % kW);
  const int64_t tiles64 = ((M + TBs - 1) / TBs) * ((Ng + TBs - 1) / TBs);
  if (tiles64 > INT32_MAX) return hipErrorInvalidValue;
  const int tiles = (int)tiles64;
  for (int64_t b0 = 0; b0 < N; b0 += kMaxGridY) {
    const int64_t nb = N - b0 < kMaxGridY ? N - b0 : kMaxGridY;
    // eight waves on the 128 and 64 tiles, as the matmul (against four:
    // 8 x 32 x 40^2 -> 96 32.4 -> 28.5 us, 4 x 64 x 56^2 -> 64 42.4 -> 32.6,
    // 16 x 128 x 28^2 -> 128 102 -> 90, 8 x 256 x 14^2 -> 256 144 -> 107,
    // 32 x 3 x 224^2 -> 32 (7 x 7, stride 2) 149 -> 143 us on MI355X)
    if (big)
      hipLaunchKernelGGL((gemm_fx_kernel<float, 128, kFBK, true, 8>), dim3(tiles, (unsigned)nb),
                         dim3(512), 0, stream, (int)M, (int)Ng, (int)K, w, K, (int64_t)1, x,
                         (int64_t)0, (int64_t)1, b, epi, 0, y, Ng, bd, b0, cv);
    else if (tiny)
      hipLaunchKernelGGL((gemm_fx_kernel<float, 32, kTinyBK<float>, true>),
                         dim3(tiles, (unsigned)nb), dim3(256), 0, stream, (int)M, (int)Ng, (int)K,
                         w, K, (int64_t)1, x, (int64_t)0, (int64_t)1, b, epi, 0, y, Ng, bd, b0,
                         cv);
    else
      hipLaunchKernelGGL((gemm_fx_kernel<float, 64, kFBK, true, 8>), dim3(tiles, (unsigned)nb),
                         dim3(512), 0, stream, (int)M, (int)Ng, (int)K, w, K, (int64_t)1, x,
                         (int64_t)0, (int64_t)1, b, epi, 0, y, Ng, bd, b0, cv);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// Column sums s[o] = sum_n X[n, o] of a row-major [N, OutF] matrix, in
// ascending n within each of `segs` consecutive row segments; a second pass
// adds the segment sums in segment order.  With segs = 1 the order is the
// strict ascending-n order of the reference's db loop.  One thread per
// column: consecutive lanes read consecutive columns of a row.
__global__ __launch_bounds__(256) void colsum_seg_kernel(const float *__restrict__ X, int64_t N,
                                                         int64_t OutF, int64_t seg_len,
                                                         float *__restrict__ out) {
  const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (o >= OutF) return;
  const int64_t n0 = (int64_t)blockIdx.y * seg_len;
  const int64_t n1 = n0 + seg_len < N ? n0 + seg_len : N;
  const float *p = X + o;
  float s = 0.0f;
  int64_t n = n0;
  for (; n + 8 <= n1; n += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = p[(n + u) * OutF];
#pragma unroll
    for (int u = 0; u < 8; ++u) s = s + v[u];
  }
  for (; n < n1; ++n) s = s + p[n * OutF];
  out[(int64_t)blockIdx.y * OutF + o] = s;
}

__global__ __launch_bounds__(256) void colsum_combine_kernel(const float *__restrict__ part,
                                                             int64_t segs, int64_t OutF,
                                                             float *__restrict__ out) {
  const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (o >= OutF) return;
  const float *p = part + o;
  float s = 0.0f;
  int64_t k = 0;
  for (; k + 8 <= segs; k += 8) {  // loads in flight together, adds in order
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = p[(k + u) * OutF];
#pragma unroll
    for (int u = 0; u < 8; ++u) s = s + v[u];
  }
  for (; k < segs; ++k) s = s + p[k * OutF];
  out[o] = s;
}

int64_t colsum_segments(int64_t N, int64_t OutF) {
  const int64_t col_blocks = (OutF + 255) / 256;
  if (N <= 1024 || col_blocks >= 1024) return 1;
  int64_t segs = (1024 + col_blocks - 1) / col_blocks;  // ~1024 workgroups in all
  const int64_t max_segs = (N + 63) / 64;              // at least 64 rows per segment
  if (segs > max_segs) segs = max_segs;
  if (segs > 65535) segs = 65535;
  return segs;
}

hipError_t launch_colsum_f32(const float *X, int64_t N, int64_t OutF, float *out, float *part,
                             int64_t segs, hipStream_t stream) {
  const unsigned cb = (unsigned)((OutF + 255) / 256);
  if (segs <= 1) {
    hipLaunchKernelGGL(colsum_seg_kernel, dim3(cb, 1), dim3(256), 0, stream, X, N, OutF, N, out);
    return hipGetLastError();
  }
  const int64_t seg_len = (N + segs - 1) / segs;
  hipLaunchKernelGGL(colsum_seg_kernel, dim3(cb, (unsigned)segs), dim3(256), 0, stream, X, N,
                     OutF, seg_len, part);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(colsum_combine_kernel, dim3(cb), dim3(256), 0, stream, part, segs, OutF,
                     out);
  return hipGetLastError();
}

// y[m] = sum_n A[m,n] x[n]: one wave per row, lanes stride over n.
template <typename T>
__global__ __launch_bounds__(256) void matvec_kernel(int M, int N, const T *__restrict__ A,
                                                     int64_t sAm, int64_t sAn,
                                                     const T *__restrict__ x, int64_t sx,
                                                     T *__restrict__ y) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const T *a = A + (int64_t)row * sAm;
  T acc = T(0);
  for (int n = lane; n < N; n += 64) acc += a[(int64_t)n * sAn] * x[(int64_t)n * sx];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) y[row] = acc;
}

hipError_t launch_matvec_f32(int64_t M, int64_t N, const float *A, int64_t sAm, int64_t sAn,
                             const float *x, int64_t sx, float *y, hipStream_t stream) {
  hipLaunchKernelGGL(matvec_kernel<float>, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, stream,
                     (int)M, (int)N, A, sAm, sAn, x, sx, y);
  return hipGetLastError();
}

hipError_t launch_matvec_f64(int64_t M, int64_t N, const double *A, int64_t sAm, int64_t sAn,
                             const double *x, int64_t sx, double *y, hipStream_t stream) {
  hipLaunchKernelGGL(matvec_kernel<double>, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, stream,
                     (int)M, (int)N, A, sAm, sAn, x, sx, y);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void activation_f32_kernel(int epi, const float *x, float *y,
                                                             int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = apply_epi(epi, x[i]);
}

hipError_t launch_activation_f32(int epi, const float *x, float *y, int64_t n,
                                 hipStream_t stream) {
  int64_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(activation_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, epi,
                     x, y, n);
  return hipGetLastError();
}

// Tensor[Float32].maximum_scalar(s) = where(x >= s, x, s)
// (tensor/tensor.mojo:4232): x itself where x >= s (so -0 stays -0 at s = 0),
// else s (NaN >= s is false, so NaN gives s).
__global__ __launch_bounds__(256) void maximum_scalar_f32_kernel(const float *x, float s, float *y,
                                                                 int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float v = x[i];
    y[i] = v >= s ? v : s;
  }
}

hipError_t launch_maximum_scalar_f32(const float *x, float s, float *y, int64_t n,
                                     hipStream_t stream) {
  int64_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(maximum_scalar_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, x,
                     s, y, n);
  return hipGetLastError();
}

// astype_f32_from_int (tensor/cast.mojo:5431-5437): Float32(Int) of each
// 64-bit element, rounded to nearest even (the conversion rounds once, from
// the exact integer).
__global__ __launch_bounds__(256) void cast_i64_f32_kernel(const int64_t *x, float *y, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = (float)x[i];
}

hipError_t launch_cast_i64_f32(const int64_t *x, float *y, int64_t n, hipStream_t stream) {
  int64_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(cast_i64_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, x, y, n);
  return hipGetLastError();
}

}  // namespace mj
