/*
 * momijo_oracle.c -- CPU restatement of momijo's tensor-engine hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP kernels in
 * momijo_amd/csrc are compared against.  Only tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py may load it.  The product path
 * (momijo_amd) never links or calls it.
 *
 * The reference (taleblou/momijo, legacy/) is Mojo source that cannot be built
 * in this image (no Mojo toolchain, and the hot-path files carry compile
 * errors), so every function below restates one reference function, loop
 * order and arithmetic included, and cites the file:line it follows.
 * Paths are relative to /root/reference/legacy/src/momijo/.
 *
 * Build: gcc -O2 -ffp-contract=off -fno-fast-math (see oracle/Makefile).
 * -ffp-contract=off keeps `acc = acc + a*b` as a rounded multiply followed by
 * a rounded add, i.e. no FMA contraction.  Whether Mojo contracts these is a
 * property of the Mojo compiler and is "parity unpinned" at the last ulp.
 *
 * Pinning (what checks each function; tests/test_oracle_*.py):
 *   rng            Vigna's published splitmix64 / xoroshiro128** definitions
 *                  (independent numpy restatement + committed golden words).
 *   matmul/linear  integer-valued inputs (exact in any order), identity and
 *                  permutation closed forms, fp64 brute force with the
 *                  K*2^-24*sum|a||b| bound, torch CPU as a cross-check.
 *   activations    closed forms against libm in double; _exp_approx family
 *                  against a numpy float32 restatement (exact IEEE sequence).
 *   int8           constructed ties, the fp32-add artifact (0.49999997 -> 1),
 *                  all-zero rows, clamps; int32 GEMM exact by brute force.
 *   bf16 rounding  torch's bfloat16 cast (RNE) on random and special values.
 *   fp64 engine    int64-exact products, identity/permutation, and the strict
 *                  k order against a one-rounding-per-step numpy loop.
 *   tensordot      per-batch equality with the pinned fp32 matmul, broadcast
 *                  batches against materialised copies, int64 einsum.
 * Functions with no independent check are listed as "parity unpinned" in the
 * docstring of oracle/__init__.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define MO_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* RNG: SplitMix64 + xoroshiro128**   (tensor/creation.mojo:57-131)          */
/* ------------------------------------------------------------------------ */

typedef struct { uint64_t s0, s1; } mo_rng;

/* SplitMix64.next (creation.mojo:63-68). */
static uint64_t splitmix64_next(uint64_t *state) {
    *state += 0x9E3779B97F4A7C15ull;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* rotl64 (creation.mojo:71-75): k is masked to 6 bits, k==0 returns x. */
static inline uint64_t rotl64(uint64_t x, int k) {
    unsigned kk = (unsigned)k & 63u;
    if (kk == 0) return x;
    return (x << kk) | (x >> (64u - kk));
}

/* RNG64.__init__ (creation.mojo:81-90): seed 0 is replaced by the golden
 * gamma, two splitmix outputs seed the state, all-zero state is patched. */
MO_API void mo_rng_init(mo_rng *r, uint64_t seed) {
    uint64_t s = seed ? seed : 0x9E3779B97F4A7C15ull;
    r->s0 = splitmix64_next(&s);
    r->s1 = splitmix64_next(&s);
    if ((r->s0 | r->s1) == 0) r->s1 = 0xFFFFFFFFFFFFFFFFull;
}

/* RNG64.next_u64 (creation.mojo:92-100): xoroshiro128** with (24,16,37). */
MO_API uint64_t mo_rng_next_u64(mo_rng *r) {
    uint64_t s0 = r->s0, s1 = r->s1;
    uint64_t res = rotl64(s0 * 5u, 7) * 9u;
    s1 ^= s0;
    r->s0 = rotl64(s0, 24) ^ s1 ^ (s1 << 16);
    r->s1 = rotl64(s1, 37);
    return res;
}

/* RNG64.next_f64 (creation.mojo:102-106): top 53 bits / 2^53. */
MO_API double mo_rng_next_f64(mo_rng *r) {
    return (double)(mo_rng_next_u64(r) >> 11) / 9007199254740992.0;
}

/* RNG64.next_f32 (creation.mojo:107-111): Float32(u>>11) / 2^53.  The
 * conversion of a 53-bit integer to fp32 rounds to nearest even here; Mojo's
 * conversion mode is parity unpinned. */
MO_API float mo_rng_next_f32(mo_rng *r) {
    uint64_t hi = mo_rng_next_u64(r) >> 11;
    return (float)hi / 9007199254740992.0f;
}

/* Fill `out` with n raw u64 words (for golden-vector pinning of the stream). */
MO_API void mo_rng_words(uint64_t seed, uint64_t *out, int64_t n) {
    mo_rng r; mo_rng_init(&r, seed);
    for (int64_t i = 0; i < n; ++i) out[i] = mo_rng_next_u64(&r);
}

/* Raw words from an explicit state (s0, s1), without the splitmix64 seeding:
 * for known-answer checks of the xoroshiro128** step itself. */
MO_API void mo_rng_words_from_state(uint64_t s0, uint64_t s1, uint64_t *out, int64_t n) {
    mo_rng r; r.s0 = s0; r.s1 = s1;
    for (int64_t i = 0; i < n; ++i) out[i] = mo_rng_next_u64(&r);
}

/* randu_with[Float32] (creation.mojo:495-526): f(low + (high-low)*next_f64)
 * with f = Float32(.) (tensor/cast.mojo:353-354). */
MO_API void mo_randu_f32(float *out, int64_t n, double low, double high, uint64_t seed) {
    mo_rng r; mo_rng_init(&r, seed);
    double scale = high - low;
    for (int64_t i = 0; i < n; ++i) out[i] = (float)(low + scale * mo_rng_next_f64(&r));
}

/* _randn_like_with_f64core (creation.mojo:550-578): Box-Muller in f64 with
 * u1 clamped at 1e-12, emitting z0 then z1.  The build maps each value as
 * Float32(mean + std*z) so the same stream yields N(0,1) and N(0,0.02)
 * inputs; std=1, mean=0 gives exactly Float32(z) as in the reference's map64.
 * libm log/cos/sin in double: the Mojo stdlib's are parity unpinned. */
MO_API void mo_randn_f32(float *out, int64_t n, double mean, double std, uint64_t seed) {
    mo_rng r; mo_rng_init(&r, seed);
    int64_t i = 0;
    while (i < n) {
        double u1 = mo_rng_next_f64(&r);
        double u2 = mo_rng_next_f64(&r);
        if (u1 < 1e-12) u1 = 1e-12;
        double rad = sqrt(-2.0 * log(u1));
        double theta = 6.283185307179586 * u2;
        double z0 = rad * cos(theta), z1 = rad * sin(theta);
        out[i] = (float)(mean + std * z0);
        if (i + 1 < n) out[i + 1] = (float)(mean + std * z1);
        i += 2;
    }
}

/* _randn_like_with_f32core (creation.mojo:581-611), the randn_f32 path:
 * Box-Muller carried out in fp32 (logf/cosf/sinf from libm). */
MO_API void mo_randn_f32_f32core(float *out, int64_t n, uint64_t seed) {
    mo_rng r; mo_rng_init(&r, seed);
    int64_t i = 0;
    while (i < n) {
        float u1 = mo_rng_next_f32(&r);
        float u2 = mo_rng_next_f32(&r);
        if (u1 < 1e-12f) u1 = 1e-12f;
        float rad = sqrtf(-2.0f * logf(u1));
        float theta = 6.283185307179586f * u2;
        out[i] = rad * cosf(theta);
        if (i + 1 < n) out[i + 1] = rad * sinf(theta);
        i += 2;
    }
}

/* ------------------------------------------------------------------------ */
/* bf16 <-> fp32 (round to nearest even; NaN stays a quiet NaN)             */
/* ------------------------------------------------------------------------ */

MO_API uint16_t mo_f32_to_bf16(float f) {
    uint32_t u; memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7FFFu + lsb;
    return (uint16_t)(u >> 16);
}

MO_API float mo_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16; float f; memcpy(&f, &u, 4); return f;
}

MO_API void mo_f32_to_bf16_n(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = mo_f32_to_bf16(x[i]);
}

MO_API void mo_bf16_to_f32_n(const uint16_t *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = mo_bf16_to_f32(x[i]);
}

/* ------------------------------------------------------------------------ */
/* fp32 matmul   (tensor/broadcast.mojo:1543-1684)                          */
/* ------------------------------------------------------------------------ */

/* matmul_core_mm (broadcast.mojo:1612-1673).  C[i,j] = sum_k A[i,k]*B[k,j]
 * with an fp32 accumulator that starts at 0 and adds the products in strict
 * ascending k (the unroll-by-8 of both paths keeps that order).  The
 * contiguous fast path (:1620-1645) and the strided path (:1647-1673) give
 * the same sums; both are kept so the CPU baseline times the loop the
 * reference runs.  Operands are (data, strides) with offset 0: the reference
 * ignores _offset on both paths.  C is row-major [M,N]. */
MO_API void mo_matmul_f32(const float *A, int64_t sAm, int64_t sAk,
                          const float *B, int64_t sBk, int64_t sBn,
                          float *C, int64_t M, int64_t N, int64_t K) {
    if (sAm == K && sAk == 1 && sBk == N && sBn == 1) {
        for (int64_t i = 0; i < M; ++i) {
            const float *a = A + i * K;
            for (int64_t j = 0; j < N; ++j) {
                float acc = 0.0f;
                int64_t k = 0, lim = (K / 8) * 8;
                for (; k < lim; k += 8) {
                    acc = acc + a[k + 0] * B[(k + 0) * N + j];
                    acc = acc + a[k + 1] * B[(k + 1) * N + j];
                    acc = acc + a[k + 2] * B[(k + 2) * N + j];
                    acc = acc + a[k + 3] * B[(k + 3) * N + j];
                    acc = acc + a[k + 4] * B[(k + 4) * N + j];
                    acc = acc + a[k + 5] * B[(k + 5) * N + j];
                    acc = acc + a[k + 6] * B[(k + 6) * N + j];
                    acc = acc + a[k + 7] * B[(k + 7) * N + j];
                }
                for (; k < K; ++k) acc = acc + a[k] * B[k * N + j];
                C[i * N + j] = acc;
            }
        }
        return;
    }
    for (int64_t i = 0; i < M; ++i) {
        const float *a = A + i * sAm;
        for (int64_t j = 0; j < N; ++j) {
            const float *b = B + j * sBn;
            float acc = 0.0f;
            for (int64_t k = 0; k < K; ++k) acc = acc + a[k * sAk] * b[k * sBk];
            C[i * N + j] = acc;
        }
    }
}

/* matmul_core_vec (broadcast.mojo:1543-1608): y[i] = sum_j A[i,j]*x[j],
 * strict ascending j. */
MO_API void mo_matvec_f32(const float *A, int64_t sAm, int64_t sAn,
                          const float *x, int64_t sx, float *y, int64_t M, int64_t N) {
    for (int64_t i = 0; i < M; ++i) {
        float acc = 0.0f;
        for (int64_t j = 0; j < N; ++j) acc = acc + A[i * sAm + j * sAn] * x[j * sx];
        y[i] = acc;
    }
}

/* Linear.forward_cpu_parallel (learn/nn/layers.mojo:383-433).  W is
 * [OutF,InF] row-major; y[n,o] = (sum_k x[n,k]*W[o,k]) + b[o]: the dot runs
 * in strict k order (unrolled 8/4/1 without reordering) and the bias is added
 * once after the sum (:426-427), only when has_bias and b has OutF entries. */
MO_API void mo_linear_fw_f32(const float *x, const float *W, const float *b, int has_bias,
                             float *y, int64_t N, int64_t InF, int64_t OutF) {
    for (int64_t n = 0; n < N; ++n) {
        const float *xr = x + n * InF;
        for (int64_t o = 0; o < OutF; ++o) {
            const float *wr = W + o * InF;
            float acc = 0.0f;
            for (int64_t k = 0; k < InF; ++k) acc = acc + xr[k] * wr[k];
            if (has_bias && b) acc = acc + b[o];
            y[n * OutF + o] = acc;
        }
    }
}

/* Linear._kernel_linear_fw (layers.mojo:436-475): the CPU-fallback kernel of
 * the device seam launch_1d_linear_fw (tensor/gpu/runtime.mojo:539-631).  It
 * takes wT as [InF,OutF] and reads wT[k*OutF+o]; one call per output tid. */
MO_API void mo_kernel_linear_fw_f32(const float *x, const float *wT, const float *b, int has_bias,
                                    float *y, int64_t N, int64_t InF, int64_t OutF) {
    int64_t total = N * OutF;
    for (int64_t tid = 0; tid < total; ++tid) {
        int64_t n = tid / OutF, o = tid - n * OutF;
        float acc = 0.0f;
        for (int64_t k = 0; k < InF; ++k) acc = acc + x[n * InF + k] * wT[k * OutF + o];
        if (has_bias && b) acc = acc + b[o];
        y[n * OutF + o] = acc;
    }
}

/* ------------------------------------------------------------------------ */
/* activations                                                              */
/* ------------------------------------------------------------------------ */

/* ReLU.forward -> _maximum_scalar(x, 0) (layers.mojo:117-137):
 * v if v > 0 else 0  (NaN -> 0, -0 -> +0). */
MO_API float mo_relu_layer32(float v) { return v > 0.0f ? v : 0.0f; }

/* Tensor.relu -> apply_unary op 8 (tensor/math.mojo:582-585):
 * if v < 0: v = 0  (NaN stays NaN, -0 stays -0). */
MO_API float mo_relu_unary32(float v) { return v < 0.0f ? 0.0f : v; }

/* Tensor[Float32].maximum_scalar(s) = where_f32(ge_t(self, s), self, s)
 * (tensor/tensor.mojo:4232): the mask x >= s picks x, else s (NaN >= s is
 * false; -0 >= 0 is true, so -0 stays). */
MO_API void mo_maximum_scalar32_n(const float *x, float s, float *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = x[i] >= s ? x[i] : s;
}

/* astype_f32_from_int (tensor/cast.mojo:5431-5437): flat.append(Float32(v))
 * for each Int of the storage in order; the C conversion of a 64-bit integer
 * rounds to nearest even under the default rounding mode. */
MO_API void mo_astype_f32_from_int(const int64_t *x, float *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = (float)x[i];
}

/* sigmoid32 / tanh32 / silu32 / gelu32 (tensor/math.mojo:272-295) with
 * exp32 = stdlib exp on Float32 (math.mojo:490).  tanh32 is the literal
 * (e^{2t}-1)/(e^{2t}+1), which is NaN once e^{2t} overflows (t > ~44.36,
 * reached by gelu32 at x > ~10.06). */
MO_API float mo_sigmoid32(float x) { return 1.0f / (1.0f + expf(-x)); }
MO_API float mo_tanh32(float x) {
    float e2x = expf(2.0f * x);
    return (e2x - 1.0f) / (e2x + 1.0f);
}
MO_API float mo_silu32(float x) { return x * mo_sigmoid32(x); }
MO_API float mo_gelu32(float x) {
    const float k = 0.7978845608028654f, c = 0.044715f;
    float x3 = x * x * x;
    float t = k * (x + c * x3);
    return 0.5f * x * (1.0f + mo_tanh32(t));
}

/* The epilogue's GELU: gelu32 wherever gelu32 is finite; where the literal
 * tanh32 overflows to inf/inf the intended value tanh(t) = 1 is used (the
 * reference's result there is NaN, tensor/math.mojo:277-279). */
MO_API float mo_gelu32_finite(float x) {
    const float k = 0.7978845608028654f, c = 0.044715f;
    float x3 = x * x * x;
    float t = k * (x + c * x3);
    float e2x = expf(2.0f * t);
    float th = isinf(e2x) ? 1.0f : (e2x - 1.0f) / (e2x + 1.0f);
    return 0.5f * x * (1.0f + th);
}

/* learn.nn.activations family (learn/nn/activations.mojo:34-51,137-163):
 * _exp_approx(x) = (1 + clamp(x,-20,20)/64)^64 by six squarings,
 * _tanh_approx clamps to +-10 first. */
static inline float clampf_(float v, float lo, float hi) {
    if (v < lo) v = lo;
    if (v > hi) v = hi;
    return v;
}
MO_API float mo_exp_approx32(float x) {
    float xv = clampf_(x, -20.0f, 20.0f);
    float y = 1.0f + xv / 64.0f;
    y = y * y; y = y * y; y = y * y; y = y * y; y = y * y; y = y * y;
    return y;
}
MO_API float mo_tanh_approx32(float x) {
    float xv = clampf_(x, -10.0f, 10.0f);
    float e2x = mo_exp_approx32(2.0f * xv);
    return (e2x - 1.0f) / (e2x + 1.0f);
}
MO_API float mo_sigmoid_approx32(float x) { return 1.0f / (1.0f + mo_exp_approx32(-x)); }
MO_API float mo_silu_approx32(float x) { return x * mo_sigmoid_approx32(x); }
MO_API float mo_gelu_approx32(float x) {
    const float s = 0.7978845608028654f;
    float x3 = x * x * x;
    float inner = s * (x + 0.044715f * x3);
    return 0.5f * x * (1.0f + mo_tanh_approx32(inner));
}

/* Epilogue selector shared with include/momijo_hip.h (MJ_EPI_*). */
enum { EPI_NONE = 0, EPI_RELU = 1, EPI_GELU_TANH = 2, EPI_SILU = 3,
       EPI_GELU_TANH_APPROX = 4, EPI_SILU_APPROX = 5, EPI_RELU_UNARY = 6 };

MO_API float mo_epilogue32(int epi, float v) {
    switch (epi) {
    case EPI_RELU: return mo_relu_layer32(v);
    case EPI_GELU_TANH: return mo_gelu32_finite(v);
    case EPI_SILU: return mo_silu32(v);
    case EPI_GELU_TANH_APPROX: return mo_gelu_approx32(v);
    case EPI_SILU_APPROX: return mo_silu_approx32(v);
    case EPI_RELU_UNARY: return mo_relu_unary32(v);
    default: return v;
    }
}

MO_API void mo_epilogue32_n(int epi, const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = mo_epilogue32(epi, x[i]);
}

/* apply_unary_impl32 op 17 / 18 literal (tensor/math.mojo:602-626), used to
 * show the NaN of gelu32 past x ~ 10.06. */
MO_API void mo_gelu32_n(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = mo_gelu32(x[i]);
}

/* Linear + epilogue: the composition Linear.forward then the activation
 * (ReLU.forward, Tensor.gelu, Tensor.silu) on the fp32 result. */
MO_API void mo_linear_act_f32(const float *x, const float *W, const float *b, int has_bias,
                              int epi, float *y, int64_t N, int64_t InF, int64_t OutF) {
    mo_linear_fw_f32(x, W, b, has_bias, y, N, InF, OutF);
    for (int64_t i = 0; i < N * OutF; ++i) y[i] = mo_epilogue32(epi, y[i]);
}

/* ------------------------------------------------------------------------ */
/* int8 helpers  (learn/api/functional.mojo:206-302)                        */
/* ------------------------------------------------------------------------ */

/* _round_to_i32 (functional.mojo:214-217) then _clamp_int8 (:208-212).
 * v + 0.5 is an fp32 add (so 0.49999997f rounds to 1), then the cast
 * truncates toward zero.  Values outside the int8 range clamp; the float is
 * clamped before the cast, which equals cast-then-clamp for every finite v.
 * NaN maps to 0 (Mojo's Int32(NaN) is parity unpinned). */
MO_API int8_t mo_quant_legacy_one(float x, float scale) {
    float v = x / scale;
    float adj = v >= 0.0f ? 0.5f : -0.5f;
    float t = v + adj;
    if (t != t) return 0;
    if (t >= 127.0f) return 127;
    if (t <= -128.0f) return -128;
    return (int8_t)(int32_t)t;
}

/* quantize_symmetric_int8 (functional.mojo:231-247): per-tensor scale, with
 * scale 0 replaced by 1. */
MO_API void mo_quantize_symmetric_int8(const float *x, int64_t n, float s, int8_t *q) {
    float scale = (s == 0.0f) ? 1.0f : s;
    for (int64_t i = 0; i < n; ++i) q[i] = mo_quant_legacy_one(x[i], scale);
}

/* matmul_i8_i8_to_i32 (functional.mojo:249-279).  Intended semantics:
 * C[i,j] = sum_p int32(A[i,p]) * int32(B[j,p]) with B = w_q [N,K] (NT).
 * legacy_literal=1 reproduces the reference literally: QuantLinear passes the
 * zero-copy view w_q.transpose() and the kernel reads bt._data[p*N + j],
 * ignoring strides (:274), i.e. B is taken as reshape(w_q.flat, [K,N]). */
MO_API void mo_matmul_i8_i8_to_i32(const int8_t *A, const int8_t *B, int32_t *C,
                                   int64_t M, int64_t N, int64_t K, int legacy_literal) {
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            int32_t acc = 0;
            for (int64_t p = 0; p < K; ++p) {
                int8_t b = legacy_literal ? B[p * N + j] : B[j * K + p];
                acc += (int32_t)A[i * K + p] * (int32_t)b;
            }
            C[i * N + j] = acc;
        }
}

/* dequantize_i32_to_f32_add_bias (functional.mojo:281-302):
 * y = Float32(acc) * sf + b[j], a rounded multiply then a rounded add. */
MO_API void mo_dequant_i32_bias(const int32_t *acc, float sf, const float *b, float *y,
                                int64_t M, int64_t N) {
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            float v = (float)acc[i * N + j] * sf;
            y[i * N + j] = v + b[j];
        }
}

/* Per-channel (and per-row) form of dequantize_i32_to_f32_add_bias
 * (learn/api/functional.mojo:281-302): y = float(acc) * (sx[m] * sw[n]) + b[n],
 * sx * sw rounded first; sx NULL means the factor sw[n], b NULL no add
 * (spec-only: the reference has the scalar-sf form above). */
MO_API void mo_dequant_i32_scaled(const int32_t *acc, const float *sx, const float *sw,
                                  const float *b, float *y, int64_t M, int64_t N) {
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            const float sf = sx ? sx[i] * sw[j] : sw[j];
            float v = (float)acc[i * N + j] * sf;
            if (b) v = v + b[j];
            y[i * N + j] = v;
        }
}

/* MinMaxObserver.observe + scale_symmetric (learn/api/sequential.mojo:
 * 232-263): min/max over the data, scale = max(|min|,|max|)/max_q, 1.0 when
 * there is no data, max_q <= 0 or the magnitude is 0. */
MO_API float mo_minmax_scale_symmetric(const float *x, int64_t n, float max_q) {
    if (n <= 0 || max_q <= 0.0f) return 1.0f;
    float mn = x[0], mx = x[0];
    for (int64_t i = 0; i < n; ++i) {
        float v = x[i];
        if (v < mn) mn = v;
        if (v > mx) mx = v;
    }
    float a = mn < 0.0f ? -mn : mn;
    float b = mx < 0.0f ? -mx : mx;
    float m = a;
    if (b > m) m = b;
    if (m <= 0.0f) return 1.0f;
    return m / max_q;
}

/* QuantLinear.forward (learn/nn/layers.mojo:1681-1685): quantize x with s_x,
 * int8 GEMM against w_q^T, dequantize with sf = s_x*s_w, add bias. */
MO_API void mo_quant_linear_fw(const float *x, const int8_t *Wq, const float *b,
                               float s_w, float s_x, float *y, int32_t *acc_scratch,
                               int8_t *xq_scratch, int64_t M, int64_t N, int64_t K,
                               int legacy_literal) {
    mo_quantize_symmetric_int8(x, M * K, s_x, xq_scratch);
    mo_matmul_i8_i8_to_i32(xq_scratch, Wq, acc_scratch, M, N, K, legacy_literal);
    float sf = s_x * s_w;
    mo_dequant_i32_bias(acc_scratch, sf, b, y, M, N);
}

/* ------------------------------------------------------------------------ */
/* Spec-only int8 weight path (no reference code: per-output-channel,       */
/* round-half-even, weight-only).  The guard conventions follow the         */
/* reference's (scale 1.0 for an all-zero row, as functional.mojo:235-236  */
/* and sequential.mojo:252-263 do for a zero scale).                        */
/* ------------------------------------------------------------------------ */

/* scale[n] = max_k |W[n,k]| / 127 (fp32 division); q = clamp(rne(W/scale),
 * -127, 127).  rintf rounds half to even in the default FP environment.
 * NaN weights do not enter the absmax (a > m is false) and quantize to 0. */
MO_API void mo_quantize_rowwise_rhe(const float *W, int64_t N, int64_t K, int8_t *Q, float *scales) {
    for (int64_t n = 0; n < N; ++n) {
        const float *w = W + n * K;
        float m = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            float a = fabsf(w[k]);
            if (a > m) m = a;
        }
        float s = m / 127.0f;
        if (s == 0.0f) s = 1.0f;
        scales[n] = s;
        for (int64_t k = 0; k < K; ++k) {
            float v = rintf(w[k] / s);
            if (v != v) v = 0.0f;
            if (v > 127.0f) v = 127.0f;
            if (v < -127.0f) v = -127.0f;
            Q[n * K + k] = (int8_t)v;
        }
    }
}

/* Per-row variant of the legacy rule (round half away via the fp32 +-0.5 add,
 * clamp to [-128,127]) with a per-row MinMax scale. */
MO_API void mo_quantize_rowwise_legacy(const float *W, int64_t N, int64_t K, int8_t *Q, float *scales) {
    for (int64_t n = 0; n < N; ++n) {
        float s = mo_minmax_scale_symmetric(W + n * K, K, 127.0f);
        scales[n] = s;
        for (int64_t k = 0; k < K; ++k) Q[n * K + k] = mo_quant_legacy_one(W[n * K + k], s);
    }
}

/* W8A16 Linear: y[m,n] = bf16(act((sum_k f32(x[m,k]) * f32(q[n,k])) *
 * scale[n] + b[n])).  The dot runs in strict k order in fp32 (the exact
 * products x*q need at most 15 significant bits); bias may be NULL. */
MO_API void mo_linear_w8a16(const uint16_t *x, const int8_t *Q, const float *scales,
                            const float *b, int epi, uint16_t *y, float *y_f32,
                            int64_t M, int64_t N, int64_t K) {
    for (int64_t m = 0; m < M; ++m) {
        const uint16_t *xr = x + m * K;
        for (int64_t n = 0; n < N; ++n) {
            const int8_t *q = Q + n * K;
            float acc = 0.0f;
            for (int64_t k = 0; k < K; ++k) acc = acc + mo_bf16_to_f32(xr[k]) * (float)q[k];
            float v = acc * scales[n];
            if (b) v = v + b[n];
            v = mo_epilogue32(epi, v);
            if (y_f32) y_f32[m * N + n] = v;
            if (y) y[m * N + n] = mo_f32_to_bf16(v);
        }
    }
}

/* W8A8 Linear with dynamic activation scales (spec-only: the per-row /
 * per-channel generalisation of QuantLinear.forward, learn/nn/layers.mojo:
 * 1681-1685, whose quantize / int8 matmul / dequantize + bias steps it keeps):
 *   row m of x upcast to fp32 (exact) and quantized by the RHE rule of
 *   mo_quantize_rowwise_rhe -> xq[m,:], sx[m];
 *   acc = sum_k xq[m,k] * Q[n,k] (exact integer sum);
 *   v = (float)acc * (sx[m] * scales[n]); v = v + b[n]; y = bf16(act(v)),
 * every fp32 operation rounded on its own.  Rows [m0, m1); xq_out / sx_out
 * (optional) receive those rows' quantized x and scales. */
MO_API void mo_linear_w8a8(const uint16_t *x, const int8_t *Q, const float *scales,
                           const float *b, int epi, uint16_t *y, float *y_f32, int8_t *xq_out,
                           float *sx_out, int64_t N, int64_t K, int64_t m0, int64_t m1) {
    float *row = (float *)malloc((size_t)K * sizeof(float));
    int8_t *q = (int8_t *)malloc((size_t)K);
    if (!row || !q) { free(row); free(q); return; }
    for (int64_t m = m0; m < m1; ++m) {
        for (int64_t k = 0; k < K; ++k) row[k] = mo_bf16_to_f32(x[m * K + k]);
        float sx;
        mo_quantize_rowwise_rhe(row, 1, K, q, &sx);
        if (xq_out) memcpy(xq_out + (m - m0) * K, q, (size_t)K);
        if (sx_out) sx_out[m - m0] = sx;
        for (int64_t n = 0; n < N; ++n) {
            const int8_t *w = Q + n * K;
            int64_t acc = 0;
            for (int64_t k = 0; k < K; ++k) acc += (int64_t)q[k] * (int64_t)w[k];
            const float sf = sx * scales[n];
            float v = (float)(int32_t)acc * sf;
            if (b) v = v + b[n];
            v = mo_epilogue32(epi, v);
            if (y_f32) y_f32[(m - m0) * N + n] = v;
            if (y) y[(m - m0) * N + n] = mo_f32_to_bf16(v);
        }
    }
    free(row);
    free(q);
}

/* bf16 NT GEMM reference: momijo has no bf16 matmul (tensor/broadcast.mojo
 * has f64 and f32 overloads only, :1531,1677), so the oracle is the fp32
 * engine's strict-k dot on exactly upcast bf16 inputs, plus bias and the
 * epilogue, rounded RNE to bf16.  A [M,K], B [N,K] (the Linear weight
 * layout).  Rows [m0, m1) only, so large shapes can be checked on a slab. */
MO_API void mo_gemm_bf16_nt(const uint16_t *A, const uint16_t *B, const float *bias, int epi,
                            uint16_t *C, float *C_f32, int64_t M, int64_t N, int64_t K,
                            int64_t m0, int64_t m1) {
    (void)M;
    for (int64_t m = m0; m < m1; ++m) {
        const uint16_t *a = A + m * K;
        for (int64_t n = 0; n < N; ++n) {
            const uint16_t *bb = B + n * K;
            float acc = 0.0f;
            for (int64_t k = 0; k < K; ++k) acc = acc + mo_bf16_to_f32(a[k]) * mo_bf16_to_f32(bb[k]);
            if (bias) acc = acc + bias[n];
            acc = mo_epilogue32(epi, acc);
            if (C_f32) C_f32[(m - m0) * N + n] = acc;
            if (C) C[(m - m0) * N + n] = mo_f32_to_bf16(acc);
        }
    }
}

/* Llama-style FFN (no reference op; composed from Linear, silu32 and the
 * elementwise product, tensor/tensor.mojo:4373):
 *   g = x Wg^T * sg, u = x Wu^T * su   (W8A16 dots in fp32),
 *   h = bf16(silu32(g) * u),  y = bf16((h Wd^T) * sd).
 * Rows [m0, m1) of x only; h_out (optional) receives those rows of h. */
MO_API void mo_mlp_w8a16(const uint16_t *x, const int8_t *Wg, const float *sg,
                         const int8_t *Wu, const float *su, const int8_t *Wd, const float *sd,
                         uint16_t *h_out, uint16_t *y, int64_t K, int64_t I, int64_t H,
                         int64_t m0, int64_t m1, uint16_t *h_row_scratch) {
    for (int64_t m = m0; m < m1; ++m) {
        const uint16_t *xr = x + m * K;
        for (int64_t i = 0; i < I; ++i) {
            float g = 0.0f, u = 0.0f;
            const int8_t *wg = Wg + i * K, *wu = Wu + i * K;
            for (int64_t k = 0; k < K; ++k) g = g + mo_bf16_to_f32(xr[k]) * (float)wg[k];
            for (int64_t k = 0; k < K; ++k) u = u + mo_bf16_to_f32(xr[k]) * (float)wu[k];
            g = g * sg[i];
            u = u * su[i];
            h_row_scratch[i] = mo_f32_to_bf16(mo_silu32(g) * u);
        }
        if (h_out) memcpy(h_out + (m - m0) * I, h_row_scratch, (size_t)I * 2);
        for (int64_t n = 0; n < H; ++n) {
            const int8_t *wd = Wd + n * I;
            float acc = 0.0f;
            for (int64_t i = 0; i < I; ++i) acc = acc + mo_bf16_to_f32(h_row_scratch[i]) * (float)wd[i];
            y[(m - m0) * H + n] = mo_f32_to_bf16(acc * sd[n]);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* fp64 matmul (tensor/broadcast.mojo:1397-1538) and matmul2d               */
/* (tensor/math.mojo:7838-7880)                                             */
/* ------------------------------------------------------------------------ */

/* matmul_core_mm f64 (broadcast.mojo:1460-1527): the f32 algorithm in fp64,
 * strict ascending k, both the contiguous and the strided path. */
MO_API void mo_matmul_f64(const double *A, int64_t sAm, int64_t sAk,
                          const double *B, int64_t sBk, int64_t sBn,
                          double *C, int64_t M, int64_t N, int64_t K) {
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k) acc = acc + A[i * sAm + k * sAk] * B[k * sBk + j * sBn];
            C[i * N + j] = acc;
        }
}

/* matmul_core_vec f64 (broadcast.mojo:1397-1457). */
MO_API void mo_matvec_f64(const double *A, int64_t sAm, int64_t sAn,
                          const double *x, int64_t sx, double *y, int64_t M, int64_t N) {
    for (int64_t i = 0; i < M; ++i) {
        double acc = 0.0;
        for (int64_t j = 0; j < N; ++j) acc = acc + A[i * sAm + j * sAn] * x[j * sx];
        y[i] = acc;
    }
}

/* tensordot f32, axes = 1 (broadcast.mojo:1694-1900): out[b, i, j] =
 * sum_k A[b, i, k] * B[b, k, j] over the broadcast batch index b, strict
 * ascending k.  The batch is given flattened: for each of nb output batches
 * the caller passes the element offsets of its A and B matrices. */
MO_API void mo_tensordot_f32(const float *A, const int64_t *a_off, int64_t sAm, int64_t sAk,
                             const float *B, const int64_t *b_off, int64_t sBk, int64_t sBn,
                             float *C, int64_t nb, int64_t M, int64_t N, int64_t K) {
    for (int64_t b = 0; b < nb; ++b)
        for (int64_t i = 0; i < M; ++i)
            for (int64_t j = 0; j < N; ++j) {
                float acc = 0.0f;
                for (int64_t k = 0; k < K; ++k)
                    acc = acc + A[a_off[b] + i * sAm + k * sAk] * B[b_off[b] + k * sBk + j * sBn];
                C[(b * M + i) * N + j] = acc;
            }
}

/* Linear.backward_cpu_parallel (learn/nn/layers.mojo:519-618): for
 * x [N,InF], W [OutF,InF] and dy [N,OutF],
 *   db[o]   = sum_n dy[n,o]                     (ascending n, :545-553)
 *   dx[n,i] = sum_o dy[n,o] * W[o,i]            (ascending o, :555-583)
 *   dW[o,i] = sum_n dy[n,o] * x[n,i]            (ascending n, :585-611)
 * each a single fp32 accumulator; the 8- and 4-wide unrolls keep the order.
 * A NULL output is skipped. */
MO_API void mo_linear_backward_f32(const float *x, const float *W, const float *dy, float *dW,
                                   float *db, float *dx, int64_t N, int64_t InF, int64_t OutF) {
    if (db)
        for (int64_t o = 0; o < OutF; ++o) {
            float s = 0.0f;
            for (int64_t n = 0; n < N; ++n) s = s + dy[n * OutF + o];
            db[o] = s;
        }
    if (dx)
        for (int64_t n = 0; n < N; ++n)
            for (int64_t i = 0; i < InF; ++i) {
                float acc = 0.0f;
                for (int64_t o = 0; o < OutF; ++o) acc = acc + dy[n * OutF + o] * W[o * InF + i];
                dx[n * InF + i] = acc;
            }
    if (dW)
        for (int64_t o = 0; o < OutF; ++o)
            for (int64_t i = 0; i < InF; ++i) {
                float acc = 0.0f;
                for (int64_t n = 0; n < N; ++n) acc = acc + dy[n * OutF + o] * x[n * InF + i];
                dW[o * InF + i] = acc;
            }
}

/* The MATMUL2D rule of the autograd tape (tensor/autograd.mojo:1542-1555) for
 * y = a @ b with a [M,K], b [K,N] and upstream gradient g [M,N], Float64:
 *   ga = matmul2d(g, b^T)  -> grads[a] = grads[a] + ga   (da [M,K])
 *   gb = matmul2d(a^T, g)  -> grads[b] = grads[b] + gb   (db [K,N])
 * matmul2d sums in ascending inner index (tensor/math.mojo:7864-7871); with
 * accumulate = 0 the gradients are overwritten instead of added to (a fresh
 * tape holds zeros there, which gives the same values).  A NULL output is
 * skipped. */
MO_API void mo_matmul_backward_f64(const double *a, const double *b, const double *g, double *da,
                                   double *db, int64_t M, int64_t N, int64_t K, int accumulate) {
    if (da)
        for (int64_t i = 0; i < M; ++i)
            for (int64_t k = 0; k < K; ++k) {
                double acc = 0.0;
                for (int64_t j = 0; j < N; ++j) acc = acc + g[i * N + j] * b[k * N + j];
                da[i * K + k] = accumulate ? da[i * K + k] + acc : acc;
            }
    if (db)
        for (int64_t k = 0; k < K; ++k)
            for (int64_t j = 0; j < N; ++j) {
                double acc = 0.0;
                for (int64_t i = 0; i < M; ++i) acc = acc + a[i * K + k] * g[i * N + j];
                db[k * N + j] = accumulate ? db[k * N + j] + acc : acc;
            }
}

/* The MATMUL2D tape rule with Float32 values and gradients (the tape's type,
 * tensor/autograd.mojo:214-216; rule :1542-1555): ga = g_out @ b^T and
 * gb = a^T @ g_out as the Float32 matmul computes them (matmul_core_mm,
 * tensor/broadcast.mojo:1620-1645: strict ascending inner index, one rounding
 * per multiply and per add), then grads[p] = grads[p].add(g): one rounding
 * of old + g. */
MO_API void mo_matmul_backward_f32(const float *a, const float *b, const float *g, float *da,
                                   float *db, int64_t M, int64_t N, int64_t K, int accumulate) {
    if (da)
        for (int64_t i = 0; i < M; ++i)
            for (int64_t k = 0; k < K; ++k) {
                float acc = 0.0f;
                for (int64_t j = 0; j < N; ++j) acc = acc + g[i * N + j] * b[k * N + j];
                da[i * K + k] = accumulate ? da[i * K + k] + acc : acc;
            }
    if (db)
        for (int64_t k = 0; k < K; ++k)
            for (int64_t j = 0; j < N; ++j) {
                float acc = 0.0f;
                for (int64_t i = 0; i < M; ++i) acc = acc + a[i * K + k] * g[i * N + j];
                db[k * N + j] = accumulate ? db[k * N + j] + acc : acc;
            }
}

/* ------------------------------------------------------------------------ */
/* conv2d                                                                   */
/* ------------------------------------------------------------------------ */

/* Conv2d.forward, NCHW, as Conv2d._kernel_conv2d_fwd computes each output
 * (learn/nn/conv.mojo:600-681; the same arithmetic as forward_cpu_parallel,
 * :494-597, and the GPU kernel _gpu_conv2d_fw_kernel,
 * tensor/gpu/runtime.mojo:159-200): for output (n, oc, oy, ox) the window
 * is clipped to the input (ky in [ky_start, ky_end), kx likewise: padded taps
 * are skipped, not multiplied by zero), sum = 0 then sum = sum + x * w over
 * ic, ky, kx in ascending order (one rounding per multiply and per add), and
 * the bias is added after the sum.  x [N,C,H,W], w [OC,C,kH,kW], b [OC] or
 * NULL, y [N,OC,OH,OW]; images n0 .. n1 - 1 only (y indexed from image n0). */
MO_API void mo_conv2d_fw_f32(const float *x, const float *w, const float *b, float *y, int64_t N,
                             int64_t C, int64_t H, int64_t W, int64_t OC, int64_t kH,
                             int64_t kW, int64_t sH, int64_t sW, int64_t pH, int64_t pW,
                             int64_t OH, int64_t OW, int64_t n0, int64_t n1) {
    (void)N;
    const int64_t HW = H * W, CHW = C * HW, kHW = kH * kW, CkHW = C * kHW;
    for (int64_t n = n0; n < n1; ++n)
        for (int64_t oc = 0; oc < OC; ++oc)
            for (int64_t oy = 0; oy < OH; ++oy) {
                const int64_t iy0 = oy * sH - pH;
                const int64_t ky_start = iy0 < 0 ? -iy0 : 0;
                int64_t ky_end = kH;
                if (iy0 + kH > H) ky_end = kH - (iy0 + kH - H);
                for (int64_t ox = 0; ox < OW; ++ox) {
                    const int64_t ix0 = ox * sW - pW;
                    const int64_t kx_start = ix0 < 0 ? -ix0 : 0;
                    int64_t kx_end = kW;
                    if (ix0 + kW > W) kx_end = kW - (ix0 + kW - W);
                    float sum = 0.0f;
                    for (int64_t ic = 0; ic < C; ++ic)
                        for (int64_t ky = ky_start; ky < ky_end; ++ky)
                            for (int64_t kx = kx_start; kx < kx_end; ++kx) {
                                const float xv = x[n * CHW + ic * HW + (iy0 + ky) * W + ix0 + kx];
                                const float wv = w[oc * CkHW + ic * kHW + ky * kW + kx];
                                sum = sum + xv * wv;
                            }
                    if (b) sum = sum + b[oc];
                    y[(((n - n0) * OC + oc) * OH + oy) * OW + ox] = sum;
                }
            }
}
