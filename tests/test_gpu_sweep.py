"""Seeded shape sweeps of the GEMM planners against the oracle, bit for bit.

Each family draws its shapes from a fixed seed, spread over the ranges where
the planners switch kernels: M from 1 (GEMVs) through the skinny-M GEMV
(M <= 16) to multi-tile GEMMs, N and K ragged against every tile, stage and
K-split boundary, with and without bias.  The operands make every sum exact
(small integers, power-of-two scales) or the path is exact by construction
(int8 sums, W8A8's integer GEMM and fixed epilogue order), so whichever tile,
split or pipeline the planner picks, the output must equal the oracle's.
The FFN family is checked to the bf16 bar (its SiLU is not exact).  Problem
sizes are capped so the oracle's scalar loops stay at a fraction of a
second per case.
"""
import os
import time

import numpy as np
import pytest

import momijo_amd as mj
from _util import bf16_dev, bf16_host_bits, bf16_host_f32, normwise_rel, to_dev

pytestmark = pytest.mark.gpu

_MAC_CAP = 2.0e8


def _draw_m(rng):
    """M spread over the GEMV, skinny-GEMV and tile ranges."""
    band = rng.integers(0, 4)
    if band == 0:
        return 1
    if band == 1:
        return int(rng.integers(2, 17))
    if band == 2:
        return int(rng.integers(17, 300))
    return int(rng.integers(300, 2200))


def _cap(M, N, K, step, n_first):
    """Shrink N, then K (kept a multiple of step), or K first, until
    M * N * K fits the cap; shrinking N first keeps long K loops (and the
    K splits of few-tile problems) in the sweep."""
    def shrink_n(N, K):
        while M * N * K > _MAC_CAP and N > 16:
            N = max(16, N // 2)
        return N, K

    def shrink_k(N, K):
        while M * N * K > _MAC_CAP and K > step:
            K = max(step, (K // 2) // step * step)
        return N, K

    N, K = shrink_n(*shrink_k(N, K)) if not n_first else shrink_k(*shrink_n(N, K))
    while M * N * K > _MAC_CAP and N > 1:
        N = max(1, N // 2)
    return N, K


def _shapes(seed, count, kstep, kmax, nmax):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        M = _draw_m(rng)
        N = int(rng.integers(1, nmax + 1))
        K = int(rng.integers(1, kmax // kstep + 1)) * kstep
        N, K = _cap(M, N, K, kstep, bool(rng.integers(0, 2)))
        out.append((M, N, K, bool(rng.integers(0, 2)), int(rng.integers(0, 2))))
    return out


_W8A16 = _shapes(101, 48, 16, 8192, 6000)
_BF16 = _shapes(202, 32, 8, 4096, 3000)
_I8 = _shapes(303, 24, 1, 3000, 2500)
_W8A8 = _shapes(404, 24, 16, 6144, 3000)


def _mlp_shapes(seed, count):
    """(M, K, I, H) with K, I multiples of 16 and M (2 I K + H I) capped."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        M = _draw_m(rng)
        K = int(rng.integers(1, 257)) * 16
        I = int(rng.integers(1, 257)) * 16
        H = int(rng.integers(1, 3001))
        while M * (2 * I * K + H * I) > _MAC_CAP and max(K, I) > 16:
            if K >= I:
                K = max(16, (K // 2) // 16 * 16)
            else:
                I = max(16, (I // 2) // 16 * 16)
        while M * (2 * I * K + H * I) > _MAC_CAP and H > 1:
            H = max(1, H // 2)
        out.append((M, K, I, H))
    return out


def _f32_shapes(seed, count):
    """(M, N, K, transpose A, transpose B) for the fp32 engine."""
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 700)), int(rng.integers(1, 700)), int(rng.integers(1, 700)),
             bool(rng.integers(0, 2)), bool(rng.integers(0, 2))) for _ in range(count)]


_MLP = _mlp_shapes(505, 16)
_F32 = _f32_shapes(606, 24)


def _epi(flag):
    return mj.EPI_RELU if flag else mj.EPI_NONE


@pytest.mark.parametrize("M,N,K,with_bias,relu", _W8A16)
def test_sweep_w8a16_linear(oracle, dev, M, N, K, with_bias, relu):
    """Integer activations in [-2, 2], int8 weights, scales 2^-8 .. 2^-3 and
    biases in quarter steps: |sum| <= 254 K < 2^21, so the sums, the scaled
    sums and the biased results are exact in fp32 and the bf16 rounding is
    the only one."""
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    x = oracle.f32_to_bf16(rng.integers(-2, 3, size=(M, K)).astype(np.float32))
    Q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    s = (2.0 ** rng.integers(-8, -2, size=N)).astype(np.float32)
    b = (rng.integers(-8, 9, size=N).astype(np.float32) / np.float32(4)) if with_bias else None
    lin = mj.W8Linear(to_dev(Q, dev), to_dev(s, dev), None if b is None else to_dev(b, dev),
                      _epi(relu))
    got = bf16_host_bits(lin.forward(bf16_dev(x, dev)))
    ref, _ = oracle.linear_w8a16(x, Q, s, b, _epi(relu))
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("M,N,K,with_bias,relu", _BF16)
def test_sweep_bf16_gemm(oracle, dev, M, N, K, with_bias, relu):
    """bf16 A [M, K] . B [N, K]^T with integer operands in [-4, 4] and biases
    in quarter steps: the sums are exact (|sum| <= 16 K), so the bf16 outputs
    must match on every tile and pipeline the planner picks."""
    rng = np.random.default_rng(M * 5 + N * 11 + K)
    A = oracle.f32_to_bf16(rng.integers(-4, 5, size=(M, K)).astype(np.float32))
    B = oracle.f32_to_bf16(rng.integers(-4, 5, size=(N, K)).astype(np.float32))
    b = (rng.integers(-8, 9, size=N).astype(np.float32) / np.float32(4)) if with_bias else None
    C = mj.gemm_bf16_nt(bf16_dev(A, dev), bf16_dev(B, dev), None if b is None else to_dev(b, dev),
                        _epi(relu))
    ref, _ = oracle.gemm_bf16_nt(A, B, b, _epi(relu))
    np.testing.assert_array_equal(bf16_host_bits(C), ref)


@pytest.mark.parametrize("M,N,K,_b,_r", _I8)
def test_sweep_int8_gemm(oracle, dev, M, N, K, _b, _r):
    """matmul_i8_i8_to_i32 at any K (K % 16 != 0 takes the generic kernel):
    int32 sums are exact, so bit-exact on every shape."""
    rng = np.random.default_rng(M * 13 + N + K * 3)
    A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    B = rng.integers(-128, 128, size=(N, K), dtype=np.int8)
    got = mj.matmul_i8_i8_to_i32(mj.Tensor(to_dev(A, dev)), mj.Tensor(to_dev(B, dev)).transpose())
    np.testing.assert_array_equal(got.numpy(), oracle.matmul_i8_i8_to_i32(A, B))


@pytest.mark.parametrize("M,N,K,with_bias,relu", _W8A8)
def test_sweep_w8a8_linear(oracle, dev, M, N, K, with_bias, relu):
    """W8A8 with dynamic per-row activation scales: the row quantize and the
    int32 sums are exact and the epilogue's fp32 operations are those of the
    oracle in the same order, so the bf16 outputs match bit for bit."""
    rng = np.random.default_rng(M * 3 + N * 17 + K)
    x = oracle.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    Q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    sw = oracle.randu_f32((N,), 0.0005, 0.004, seed=M + N + K)
    b = oracle.randu_f32((N,), -0.25, 0.25, seed=M + N + K + 1) if with_bias else None
    lin = mj.W8A8Linear(to_dev(Q, dev), to_dev(sw, dev), None if b is None else to_dev(b, dev),
                        _epi(relu))
    got = bf16_host_bits(lin.forward(bf16_dev(x, dev)))
    ref, _, _, _ = oracle.linear_w8a8(x, Q, sw, b, _epi(relu))
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("M,K,I,H", _MLP)
def test_sweep_w8a16_mlp(oracle, dev, M, K, I, H):
    """The SiLU-gated FFN (gate/up GEMM or GEMV, SiLU * up, down projection
    with or without a K split) against the oracle's FFN within the bf16
    bar (normwise 2e-2 on h and on y); a wrong tile, split or column
    pairing moves whole blocks by their own magnitude."""
    x = oracle.f32_to_bf16(oracle.randn_f32((M, K), seed=M + K))
    Wg, sg = oracle.quantize_rowwise_rhe(oracle.randn_f32((I, K), std=0.02, seed=I + 1))
    Wu, su = oracle.quantize_rowwise_rhe(oracle.randn_f32((I, K), std=0.02, seed=I + 2))
    Wd, sd = oracle.quantize_rowwise_rhe(oracle.randn_f32((H, I), std=0.02, seed=H + 3))
    mk = lambda q, s: mj.W8Linear(to_dev(q, dev), to_dev(s, dev))  # noqa: E731
    y, h = mj.W8MLP(mk(Wg, sg), mk(Wu, su), mk(Wd, sd)).forward(bf16_dev(x, dev))
    hr, yr = oracle.mlp_w8a16(x, Wg, sg, Wu, su, Wd, sd)
    assert normwise_rel(bf16_host_f32(h), oracle.bf16_to_f32(hr)) <= 2e-2
    assert normwise_rel(bf16_host_f32(y), oracle.bf16_to_f32(yr)) <= 2e-2


def _f32_view(M, dev, transposed):
    if not transposed:
        return mj.Tensor(to_dev(M, dev))
    return mj.Tensor(to_dev(np.ascontiguousarray(M.T), dev)).transpose()


@pytest.mark.parametrize("M,N,K,ta,tb", _F32)
def test_sweep_f32_matmul(dev, M, N, K, ta, tb):
    """fp32 matmul on the MFMA engine over every tile size (32, 64, 128) and
    loader orientation: small-integer operands make the sums exact, so the
    result equals the exact product."""
    rng = np.random.default_rng(M + 3 * N + 7 * K)
    A = rng.integers(-8, 9, size=(M, K)).astype(np.float32)
    B = rng.integers(-8, 9, size=(K, N)).astype(np.float32)
    got = mj.matmul(_f32_view(A, dev, ta), _f32_view(B, dev, tb)).numpy()
    np.testing.assert_array_equal(got, (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32))


# ------------------------------------------------------------- long sweep
# Opt-in (MJ_LONG_SWEEP=<seconds>): random shapes up to M = 4096, N = 12000,
# K = 16384 for as long as asked, over the W8A16 Linear, the bf16 GEMM, the
# int8 GEMM and the fp32 matmul (with transposed views), every output compared
# with exact float64 products (small-integer operands, power-of-two scales)
# rounded by the oracle's pinned bf16 rounding; over the two quantizers
# (per-row RHE / legacy with exact-tie rows, per-tensor legacy with
# near-ties), bit for bit against the oracle; and over the W8A16 FFN (decode
# and prefill sizes) against float64 bounds.  A third of the W8A16 Linear cases
# take 3-48 x rows at K = 1024 j <= 4096 (the skinny GEMV's range).
_LONG = float(os.environ.get("MJ_LONG_SWEEP", "0"))


def _long_case(rng, fam, dev, to_bf16, oracle_quantize_rowwise=None, oracle_quantize_tensor=None):
    def draw_m():
        return [1, int(rng.integers(2, 17)), int(rng.integers(17, 257)),
                int(rng.integers(257, 1500)), int(rng.integers(1500, 4097))][rng.integers(0, 5)]

    def cap(M, N, K, step):
        while M * N * K > 3e10 and (N > 16 or K > step):
            if (rng.integers(0, 2) and K > step) or N <= 16:
                K = max(step, (K // 2) // step * step)
            else:
                N = max(16, N // 2)
        return N, K

    def bf16_ref(sum64, s, b, relu):
        v = sum64 * (1.0 if s is None else s[None, :]) + (0.0 if b is None else b[None, :])
        v = v.astype(np.float32)
        return to_bf16(np.where(v > 0, v, np.float32(0)) if relu else v)

    relu = bool(rng.integers(0, 2))
    epi = mj.EPI_RELU if relu else mj.EPI_NONE
    if fam == "w8a16":
        M, N, K = draw_m(), int(rng.integers(1, 12001)), int(rng.integers(1, 1025)) * 16
        if rng.integers(0, 3) == 0:
            # the skinny MFMA GEMV's own range: 3-48 x rows at K = 1024 j <= 4096
            M, K = int(rng.integers(3, 49)), int(rng.integers(1, 5)) * 1024
        N, K = cap(M, N, K, 16)
        x = rng.integers(-2, 3, size=(M, K)).astype(np.float32)
        Q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
        s = (2.0 ** rng.integers(-8, -2, size=N)).astype(np.float32)
        b = (rng.integers(-8, 9, size=N) / 4).astype(np.float32) if rng.integers(0, 2) else None
        lin = mj.W8Linear(to_dev(Q, dev), to_dev(s, dev), None if b is None else to_dev(b, dev), epi)
        got = bf16_host_bits(lin.forward(bf16_dev(to_bf16(x), dev)))
        ref = bf16_ref(x.astype(np.float64) @ Q.astype(np.float64).T, s.astype(np.float64),
                       None if b is None else b.astype(np.float64), relu)
    elif fam == "bf16":
        M, N, K = draw_m(), int(rng.integers(1, 9001)), int(rng.integers(1, 1025)) * 8
        N, K = cap(M, N, K, 8)
        A = rng.integers(-4, 5, size=(M, K)).astype(np.float32)
        B = rng.integers(-4, 5, size=(N, K)).astype(np.float32)
        b = (rng.integers(-8, 9, size=N) / 4).astype(np.float32) if rng.integers(0, 2) else None
        got = bf16_host_bits(mj.gemm_bf16_nt(bf16_dev(to_bf16(A), dev),
                                             bf16_dev(to_bf16(B), dev),
                                             None if b is None else to_dev(b, dev), epi))
        ref = bf16_ref(A.astype(np.float64) @ B.astype(np.float64).T, None,
                       None if b is None else b.astype(np.float64), relu)
    elif fam == "i8":
        M, N, K = draw_m(), int(rng.integers(1, 9001)), int(rng.integers(1, 8193))
        N, K = cap(M, N, K, 1)
        A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
        B = rng.integers(-128, 128, size=(N, K), dtype=np.int8)
        got = mj.matmul_i8_i8_to_i32(mj.Tensor(to_dev(A, dev)), mj.Tensor(to_dev(B, dev)).transpose()).numpy()
        ref = (A.astype(np.float64) @ B.astype(np.float64).T).astype(np.int32)
    elif fam == "qrow":
        # per-row quantize/pack: random rows over many decades, rows of exact
        # ties (absmax 127 * 2^e, others (k + 1/2) 2^e), all-zero rows
        N, K = int(rng.integers(1, 3001)), int(rng.integers(1, 9001))
        W = (rng.standard_normal((N, K)) * 10.0 ** rng.uniform(-6, 6, size=(N, 1))).astype(np.float32)
        kind = rng.integers(0, 8, size=N)
        e = rng.integers(-20, 20, size=N).astype(np.float64)
        ties = (rng.integers(-127, 127, size=(N, K)) + 0.5) * 2.0 ** e[:, None]
        ties[:, 0] = 127 * 2.0 ** e
        W = np.where((kind == 0)[:, None], ties.astype(np.float32), W)
        W[kind == 1] = 0.0
        rounding = mj.ROUND_RHE if rng.integers(0, 2) else mj.ROUND_LEGACY
        q, sc = mj.quantize_rowwise_int8(to_dev(W, dev), rounding)
        rq, rs = (oracle_quantize_rowwise(W, rounding))
        got = np.concatenate([q.cpu().numpy().view(np.uint8).ravel(), sc.cpu().numpy().view(np.uint8)])
        ref = np.concatenate([rq.view(np.uint8).ravel(), rs.view(np.uint8)])
        return (fam, N, K, rounding), got, ref
    elif fam == "qtensor":
        # per-tensor legacy quantize: near-ties (k + 1/2) s, random values,
        # a tail of n % 4 elements, sometimes a view that is not 16-byte aligned
        n, off = int(rng.integers(1, 3_000_001)), int(rng.integers(0, 2))
        sv = np.float32(10.0 ** rng.uniform(-4, 1))
        k = rng.integers(-300, 300, n + off) + 0.5
        x = np.where(rng.random(n + off) < 0.5, k * sv,
                     rng.standard_normal(n + off) * 100 * sv).astype(np.float32)
        got = mj.quantize_symmetric_int8(mj.Tensor(to_dev(x, dev)[off:]), float(sv)).numpy()
        return (fam, n, off, float(sv)), got, oracle_quantize_tensor(x[off:], sv)
    elif fam == "mlp":
        # the FFN over its GEMV and GEMM paths: 1, 2-4, 5-16, 17-32 or 33-600 x
        # rows, K up to 16384 (a third of the cases K = 1024 j <= 4096), exact
        # gate/up sums; h within one bf16 step of the float64 value from them,
        # y within one bf16 step plus 2^-16 of the sum of |h Wd| (fp32 summation)
        M = [1, int(rng.integers(2, 5)), int(rng.integers(5, 17)), int(rng.integers(17, 33)),
             int(rng.integers(33, 601))][rng.integers(0, 5)]
        K = int(rng.integers(1, 5)) * 1024 if rng.integers(0, 3) == 0 else \
            int(rng.integers(1, 1025)) * 16
        I, H = int(rng.integers(1, 751)) * 16, int(rng.integers(1, 4097))
        while (M * (2 * I * K + H * I) > 6e9 or 2 * I * K + H * I > 1.5e8) and (K > 16 or I > 16):
            if K >= I:
                K = max(16, (K // 2) // 16 * 16)
            else:
                I = max(16, (I // 2) // 16 * 16)
        x = rng.integers(-4, 5, size=(M, K)).astype(np.float32)
        Wg = rng.integers(-127, 128, size=(I, K), dtype=np.int8)
        Wu = rng.integers(-127, 128, size=(I, K), dtype=np.int8)
        Wd = rng.integers(-127, 128, size=(H, I), dtype=np.int8)
        sg = (2.0 ** rng.integers(-14, -10, size=I)).astype(np.float32)
        su = (2.0 ** rng.integers(-14, -10, size=I)).astype(np.float32)
        sd = (2.0 ** rng.integers(-12, -8, size=H)).astype(np.float32)
        mk = lambda q, sc: mj.W8Linear(to_dev(q, dev), to_dev(sc, dev))  # noqa: E731
        y, h = mj.W8MLP(mk(Wg, sg), mk(Wu, su), mk(Wd, sd)).forward(bf16_dev(to_bf16(x), dev))
        h, y = bf16_host_f32(h).astype(np.float64), bf16_host_f32(y).astype(np.float64)
        xf = x.astype(np.float64)
        g = (xf @ Wg.astype(np.float64).T) * sg.astype(np.float64)
        u = (xf @ Wu.astype(np.float64).T) * su.astype(np.float64)
        href = g / (1.0 + np.exp(-g)) * u
        hbad = np.abs(h - href) > np.maximum(np.abs(href) * 2.0 ** -8, 1e-6)
        Wdf = Wd.astype(np.float64)
        yref = (h @ Wdf.T) * sd.astype(np.float64)
        ybound = np.abs(yref) * 2.0 ** -8 + 2.0 ** -16 * (np.abs(h) @ np.abs(Wdf).T) * sd + 1e-30
        ybad = np.abs(y - yref) > ybound
        return (fam, M, K, I, H), np.array([int(hbad.sum()), int(ybad.sum())]), np.array([0, 0])
    else:
        M, N, K = (int(v) for v in rng.integers(1, 3000, size=3))
        ta, tb = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
        A = rng.integers(-8, 9, size=(M, K)).astype(np.float32)
        B = rng.integers(-8, 9, size=(K, N)).astype(np.float32)
        got = mj.matmul(_f32_view(A, dev, ta), _f32_view(B, dev, tb)).numpy()
        ref = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    return (fam, M, N, K), got, ref


@pytest.mark.skipif(_LONG <= 0, reason="opt-in: set MJ_LONG_SWEEP=<seconds>")
def test_long_random_sweep(oracle, dev):
    rng = np.random.default_rng(int(os.environ.get("MJ_LONG_SWEEP_SEED", "7")))
    t_end, n, bad = time.time() + _LONG, 0, []
    fams = ("w8a16", "bf16", "i8", "f32", "qrow", "qtensor", "mlp")
    qrow = lambda W, r: oracle.quantize_rowwise_rhe(W) if r == mj.ROUND_RHE else \
        oracle.quantize_rowwise_legacy(W)  # noqa: E731
    while time.time() < t_end:
        desc, got, ref = _long_case(rng, fams[n % len(fams)], dev, oracle.f32_to_bf16, qrow,
                                    oracle.quantize_symmetric_int8)
        n += 1
        if got.shape != ref.shape or not np.array_equal(got, ref):
            bad.append(desc)
        if n % 50 == 0:
            print(f"{n} cases, {len(bad)} mismatches (last {desc})", flush=True)
    print(f"{n} cases, {len(bad)} mismatches", flush=True)
    assert not bad, bad[:10]
