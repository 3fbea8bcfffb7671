"""Host-side address check of the W8A8 Linear (mj_linear_w8a8) launch.

Every global-memory access of the two kernels the entry point enqueues
(quantize_rows_bf16_reg, then gemm_i8_w4_kernel<BN, 2>) is enumerated on the
CPU for every workgroup, wave and lane of the grid the launchers compute, and
checked against the allocations the caller and the entry point provide:
x [M,K] bf16, Q [N,K] int8, scales / bias [N] fp32, y [M,N] bf16, and the
workspace holding xq [M,K] int8 at offset 0 and sx [M] fp32 at
round_up(M*K, 256), of exactly that size (the size a graph-owned
stream-ordered allocation had when the W8A8 Linear was captured).

Each step below mirrors one statement of the kernels (quant.hip
quantize_rows_bf16_reg / launch_rows_reg / launch_quantize_rows_bf16,
gemm_nt.hip gemm_i8_w4_kernel / store_w8a8 / launch_i8_w4, common.h
tile_coords / group_coords); raw buffer loads (the GEMM's operand loads) are
range-checked by the hardware against their resource, so for them the check
is that each resource lies inside its allocation and that every offset is
inside the resource or the out-of-range sentinel.  The check also asserts
that the epilogue writes every output element exactly once.
"""
import numpy as np
import pytest

K_OOB = 0x7FFFFFF0          # kOobOffset (common.h)


def group_coords(logical, tiles_m, tiles_n, group_m):
    per_group = group_m * tiles_n
    g = logical // per_group
    first_m = g * group_m
    gsize = min(tiles_m - first_m, group_m)
    in_g = logical - g * per_group
    return first_m + in_g % gsize, in_g // gsize


def tile_coords(bid, tiles_m, tiles_n, group_m):
    total = tiles_m * tiles_n
    x, q, r = bid & 7, total >> 3, total & 7
    logical = x * q + min(x, r) + (bid >> 3)
    return group_coords(logical, tiles_m, tiles_n, group_m)


def quantizer_accesses(M, K):
    """quantize_rows_bf16_reg<W, CH> as launch_quantize_rows_bf16 picks it:
    byte ranges [lo, hi) of x read, xq written, sx written."""
    assert K % 512 == 0 and K // 512 <= 16
    n = K // 512
    W = 4 if n % 4 == 0 else (2 if n % 2 == 0 else 1)
    CH = n // W
    rows_per_wg = 4 // W
    blocks = (M + rows_per_wg - 1) // rows_per_wg
    reads, writes_q, writes_s = [], [], []
    t_all = np.arange(256)
    wave = t_all >> 6
    lane = t_all & 63
    for b in range(blocks):
        row = b * rows_per_wg + wave // W
        t = (wave % W) * 64 + lane
        live = row < M
        for c in range(CH):
            idx = c * 64 * W + t                      # uint4 of x, uint2 of xq
            xr = np.where(live, row, 0) * K * 2 + idx * 16
            reads.append(np.stack([xr, xr + 16]))
            qw = row[live] * K + idx[live] * 8
            writes_q.append(np.stack([qw, qw + 8]))
        sw = row[live & (t == 0)] * 4
        writes_s.append(np.stack([sw, sw + 4]))
    cat = lambda v: np.concatenate(v, axis=1)   # noqa: E731
    return cat(reads), cat(writes_q), cat(writes_s)


def gemm_accesses(M, N, K):
    """gemm_i8_w4_kernel<BN, 2> as launch_i8_w4 picks it."""
    BM = 256
    tiles256 = ((M + 255) // 256) * ((N + 255) // 256)
    BN = 256 if tiles256 >= 192 else 128
    tiles_m, tiles_n = (M + BM - 1) // BM, (N + BN - 1) // BN
    DPA, DPB, KS = 8, BN // 32, 128
    nk = (K + KS - 1) // KS
    # the unrolled loop `for (kt = 0; kt + 8 <= nk_full; kt += 6)` runs L
    # rounds of six stages, each loading stage kt + 2 with its K offset in
    # soffset ("fast"); the prologue (stages 0, 1) and the tail loop check K
    nk_full = K // KS
    L = (nk_full - 8) // 6 + 1 if nk_full >= 8 else 0
    fast_stages = set(range(2, 6 * L + 2))
    lanes = np.arange(64)
    rsrc, offs, y_writes, sx_reads, sw_reads = [], [], [], [], []
    for bid in range(tiles_m * tiles_n):
        tm, tn = tile_coords(bid, tiles_m, tiles_n, 4)
        m0, n0 = tm * BM, tn * BN
        rA = (m0 * K, m0 * K + (M - m0) * K)          # make_rsrc(A + m0*lda, (M-m0)*lda)
        rB = (n0 * K, n0 * K + (N - n0) * K)
        rsrc.append((rA, rB))
        for wave in range(4):
            for i in range(DPA):
                r = (i * 4 + wave) * 8 + (lanes >> 3)
                c = (lanes & 7) ^ ((r >> 1) & 7)
                a_off = np.where(m0 + r < M, r * K + c * 16, K_OOB)
                b_off = np.where(n0 + r < N, r * K + c * 16, K_OOB)
                for kt in range(nk + 2):
                    k0 = kt * KS
                    fast = kt in fast_stages
                    for off, lim, use in ((a_off, rA[1] - rA[0], True),
                                          (b_off, rB[1] - rB[0], i < DPB)):
                        if not use:
                            continue
                        if fast:
                            v = np.where(off == K_OOB, K_OOB, off + k0)
                        else:
                            ok = k0 + c * 16 < K
                            v = np.where(ok & (off != K_OOB), off + k0, K_OOB)
                        offs.append((v, lim))
            # store_w8a8: wm = wave >> 1, wn = wave & 1
            wm, wn = wave >> 1, wave & 1
            fr, fh = lanes & 15, lanes >> 4
            WN = BN // 2
            for i in range(8):
                m = m0 + wm * 128 + i * 16 + fr
                sx_reads.append(np.where(m < M, m, M - 1))
                for j in range(WN // 16):
                    nb = n0 + wn * WN + j * 16 + 4 * fh
                    for q in range(4):
                        sw_reads.append(np.minimum(nb + q, N - 1))
                        live = (m < M) & (nb + q < N)
                        y_writes.append(m[live] * N + nb[live] + q)
    return (BN, rsrc, offs, np.concatenate(y_writes), np.concatenate(sx_reads),
            np.concatenate(sw_reads))


@pytest.mark.parametrize("M,N,K", [(64, 1024, 4096), (1, 256, 512), (300, 520, 1536),
                                   (257, 1000, 2048), (2048, 4096, 4096)])
def test_w8a8_launch_stays_in_bounds(M, N, K):
    # the entry point's workspace: xq [M*K] then sx [M] at round_up(M*K, 256)
    xq_bytes = (M * K + 255) & ~255
    ws_bytes = xq_bytes + 4 * M
    x_bytes, q_bytes, y_bytes = M * K * 2, N * K, M * N * 2

    reads, wq, ws_ = quantizer_accesses(M, K)
    assert reads.min() >= 0 and reads[1].max() <= x_bytes
    assert wq.min() >= 0 and wq[1].max() <= M * K <= xq_bytes
    assert ws_.shape[1] == M                                  # one scale per row
    assert (xq_bytes + ws_).min() >= xq_bytes and (xq_bytes + ws_[1]).max() <= ws_bytes
    # every xq byte the GEMM reads was written by the quantizer
    covered = np.zeros(M * K, dtype=np.int32)
    for lo in wq[0]:
        covered[lo:lo + 8] += 1
    assert np.all(covered == 1)

    BN, rsrc, offs, yw, sx_r, sw_r = gemm_accesses(M, N, K)
    for (a_lo, a_hi), (b_lo, b_hi) in rsrc:
        assert 0 <= a_lo <= a_hi <= M * K <= xq_bytes
        assert 0 <= b_lo <= b_hi <= q_bytes
    for v, lim in offs:
        inside = (v + 16 <= lim)
        assert np.all(inside | (v == K_OOB)), "a direct load neither in range nor the sentinel"
        assert np.all(v[~inside] >= lim)                       # sentinel loads read zeros
    assert sx_r.min() >= 0 and sx_r.max() < M
    assert sw_r.min() >= 0 and sw_r.max() < N
    assert yw.min() >= 0 and yw.max() * 2 + 2 <= y_bytes
    counts = np.bincount(yw, minlength=M * N)
    assert np.all(counts == 1), "an output element written twice or never"
