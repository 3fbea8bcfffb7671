#!/usr/bin/env python3
"""Benchmark of the MI355X backend on BASELINE.json's headline configurations.

Headline (``value``): config C2, the bf16 NT GEMM at M=N=K=4096 with fp32
accumulation, in TFLOP/s; a "step" is one GEMM launch over inputs already
resident in HBM.  The int8 weight-only decode GEMV (config C3, GB/s against
the HBM roofline) and the other configs are reported under ``secondary``.

Timing: ``--warmup`` untimed launches, then further untimed launches of the
same workload until ``--settle`` seconds of load have passed (MI355X raises
its clock over the first tens of milliseconds of load after idle; without
this the first ~100 launches are timed on the ramp and read 10-20 % slow),
then ``--steps`` launches bracketed by torch.cuda.synchronize() and HIP events
recorded on the stream the kernels are launched on (torch's current stream,
which the C ABI is handed).

The GEMV's weights (45 MB) would fit in the 256 MB MALL, so its timed loop
rotates over enough weight copies (> 256 MB) that every launch streams its
weights from HBM.

``cpu_baseline`` times the oracle (the C restatement of momijo's CPU tensor
engine, single-threaded as the reference is) on a row slab of C2, on this
box's host cores, using the very bytes the GPU leg multiplied (copied back
from the device after its timed region; sha256 recorded).  The C3, C3-pack
and C1 entries carry their own ``cpu_baseline``, timed in full the same way;
C4 and C5 carry one timed on a row slab of their x with the full weights
(every row costs the same, so the slab's rate is the problem's; the full
problem's time is extrapolated linearly in M and stated).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_INT8_TOPS = 5000.0     # MI355X dense int8 MFMA
PEAK_FP32_TFLOPS = 157.3    # MI355X fp32 matrix
PEAK_FP64_TFLOPS = 78.6     # MI355X fp64 matrix
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E


def _traffic(name: str):
    """HBM bytes per launch of a kernel as measured by rocprofv3 counters
    (FETCH_SIZE x2.0 + WRITE_SIZE, calibrated against a copy of known size);
    recorded in profiles/hbm_traffic.json, None where not measured."""
    try:
        with open(os.path.join(ROOT, "profiles", "hbm_traffic.json")) as f:
            return json.load(f).get(name, {}).get("bytes")
    except (OSError, ValueError):
        return None


def _args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--settle", type=float, default=0.3,
                   help="seconds of untimed load after the warmup launches of each workload")
    p.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    p.add_argument("--only", default="", help="comma list of workloads (c1,c2,c3,c3batch,c3pack,c4,c4w8a8,c5,"
                   "c5decode,qlinear,bwd,conv2d,f64,copy,vendor); copy and vendor are run only when named")
    return p.parse_args()


SETTLE_S = 0.3  # set from --settle in main()


def _settle(fn):
    """Untimed launches of fn(i) until SETTLE_S seconds of load have passed."""
    import torch
    t0 = time.perf_counter()
    i = 0
    while time.perf_counter() - t0 < SETTLE_S:
        for _ in range(8):
            fn(i)
            i += 1
        torch.cuda.synchronize()


def _time_launches(fn, steps: int, warmup: int):
    """Average ms per launch of fn() over `steps` launches (HIP events on the
    current stream), after `warmup` untimed ones and the settle period."""
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    _settle(fn)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def _rand_bf16(shape, seed, std=1.0):
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(shape, generator=g, device="cuda") * std).to(torch.bfloat16)


def _rand_f32(shape, seed, std=1.0):
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(shape, generator=g, device="cuda") * std


# Inputs of the GPU legs that the CPU baseline re-times on the same bytes
# (copied from the device after the timed region): name -> host arrays.
_CPU_INPUTS = {}
# Rows of x in the CPU legs' row slabs of C4 and C5 (each row costs the CPU
# the same work, so the slab's rate is the full problem's rate).
CPU_SLAB_C4 = 32
CPU_SLAB_C5 = 8


def _host_bf16_bits(t):
    """bf16 device tensor -> uint16 host array of its bit patterns."""
    import numpy as np
    import torch
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def bench_c2(steps, warmup):
    import momijo_amd as mj
    M = N = K = 4096
    A = _rand_bf16((M, K), 1)
    B = _rand_bf16((N, K), 2)
    C = mj.gemm_bf16_nt(A, B)
    ms = _time_launches(lambda i: mj.gemm_bf16_nt(A, B, out=C), steps, warmup)
    # the CPU leg times the oracle on a row slab of these exact bytes
    _CPU_INPUTS["c2"] = (_host_bf16_bits(A[:256]), _host_bf16_bits(B))
    flops = 2.0 * M * N * K
    tflops = flops / (ms * 1e-3) / 1e12
    return {
        "name": "c2_bf16_gemm_4096",
        "metric": "bf16 NT GEMM TFLOP/s at 4096^3",
        "value": tflops, "unit": "TFLOP/s", "ms_per_launch": ms,
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": tflops / PEAK_BF16_TFLOPS,
                     "traffic": _traffic("c2_bf16_gemm_4096")},
        "flops_per_launch": flops,
    }


def _graph_ms_per_launch(launch, n_in_graph: int, replays: int):
    """GPU time per launch of `launch(i)` with host overhead removed: n_in_graph
    launches are captured into one HIP graph (torch.cuda.CUDAGraph) and the
    graph is replayed `replays` times between two events."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(3):
            launch(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n_in_graph):
            launch(i)
    g.replay()
    torch.cuda.synchronize()
    _settle(lambda i: g.replay())
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (replays * n_in_graph)


def bench_c3(steps, warmup):
    import torch
    import momijo_amd as mj
    N, K = 11008, 4096
    W = _rand_f32((N, K), 4, 0.02)
    q0, s = mj.quantize_rowwise_int8(W)
    del W
    bias = (torch.rand(N, device="cuda") - 0.5) / 8
    x = _rand_bf16((1, K), 3)
    y = torch.empty((1, N), dtype=torch.bfloat16, device="cuda")
    copies = 8  # 8 x 45 MB > the 256 MB MALL: each launch reads from HBM
    qs = [q0] + [q0.clone() for _ in range(copies - 1)]
    lins = [mj.W8Linear(q, s, bias) for q in qs]
    n_launch = max(steps, 400)
    # eager back-to-back launches (host overhead per call is below the
    # kernel's duration, so the GPU stays busy) ...
    eager_ms = _time_launches(lambda i: lins[i % copies].forward(x, out=y), n_launch,
                              max(warmup, 16))
    hot_ms = _time_launches(lambda i: lins[0].forward(x, out=y), n_launch, max(warmup, 16))
    # ... and the same launches replayed from a captured graph (no host cost)
    ms = _graph_ms_per_launch(lambda i: lins[i % copies].forward(x, out=y), 64,
                              max(n_launch // 64, 4))
    # the device-side cost of one dispatch of this kernel over 4 weight rows:
    # a floor that every launch pays whatever its size
    tiny = mj.W8Linear(q0[:4].contiguous(), s[:4].contiguous(), bias[:4].contiguous())
    y4 = torch.empty((1, 4), dtype=torch.bfloat16, device="cuda")
    floor_ms = _graph_ms_per_launch(lambda i: tiny.forward(x, out=y4), 64, 4)
    bytes_ = N * K + N * 4 + K * 2 + N * 4 + N * 2   # Q + scales + x + bias(f32) + y
    gbs = bytes_ / (ms * 1e-3) / 1e9
    _CPU_INPUTS["c3"] = (_host_bf16_bits(x), q0.cpu().numpy(), s.cpu().numpy(), bias.cpu().numpy())
    return {
        "name": "c3_int8_gemv_11008x4096",
        "metric": "int8 weight-only GEMV GB/s (M=1)",
        "value": gbs, "unit": "GB/s", "ms_per_launch": ms,
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": gbs / PEAK_HBM_GBS, "traffic": _traffic("c3_int8_gemv_11008x4096")},
        "bytes_per_launch": bytes_,
        "timing": "graph replay of 64 launches rotating over 8 weight copies (> MALL)",
        "eager_ms_per_launch": eager_ms,
        "weights_rotated_over": copies,
        "cache_hot_GBs": bytes_ / (hot_ms * 1e-3) / 1e9,
        "dispatch_floor_us": floor_ms * 1e3,
    }


def bench_c3_batch(steps, warmup):
    """The C3 weight (11008 x 4096 int8, per-channel scales, bias) at 4, 16
    and 32 x rows: batched decode on the skinny GEMV, HBM-bound like C3.
    Graph replay over 8 weight copies, as the C3 line."""
    import torch
    import momijo_amd as mj
    N, K = 11008, 4096
    W = _rand_f32((N, K), 4, 0.02)
    q0, s = mj.quantize_rowwise_int8(W)
    del W
    bias = (torch.rand(N, device="cuda") - 0.5) / 8
    copies = 8
    qs = [q0] + [q0.clone() for _ in range(copies - 1)]
    lins = [mj.W8Linear(q, s, bias) for q in qs]
    out = []
    for M in (4, 16, 32):
        x = _rand_bf16((M, K), 30 + M)
        y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        ms = _graph_ms_per_launch(lambda i: lins[i % copies].forward(x, out=y), 64,
                                  max(max(steps, 400) // 64, 4))
        bytes_ = N * K + N * 4 + M * K * 2 + N * 4 + M * N * 2
        gbs = bytes_ / (ms * 1e-3) / 1e9
        out.append({
            "name": f"c3batch_int8_gemv_11008x4096_m{M}",
            "metric": f"int8 weight-only GEMV GB/s (M={M})",
            "value": gbs, "unit": "GB/s", "ms_per_launch": ms,
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": gbs / PEAK_HBM_GBS,
                         "traffic": _traffic(f"c3batch_int8_gemv_11008x4096_m{M}")},
            "bytes_per_launch": bytes_,
            "timing": "graph replay of 64 launches rotating over 8 weight copies (> MALL)",
        })
    return out


def bench_c5_decode(steps, warmup):
    """The C5 FFN (4096 -> 11008 -> 4096, W8A16) at decode sizes, 1, 4 and 16
    x rows: the gate/up GEMV and the down GEMV, HBM-bound on the 135 MB of
    weights.  Graph replay rotating over 3 weight sets (405 MB > the MALL)."""
    import torch
    import momijo_amd as mj
    K, I, H = 4096, 11008, 4096
    copies = 3

    def lin(n, k, seed):
        W = _rand_f32((n, k), seed, 0.02)
        q, s = mj.quantize_rowwise_int8(W)
        del W
        return mj.W8Linear(q, s)

    mlps = [mj.W8MLP(lin(I, K, 60 + 3 * c), lin(I, K, 61 + 3 * c), lin(H, I, 62 + 3 * c))
            for c in range(copies)]
    out = []
    for M in (1, 4, 16):
        x = _rand_bf16((M, K), 70 + M)
        h = torch.empty((M, I), dtype=torch.bfloat16, device="cuda")
        y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
        ms = _graph_ms_per_launch(lambda i: mlps[i % copies].forward(x, h, y), 48,
                                  max(max(steps, 400) // 48, 4))
        # weights and scales of the three projections, x, h written and read, y
        bytes_ = (3 * I * K + (2 * I + H) * 4 + M * K * 2 + 2 * M * I * 2 + M * H * 2)
        gbs = bytes_ / (ms * 1e-3) / 1e9
        out.append({
            "name": f"c5decode_ffn_w8a16_m{M}",
            "metric": f"W8A16 FFN 4096-11008-4096 GB/s (M={M})",
            "value": gbs, "unit": "GB/s", "ms_per_launch": ms,
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": gbs / PEAK_HBM_GBS, "traffic": _traffic(f"c5decode_ffn_w8a16_m{M}")},
            "bytes_per_launch": bytes_,
            "timing": "graph replay of 48 FFN calls (two GEMV launches each) rotating over "
                      "3 weight sets (> MALL)",
        })
    return out


def bench_c3_pack(steps, warmup):
    import torch
    import momijo_amd as mj
    from momijo_amd import _lib
    N, K = 11008, 4096
    Ws = [_rand_f32((N, K), 4 + i, 0.02) for i in range(2)]  # 2 x 180 MB: no MALL reuse
    q = torch.empty((N, K), dtype=torch.int8, device="cuda")
    s = torch.empty((N,), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream

    def run(i):
        _lib.call("mj_quantize_rowwise_i8", Ws[i % 2].data_ptr(), N, K, _lib.ROUND_RHE,
                  q.data_ptr(), s.data_ptr(), stream)

    ms = _time_launches(run, max(steps // 2, 20), warmup)
    bytes_ = N * K * 4 + N * K + N * 4
    gbs = bytes_ / (ms * 1e-3) / 1e9
    _CPU_INPUTS["c3pack"] = (Ws[0].cpu().numpy(),)
    return {
        "name": "c3pack_quantize_rowwise_11008x4096",
        "metric": "per-channel int8 quantize/pack GB/s",
        "value": gbs, "unit": "GB/s", "ms_per_launch": ms,
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": gbs / PEAK_HBM_GBS,
                     "traffic": _traffic("c3pack_quantize_rowwise_11008x4096")},
        "bytes_per_launch": bytes_,
    }


def bench_c4(steps, warmup):
    import torch
    import momijo_amd as mj
    M, N, K = 2048, 4096, 4096
    lin = mj.W8Linear.from_float(_rand_f32((N, K), 6, 0.02),
                                 (torch.rand(N, device="cuda") - 0.5) / 8, mj.EPI_GELU_TANH)
    x = _rand_bf16((M, K), 5)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ms = _time_launches(lambda i: lin.forward(x, out=y), steps, warmup)
    flops = 2.0 * M * N * K
    tf = flops / (ms * 1e-3) / 1e12
    _CPU_INPUTS["c4"] = (_host_bf16_bits(x[:CPU_SLAB_C4]), lin.q.cpu().numpy(),
                         lin.scales.cpu().numpy(), lin.bias.cpu().numpy(), M)
    return {
        "name": "c4_w8a16_prefill_gelu_2048x4096x4096",
        "metric": "W8A16 GEMM + bias + GELU TFLOP/s",
        "value": tf, "unit": "TFLOP/s", "ms_per_launch": ms,
        "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": tf / PEAK_BF16_TFLOPS,
                     "traffic": _traffic("c4_w8a16_prefill_gelu_2048x4096x4096")},
    }


def bench_c4_w8a8(steps, warmup):
    """C4's shape and epilogue (2048 x 4096 x 4096, bias + GELU, bf16 out) on
    the W8A8-dynamic path: per-row int8 quantize of x, int8 MFMA with exact
    int32 sums, both scales + bias + GELU in the epilogue.  The quantize
    launch is inside the timed region; priced against the int8 peak."""
    import torch
    import momijo_amd as mj
    M, N, K = 2048, 4096, 4096
    lin = mj.W8A8Linear.from_float(_rand_f32((N, K), 6, 0.02),
                                   (torch.rand(N, device="cuda") - 0.5) / 8, mj.EPI_GELU_TANH)
    x = _rand_bf16((M, K), 5)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ms = _time_launches(lambda i: lin.forward(x, out=y), steps, warmup)
    ops = 2.0 * M * N * K
    tops = ops / (ms * 1e-3) / 1e12
    return {
        "name": "c4_w8a8_dynamic_prefill_gelu_2048x4096x4096",
        "metric": "W8A8-dynamic Linear + bias + GELU TOP/s (row quantize + int8 GEMM)",
        "value": tops, "unit": "TOP/s", "ms_per_call": ms,
        "roofline": {"bound": "mfma", "achieved": tops, "peak": PEAK_INT8_TOPS, "unit": "TOP/s",
                     "frac": tops / PEAK_INT8_TOPS,
                     "traffic": _traffic("c4_w8a8_dynamic_prefill_gelu_2048x4096x4096")},
    }


def bench_c5(steps, warmup):
    import torch
    import momijo_amd as mj
    M, K, I, H = 512, 4096, 11008, 4096
    g = mj.W8Linear.from_float(_rand_f32((I, K), 6, 0.02))
    u = mj.W8Linear.from_float(_rand_f32((I, K), 7, 0.02))
    d = mj.W8Linear.from_float(_rand_f32((H, I), 8, 0.02))
    mlp = mj.W8MLP(g, u, d)
    x = _rand_bf16((M, K), 9)
    h = torch.empty((M, I), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((M, H), dtype=torch.bfloat16, device="cuda")
    ms = _time_launches(lambda i: mlp.forward(x, h, y), steps, warmup)
    flops = 3 * 2.0 * M * K * I
    tf = flops / (ms * 1e-3) / 1e12
    _CPU_INPUTS["c5"] = (_host_bf16_bits(x[:CPU_SLAB_C5]), g.q.cpu().numpy(), g.scales.cpu().numpy(),
                         u.q.cpu().numpy(), u.scales.cpu().numpy(), d.q.cpu().numpy(),
                         d.scales.cpu().numpy(), M)
    return {
        "name": "c5_w8a16_mlp_512x4096x11008",
        "metric": "W8A16 Llama FFN TFLOP/s (gate/up + down)",
        "value": tf, "unit": "TFLOP/s", "ms_per_step": ms,
        "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": tf / PEAK_BF16_TFLOPS,
                     "traffic": _traffic("c5_w8a16_mlp_512x4096x11008")},
    }


def bench_qlinear(steps, warmup):
    """QuantLinear.forward (learn/nn/layers.mojo:1681-1685) at 4096^3: the
    legacy per-tensor W8A8 path -- x quantized with s_x, int8 x int8 -> int32
    on the int8 matrix cores, dequantize + bias fused, fp32 out.  Not a
    BASELINE config: it shows the int8 MFMA path against the int8 peak."""
    import torch
    import momijo_amd as mj
    M = N = K = 4096
    W = _rand_f32((N, K), 11, 0.02)
    s_w = float(W.abs().max()) / 127.0
    Wq = torch.clamp(torch.round(W / s_w), -127, 127).to(torch.int8)
    del W
    x = mj.Tensor(_rand_f32((M, K), 12))
    s_x = float(x.torch.abs().max()) / 127.0
    b = mj.Tensor((torch.rand(N, device="cuda") - 0.5) / 8)
    ql = mj.QuantLinear(K, N, mj.Tensor(Wq), b, s_w, s_x)
    ms = _time_launches(lambda i: ql.forward(x), steps, warmup)
    ops = 2.0 * M * N * K
    tops = ops / (ms * 1e-3) / 1e12
    return {
        "name": "quant_linear_w8a8_4096",
        "metric": "QuantLinear (per-tensor W8A8) TOP/s, quantize + int8 GEMM + dequant",
        "value": tops, "unit": "TOP/s", "ms_per_call": ms,
        "roofline": {"bound": "mfma", "achieved": tops, "peak": PEAK_INT8_TOPS, "unit": "TOP/s",
                     "frac": tops / PEAK_INT8_TOPS, "traffic": _traffic("quant_linear_w8a8_4096")},
    }


def bench_c1(steps, warmup):
    import torch
    import momijo_amd as mj
    x = mj.Tensor(_rand_f32((256, 256), 1))
    lin = mj.Linear(256, 256)
    lin.weight.torch.copy_(_rand_f32((256, 256), 2))
    lin.bias_t.torch.copy_((torch.rand(256, device="cuda") - 0.5) / 8)
    ms = _time_launches(lambda i: lin.forward_act(x, mj.EPI_RELU), steps, warmup)
    _CPU_INPUTS["c1"] = (x.torch.cpu().numpy(), lin.weight.torch.cpu().numpy(),
                         lin.bias_t.torch.cpu().numpy())
    flops = 2.0 * 256 ** 3
    tf = flops / (ms * 1e-3) / 1e12
    return {
        "name": "c1_fp32_linear_relu_256",
        "metric": "fp32 Linear(256->256)+bias+ReLU TFLOP/s",
        "value": tf, "unit": "TFLOP/s", "ms_per_launch": ms,
        "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK_FP32_TFLOPS,
                     "unit": "TFLOP/s", "frac": tf / PEAK_FP32_TFLOPS, "traffic": None},
    }


def bench_backward(steps, warmup):
    """Linear.backward (dx, dW, db) in fp32: at the C1 size, and at a
    4096-wide training shape where the fp32 MFMA engine is the bound."""
    import momijo_amd as mj
    out = []
    for n in (256, 4096):
        x = mj.Tensor(_rand_f32((n, n), 11))
        dy = mj.Tensor(_rand_f32((n, n), 12))
        lin = mj.Linear(n, n)
        lin.weight.torch.copy_(_rand_f32((n, n), 13))
        st = steps if n == 256 else max(3, steps // 20)
        ms = _time_launches(lambda i: lin.backward(x, dy), st, max(1, warmup // 5))
        flops = 2 * 2.0 * n ** 3  # dx and dW; db is N*OutF adds
        tf = flops / (ms * 1e-3) / 1e12
        out.append({
            "name": f"linear_backward_f32_{n}",
            "metric": f"fp32 Linear({n}->{n}).backward, N={n}: dx + dW + db TFLOP/s",
            "value": tf, "unit": "TFLOP/s", "ms_per_step": ms,
            "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK_FP32_TFLOPS,
                         "unit": "TFLOP/s", "frac": tf / PEAK_FP32_TFLOPS, "traffic": None},
        })
    return out


def bench_conv2d(steps, warmup):
    """Conv2d.forward (learn/nn/conv.mojo:600-697), fp32 NCHW, on a ResNet-50
    3 x 3 layer shape: x [32, 64, 56, 56], w [64, 64, 3, 3], stride 1, pad 1,
    bias; one implicit GEMM per image on the fp32 matrix cores."""
    import torch
    import momijo_amd as mj
    N, C, H, W, OC, k = 32, 64, 56, 56, 64, 3
    layer = mj.Conv2d(C, OC, (k, k), (1, 1), (1, 1))
    layer.weight.torch.copy_(_rand_f32((OC, C, k, k), 14, float((2.0 / (C * k * k)) ** 0.5)))
    layer.bias_t.torch.copy_((torch.rand(OC, device="cuda") - 0.5) / 8)
    x = mj.Tensor(_rand_f32((N, C, H, W), 15))
    ms = _time_launches(lambda i: layer.forward(x), steps, warmup)
    OH, OW = layer.out_size(H, W)
    flops = 2.0 * N * OC * OH * OW * C * k * k
    tf = flops / (ms * 1e-3) / 1e12
    _CPU_INPUTS["conv2d"] = (x.torch[:1].cpu().numpy(), layer.weight.torch.cpu().numpy(),
                             layer.bias_t.torch.cpu().numpy(), N)
    return {
        "name": "conv2d_f32_32x64x56x56_3x3",
        "metric": "fp32 Conv2d.forward TFLOP/s (NCHW, 3x3, stride 1, pad 1, bias)",
        "value": tf, "unit": "TFLOP/s", "ms_per_call": ms, "flops_per_call": flops,
        "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK_FP32_TFLOPS,
                     "unit": "TFLOP/s", "frac": tf / PEAK_FP32_TFLOPS,
                     "traffic": _traffic("conv2d_f32_32x64x56x56_3x3")},
    }


def bench_f64(steps, warmup):
    """Float64 matmul (matmul_core_mm / matmul2d) at 2048^3 on fp64 MFMA."""
    import torch
    import momijo_amd as mj
    n = 2048
    g = torch.Generator(device="cuda").manual_seed(21)
    a = mj.Tensor(torch.randn((n, n), generator=g, device="cuda", dtype=torch.float64))
    b = mj.Tensor(torch.randn((n, n), generator=g, device="cuda", dtype=torch.float64))
    ms = _time_launches(lambda i: mj.matmul(a, b), max(3, steps // 10), max(1, warmup // 5))
    tf = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
    return {
        "name": "matmul_f64_2048",
        "metric": "fp64 matmul 2048^3 TFLOP/s",
        "value": tf, "unit": "TFLOP/s", "ms_per_launch": ms,
        "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK_FP64_TFLOPS,
                     "unit": "TFLOP/s", "frac": tf / PEAK_FP64_TFLOPS, "traffic": None},
    }


def bench_copy(steps, warmup):
    """A plain device copy of known size: the calibration point for the
    rocprof FETCH_SIZE / WRITE_SIZE counters and the achievable HBM rate."""
    import torch
    n = 256 * 1024 * 1024 // 4  # 256 MiB per buffer
    srcs = [torch.ones(n, device="cuda") for _ in range(2)]
    dst = torch.empty(n, device="cuda")
    ms = _time_launches(lambda i: dst.copy_(srcs[i % 2]), max(steps // 4, 10), warmup)
    bytes_ = 2 * n * 4
    gbs = bytes_ / (ms * 1e-3) / 1e9
    return {"name": "copy_256MiB", "metric": "device copy GB/s (read+write)", "value": gbs,
            "unit": "GB/s", "ms_per_launch": ms, "bytes_per_launch": bytes_,
            "read_bytes": n * 4, "write_bytes": n * 4}


def bench_vendor(steps, warmup):
    """torch.matmul (hipBLASLt) on the C2 inputs and on the bf16 shapes of C4
    and C5, and torch's conv2d (MIOpen) on the conv2d line's layer: the vendor
    libraries' times for the same work, for comparison only (run when named)."""
    import torch
    out = []
    for (M, N, K, name) in ((4096, 4096, 4096, "c2"), (2048, 4096, 4096, "c4_shape_bf16"),
                            (512, 22016, 4096, "c5_gateup_shape_bf16"),
                            (512, 4096, 11008, "c5_down_shape_bf16")):
        A = _rand_bf16((M, K), 1)
        Bt = _rand_bf16((N, K), 2).t()
        C = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        ms = _time_launches(lambda i: torch.matmul(A, Bt, out=C), steps, warmup)
        tf = 2.0 * M * N * K / (ms * 1e-3) / 1e12
        out.append({"name": f"vendor_hipblaslt_{name}", "metric": f"torch.matmul bf16 {M}x{N}x{K}",
                    "value": tf, "unit": "TFLOP/s", "ms_per_launch": ms})
    # MIOpen (torch's conv2d, its fastest algorithm for the shape) on the
    # conv2d line's layer; TFLOP/s counts the direct convolution's flops
    torch.backends.cudnn.benchmark = True
    N, C, H, W, OC, k = 32, 64, 56, 56, 64, 3
    x = _rand_f32((N, C, H, W), 15)
    w = _rand_f32((OC, C, k, k), 14, float((2.0 / (C * k * k)) ** 0.5))
    b = (torch.rand(OC, device="cuda") - 0.5) / 8
    ms = _time_launches(lambda i: torch.nn.functional.conv2d(x, w, b, padding=1), steps, warmup)
    tf = 2.0 * N * OC * H * W * C * k * k / (ms * 1e-3) / 1e12
    out.append({"name": "vendor_miopen_conv2d_f32_32x64x56x56_3x3",
                "metric": "torch.nn.functional.conv2d fp32 (direct-convolution flops)",
                "value": tf, "unit": "TFLOP/s", "ms_per_call": ms})
    return out


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def _sha256(*arrays) -> str:
    import hashlib
    h = hashlib.sha256()
    for a in arrays:
        h.update(a.tobytes())
    return h.hexdigest()


def _time_cpu(fn, min_s: float):
    """Seconds per call of fn(), repeated until min_s seconds have passed."""
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= min_s:
            return dt / n, n


def cpu_baseline_c2():
    """The oracle's strict-k fp32 dot on upcast bf16 inputs (momijo's CPU
    engine applied to bf16 data, single thread), on the first 256 rows of the
    exact A and the full B the GPU leg multiplied (about 10 s of CPU work)."""
    import oracle
    oracle.build()
    A, B = _CPU_INPUTS["c2"]
    rows = A.shape[0]
    N, K = B.shape
    t0 = time.perf_counter()
    oracle.gemm_bf16_nt(A, B, rows=(0, rows))
    dt = time.perf_counter() - t0
    flops = 2.0 * rows * N * K
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"C2 row slab: rows 0..{rows - 1} of the GPU leg's A (4096 x 4096) times "
                      f"its full B (N={N}, K={K}), the same bf16 bytes ({dt:.1f} s, "
                      "oracle/momijo_oracle.c mo_gemm_bf16_nt, gcc -O2, 1 thread)",
            "input_sha256": _sha256(A, B), "host_nproc": os.cpu_count(),
            "cpu_model": _cpu_model()}


def cpu_baseline_c3():
    """The W8A16 GEMV restated in the oracle (strict-k fp32 dot per row),
    timed in full on the GPU leg's x, Q, scales and bias, single thread."""
    import oracle
    oracle.build()
    x, Q, s, b = _CPU_INPUTS["c3"]
    per_call, n = _time_cpu(lambda: oracle.linear_w8a16(x, Q, s, b), 2.0)
    bytes_ = Q.size + s.nbytes + x.nbytes + b.nbytes + Q.shape[0] * 2
    return {"value": bytes_ / per_call / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "ms_per_call": per_call * 1e3,
            "sample": f"full C3 (1 x {Q.shape[0]} x {Q.shape[1]}), {n} calls on the GPU leg's "
                      "bytes (oracle mo_linear_w8a16, gcc -O2, 1 thread)",
            "input_sha256": _sha256(x, Q, s, b)}


def cpu_baseline_c1():
    """Linear(256 -> 256) + bias + ReLU as momijo's forward_cpu_parallel
    computes it (oracle), in full, on the GPU leg's x, W and b."""
    import oracle
    oracle.build()
    x, W, b = _CPU_INPUTS["c1"]
    per_call, n = _time_cpu(lambda: oracle.linear_act_f32(x, W, b, oracle.EPI_RELU), 1.0)
    return {"value": 2.0 * 256 ** 3 / per_call / 1e12, "unit": "TFLOP/s", "cores": 1,
            "kind": "port", "ms_per_call": per_call * 1e3,
            "sample": f"full C1 Linear+ReLU 256^3, {n} calls on the GPU leg's bytes "
                      "(oracle mo_linear_act_f32, gcc -O2, 1 thread)",
            "input_sha256": _sha256(x, W, b)}


def cpu_baseline_c3pack():
    """The per-channel RHE quantize/pack restated in the oracle (a division
    and rint per element, as the spec reads), timed in full on the GPU leg's
    W, single thread."""
    import oracle
    oracle.build()
    (W,) = _CPU_INPUTS["c3pack"]
    per_call, n = _time_cpu(lambda: oracle.quantize_rowwise_rhe(W), 2.0)
    N, K = W.shape
    bytes_ = N * K * 4 + N * K + N * 4
    return {"value": bytes_ / per_call / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "ms_per_call": per_call * 1e3,
            "sample": f"full C3-pack ({N} x {K} fp32 -> int8 + scales), {n} calls on the GPU "
                      "leg's W (oracle mo_quantize_rowwise_rhe, gcc -O2, 1 thread)",
            "input_sha256": _sha256(W)}


def cpu_baseline_c4():
    """momijo's Linear loop (strict-k fp32 dot per output, bias after the sum,
    layers.mojo:383-433) on the widened int8 weights with the GELU epilogue
    (oracle mo_linear_w8a16), on a row slab of the GPU leg's x with its full
    weights; every row costs the same, so the slab's rate is the problem's."""
    import oracle
    oracle.build()
    x, Q, s, b, M = _CPU_INPUTS["c4"]
    per_call, n = _time_cpu(lambda: oracle.linear_w8a16(x, Q, s, b, oracle.EPI_GELU_TANH), 2.0)
    rows, K = x.shape
    N = Q.shape[0]
    flops = 2.0 * rows * N * K
    return {"value": flops / per_call / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "ms_per_call": per_call * 1e3,
            "full_problem_s": per_call * M / rows,
            "sample": f"C4 row slab: rows 0..{rows - 1} of the GPU leg's x ({M} x {K}) times its "
                      f"full int8 W ({N} x {K}) + bias + GELU, {n} calls; the full {M} rows "
                      f"extrapolate linearly to {per_call * M / rows:.0f} s (oracle "
                      "mo_linear_w8a16, gcc -O2, 1 thread)",
            "input_sha256": _sha256(x, Q, s, b)}


def cpu_baseline_c5():
    """The FFN restated in the oracle (gate/up dots, silu(g)*u rounded to
    bf16, down dot; strict-k fp32 sums), on a row slab of the GPU leg's x
    with its full weights."""
    import oracle
    oracle.build()
    x, Wg, sg, Wu, su, Wd, sd, M = _CPU_INPUTS["c5"]
    rows, K = x.shape
    per_call, n = _time_cpu(lambda: oracle.mlp_w8a16(x, Wg, sg, Wu, su, Wd, sd), 2.0)
    I = Wg.shape[0]
    flops = 3 * 2.0 * rows * K * I
    return {"value": flops / per_call / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "ms_per_call": per_call * 1e3,
            "full_problem_s": per_call * M / rows,
            "sample": f"C5 row slab: rows 0..{rows - 1} of the GPU leg's x ({M} x {K}) through "
                      f"the full gate/up ({I} x {K}) and down ({Wd.shape[0]} x {I}) int8 "
                      f"weights, {n} calls; the full {M} rows extrapolate linearly to "
                      f"{per_call * M / rows:.0f} s (oracle mo_mlp_w8a16, gcc -O2, 1 thread)",
            "input_sha256": _sha256(x, Wg, sg, Wu, su, Wd, sd)}


def cpu_baseline_conv2d():
    """Conv2d.forward as the reference computes each output (oracle
    mo_conv2d_fw_f32: clipped window, strict c, ky, kx order), on the first
    image of the GPU leg's batch with its weights and bias."""
    import oracle
    oracle.build()
    x, w, b, N = _CPU_INPUTS["conv2d"]
    per_call, n = _time_cpu(lambda: oracle.conv2d_fw_f32(x, w, b, (1, 1), (1, 1)), 2.0)
    _, C, H, W = x.shape
    OC, _, k, _ = w.shape
    flops = 2.0 * OC * H * W * C * k * k
    return {"value": flops / per_call / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "ms_per_call": per_call * 1e3, "full_problem_s": per_call * N,
            "sample": f"image 0 of the GPU leg's batch ({N} images), {n} calls; the full batch "
                      f"extrapolates linearly to {per_call * N:.1f} s (oracle mo_conv2d_fw_f32, "
                      "gcc -O2, 1 thread)",
            "input_sha256": _sha256(x, w, b)}


def main():
    a = _args()
    if a.gpus != 1:
        print(json.dumps({"error": f"--gpus {a.gpus}: this backend is single-GPU; every GPU box "
                                   "in this setup has one GPU, so only --gpus 1 is measured"}))
        sys.exit(2)
    import torch
    import momijo_amd as mj
    if not mj.gpu_available():
        print(json.dumps({"error": "no gfx950 device or libmomijo_hip.so not built"}))
        sys.exit(1)
    torch.cuda.set_device(0)
    global SETTLE_S
    SETTLE_S = max(0.0, a.settle)
    only = set(filter(None, a.only.split(",")))
    want = lambda k: not only or k in only  # noqa: E731

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    head = bench_c2(a.steps, a.warmup) if want("c2") else None
    print(f"# c2 done: {head and round(head['value'], 1)} TFLOP/s", file=sys.stderr, flush=True)
    secondary = []
    for key, fn in (("c3", bench_c3), ("c3batch", bench_c3_batch), ("c3pack", bench_c3_pack),
                    ("c4", bench_c4),
                    ("c4w8a8", bench_c4_w8a8), ("c5", bench_c5), ("c5decode", bench_c5_decode),
                    ("qlinear", bench_qlinear), ("c1", bench_c1),
                    ("bwd", bench_backward), ("conv2d", bench_conv2d),
                    ("f64", bench_f64), ("copy", bench_copy), ("vendor", bench_vendor)):
        if want(key) and (key not in ("copy", "vendor") or key in only):
            rs = fn(a.steps, a.warmup)
            for r in rs if isinstance(rs, list) else [rs]:
                secondary.append(r)
                print(f"# {r['name']} done: {r['value']:.1f} {r['unit']}", file=sys.stderr,
                      flush=True)
    torch.cuda.synchronize()
    gpu_wall = time.perf_counter() - t0

    cpu = None
    if not a.no_cpu:
        if "c2" in _CPU_INPUTS:
            cpu = cpu_baseline_c2()
            print(f"# cpu baseline done: {cpu['value']:.2e} TFLOP/s", file=sys.stderr, flush=True)
        for key, fn in (("c3", cpu_baseline_c3), ("c3pack", cpu_baseline_c3pack),
                        ("c4", cpu_baseline_c4), ("c5", cpu_baseline_c5),
                        ("c1", cpu_baseline_c1), ("conv2d", cpu_baseline_conv2d)):
            if key in _CPU_INPUTS:
                entry = next(r for r in secondary if r["name"].startswith(key + "_"))
                entry["cpu_baseline"] = fn()
                print(f"# {key} cpu baseline done: {entry['cpu_baseline']['value']:.3g} "
                      f"{entry['cpu_baseline']['unit']}", file=sys.stderr, flush=True)

    out = {
        "metric": "GEMM TFLOP/s (% MFMA peak) at 4096^3 bf16; int8 GEMV GB/s (% HBM peak)",
        "value": head["value"] if head else None,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "settle_s": SETTLE_S,
        "ms_per_step": head["ms_per_launch"] if head else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (torch.randn on device, seeded; the CPU leg re-times the same bytes)",
        "config": {"workload": "C2: bf16 NT GEMM M=N=K=4096, fp32 accumulate, bf16 out",
                   "M": 4096, "N": 4096, "K": 4096, "parallelism": "single GPU"},
        "roofline": head["roofline"] if head else None,
        "cpu_baseline": cpu,
        "secondary": secondary,
        "gpu_wall_s": gpu_wall,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
