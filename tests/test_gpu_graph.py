"""Entry points and HIP graph capture (torch.cuda.graph).

Calls that need the library's per-stream workspace (the split-K W8A16 GEMM,
QuantLinear, the W8A8 Linear) are refused under capture with
MJ_ERR_UNSUPPORTED.  test_graph_replays_match_eager is the earlier design,
in which such calls took stream-ordered allocations owned by the graph; it
is skipped: one run of it (with the W8A8 Linear in the captured sequence,
after the int8 suites in the same process) faulted the GPU and the cause was
not found, so that code path was removed.
"""
import numpy as np
import pytest
import torch

import momijo_amd as mj
from _util import bf16_host_bits, to_dev

pytestmark = pytest.mark.gpu


def test_capture_refuses_workspace_calls(oracle, dev):
    """A call that needs the per-stream workspace raises under capture and
    enqueues nothing; the same call works eagerly afterwards."""
    K = 1024
    W = oracle.randn_f32((256, K), std=0.02, seed=81)
    q, s = mj.quantize_rowwise_int8(to_dev(W, dev))
    lin8 = mj.W8A8Linear(q, s)
    x = torch.ones((64, K), dtype=torch.bfloat16, device=dev)
    y = torch.empty((64, 256), dtype=torch.bfloat16, device=dev)
    lin8.forward(x, out=y)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(mj.MomijoHipError, match="graph capture"):
        with torch.cuda.graph(graph):
            lin8.forward(x, out=y)
    torch.cuda.synchronize()
    want = bf16_host_bits(y).copy()
    y.zero_()
    lin8.forward(x, out=y)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bf16_host_bits(y), want)
    assert np.any(want != 0)


@pytest.mark.skip(reason="faulted the GPU once (workspace calls captured with graph-owned "
                         "allocations, W8A8 Linear included, run after the int8 suites); cause "
                         "not found, and capture of workspace calls is now refused")
def test_graph_replays_match_eager(oracle, dev):
    K = 4096
    W = oracle.randn_f32((1024, K), std=0.02, seed=71)
    q, s = mj.quantize_rowwise_int8(to_dev(W, dev))
    b = to_dev(oracle.randu_f32((1024,), -0.0625, 0.0625, seed=72), dev)
    lin = mj.W8Linear(q, s, b, mj.EPI_GELU_TANH)   # M = 64 at K = 4096: split K
    lin8 = mj.W8A8Linear(q, s, b, mj.EPI_RELU)     # row quantize + int8 GEMM
    Wq8 = torch.randint(-127, 128, (384, 512), dtype=torch.int8, device=dev)
    ql = mj.QuantLinear(512, 384, mj.Tensor(Wq8),
                        mj.Tensor(to_dev(oracle.randu_f32((384,), -1, 1, seed=73), dev)),
                        0.01, 0.02)

    x64 = torch.empty((64, K), dtype=torch.bfloat16, device=dev)
    x1 = torch.empty((1, K), dtype=torch.bfloat16, device=dev)
    xf = torch.empty((256, 512), dtype=torch.float32, device=dev)
    A = torch.empty((512, 1024), dtype=torch.bfloat16, device=dev)
    B = torch.empty((768, 1024), dtype=torch.bfloat16, device=dev)
    y64 = torch.empty((64, 1024), dtype=torch.bfloat16, device=dev)
    y1 = torch.empty((1, 1024), dtype=torch.bfloat16, device=dev)
    y8 = torch.empty((64, 1024), dtype=torch.bfloat16, device=dev)
    C = torch.empty((512, 768), dtype=torch.bfloat16, device=dev)
    yq = [None]

    def fill(seed):
        g = torch.Generator(device=dev).manual_seed(seed)
        for t in (x64, x1, A, B):
            t.copy_(torch.randn(t.shape, generator=g, device=dev).to(torch.bfloat16))
        xf.copy_(torch.randn(xf.shape, generator=g, device=dev))

    def run():
        lin.forward(x64, out=y64)
        lin.forward(x1, out=y1)
        lin8.forward(x64, out=y8)
        yq[0] = ql.forward(mj.Tensor(xf)).torch
        mj.gemm_bf16_nt(A, B, out=C)

    def outputs():
        return [bf16_host_bits(y64), bf16_host_bits(y1), yq[0].cpu().numpy().copy(),
                bf16_host_bits(C), bf16_host_bits(y8)]

    # eager warm-up on a side stream (kernel attributes set, workspaces made)
    fill(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    torch.cuda.synchronize()
    graph_yq = yq[0]

    names = ("W8A16 split-K GEMM", "K-split GEMV", "QuantLinear", "bf16 GEMM", "W8A8 Linear")
    for rep in range(3):
        fill(rep + 1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        yq[0] = graph_yq
        got = outputs()
        run()                          # eager, same inputs
        torch.cuda.synchronize()
        want = outputs()
        for name, g_, w_ in zip(names, got, want):
            np.testing.assert_array_equal(g_, w_, err_msg=f"replay {rep}: {name}")
        assert np.any(got[0] != 0) and np.all(np.isfinite(got[2]))
