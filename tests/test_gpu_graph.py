"""Entry points and HIP graph capture (torch.cuda.graph).

Calls that need the library's per-stream workspace (the split-K W8A16 GEMM,
the FFN when its down projection splits K, QuantLinear, the W8A8 Linear,
Linear.backward's column sums beyond 1024 rows, the min/max observer) are
refused under capture with MJ_ERR_UNSUPPORTED before they enqueue anything:
the captured graph holds no node of theirs.  test_graph_replays_match_eager
is the earlier design, in which such calls took stream-ordered allocations
owned by the graph; it is skipped: one run of it (with the W8A8 Linear in the
captured sequence, after the int8 suites in the same process) faulted the
GPU and the cause was not found, so that code path was removed.
"""
import ctypes
import threading

import numpy as np
import pytest
import torch

import momijo_amd as mj
from momijo_amd import _lib
from _util import bf16_host_bits, to_dev

pytestmark = pytest.mark.gpu


def _hip_runtime():
    """The HIP runtime torch has loaded (its path from /proc/self/maps)."""
    with open("/proc/self/maps") as f:
        for line in f:
            if "libamdhip64.so" in line:
                return ctypes.CDLL(line.split()[-1])
    raise RuntimeError("libamdhip64 is not loaded")


def graph_nodes(graph: torch.cuda.CUDAGraph) -> int:
    """Number of nodes of a captured graph (kept with keep_graph=True)."""
    hip = _hip_runtime()
    hip.hipGraphGetNodes.argtypes = [ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.POINTER(ctypes.c_size_t)]
    n = ctypes.c_size_t(0)
    assert hip.hipGraphGetNodes(ctypes.c_void_p(graph.raw_cuda_graph()), None,
                                ctypes.byref(n)) == 0
    return int(n.value)


def refused_under_capture(fn) -> int:
    """Runs fn under capture, expects the workspace refusal, and returns the
    number of nodes the capture recorded."""
    graph = torch.cuda.CUDAGraph(keep_graph=True)
    with pytest.raises(mj.MomijoHipError, match="graph capture"):
        with torch.cuda.graph(graph):
            fn()
    torch.cuda.synchronize()
    return graph_nodes(graph)


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
    assert refused_under_capture(lambda: lin8.forward(x, out=y)) == 0
    want = bf16_host_bits(y).copy()
    y.zero_()
    lin8.forward(x, out=y)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bf16_host_bits(y), want)
    assert np.any(want != 0)


def test_capture_refuses_backward_and_observer(oracle, dev):
    """Linear.backward at N = 2048 rows (its column sums use the workspace)
    and the min/max observer raise under capture with an empty graph; dx and
    dW, which would run before the column sums, are not enqueued either."""
    N, InF, OutF = 2048, 256, 384
    lin = mj.Linear(InF, OutF)
    lin.weight.torch.copy_(to_dev(oracle.randn_f32((OutF, InF), seed=82), dev))
    x = mj.Tensor(to_dev(oracle.randn_f32((N, InF), seed=83), dev))
    dy = mj.Tensor(to_dev(oracle.randn_f32((N, OutF), seed=84), dev))
    dW0, db0, dx0 = (t.numpy() for t in lin.backward(x, dy))
    torch.cuda.synchronize()
    assert refused_under_capture(lambda: lin.backward(x, dy)) == 0
    dW1, db1, dx1 = (t.numpy() for t in lin.backward(x, dy))
    np.testing.assert_array_equal(dW1, dW0)
    np.testing.assert_array_equal(db1, db0)
    np.testing.assert_array_equal(dx1, dx0)

    obs = mj.MinMaxObserver()
    xs = mj.Tensor(to_dev(oracle.randn_f32((4096,), seed=85), dev))
    assert refused_under_capture(lambda: obs.observe(xs)) == 0
    assert not obs.has_data
    assert refused_under_capture(lambda: mj.functional.scale_symmetric_device(xs)) == 0
    obs.observe(xs)
    ref = oracle.randn_f32((4096,), seed=85)
    assert (obs.min_v, obs.max_v) == (float(ref.min()), float(ref.max()))


def test_capture_refuses_split_ffn_before_gate_up(oracle, dev):
    """The FFN at M = 512 splits its down projection's K: capture is refused
    before the gate/up GEMM (which needs no workspace) is enqueued."""
    M, K, I, H = 512, 1024, 2048, 1024
    mk = lambda n, k, seed: mj.W8Linear(*mj.quantize_rowwise_int8(  # noqa: E731
        to_dev(oracle.randn_f32((n, k), std=0.02, seed=seed), dev)))
    mlp = mj.W8MLP(mk(I, K, 86), mk(I, K, 87), mk(H, I, 88))
    x = to_dev(oracle.f32_to_bf16(oracle.randn_f32((M, K), seed=89)).view(np.int16),
               dev).view(torch.bfloat16)
    h = torch.zeros((M, I), dtype=torch.bfloat16, device=dev)
    y = torch.zeros((M, H), dtype=torch.bfloat16, device=dev)
    assert refused_under_capture(lambda: mlp.forward(x, h, y)) == 0
    assert not torch.any(h != 0).item() and not torch.any(y != 0).item()
    mlp.forward(x, h, y)
    torch.cuda.synchronize()
    assert torch.any(y != 0).item()


@pytest.mark.parametrize("shared", [True, False], ids=["shared-stream", "per-thread-stream"])
def test_workspace_calls_from_two_threads(oracle, dev, shared):
    """Two host threads issue W8A8 Linears (row quantize into the workspace,
    then the int8 GEMM reading it) with different inputs, either on one
    shared stream or on hipStreamPerThread; every result equals the eager
    single-thread result of its input."""
    M, N, K = 256, 512, 1024
    W = oracle.randn_f32((N, K), std=0.02, seed=90)
    q, s = mj.quantize_rowwise_int8(to_dev(W, dev))
    lin8 = mj.W8A8Linear(q, s)
    xs = [to_dev(oracle.f32_to_bf16(oracle.randn_f32((M, K), seed=91 + t)).view(np.int16),
                 dev).view(torch.bfloat16) for t in range(2)]
    want = [bf16_host_bits(lin8.forward(x)) for x in xs]
    torch.cuda.synchronize()
    reps = 24
    outs = [[torch.empty((M, N), dtype=torch.bfloat16, device=dev) for _ in range(reps)]
            for _ in range(2)]
    stream = torch.cuda.Stream() if shared else None
    handle = stream.cuda_stream if shared else 2      # hipStreamPerThread
    errors = []
    start = threading.Barrier(2)

    def work(t):
        try:
            torch.cuda.set_device(0)
            start.wait()
            for r in range(reps):
                _lib.call("mj_linear_w8a8", xs[t].data_ptr(), q.data_ptr(), s.data_ptr(), None,
                          _lib.EPI_NONE, outs[t][r].data_ptr(), M, N, K, handle)
            _lib.call("mj_stream_synchronize", handle)
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(e)

    threads = [threading.Thread(target=work, args=(t,)) for t in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for t in range(2):
        for r in range(reps):
            np.testing.assert_array_equal(bf16_host_bits(outs[t][r]), want[t],
                                          err_msg=f"thread {t} call {r}")


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


def test_decode_ffn_graph_replays_match_eager(oracle, dev):
    """The FFN at one x row needs no workspace (gate/up GEMV, then the down
    GEMV at K = 11008): it captures, and three replays over fresh inputs, with
    eager calls and synchronizations between them, equal the eager result bit
    for bit."""
    K, I, H = 4096, 11008, 4096
    mk = lambda n, k, seed: mj.W8Linear(*mj.quantize_rowwise_int8(  # noqa: E731
        to_dev(oracle.randn_f32((n, k), std=0.02, seed=seed), dev)))
    mlp = mj.W8MLP(mk(I, K, 90), mk(I, K, 91), mk(H, I, 92))
    x = torch.empty((1, K), dtype=torch.bfloat16, device=dev)
    h = torch.empty((1, I), dtype=torch.bfloat16, device=dev)
    y = torch.empty((1, H), dtype=torch.bfloat16, device=dev)

    def fill(seed):
        g = torch.Generator(device=dev).manual_seed(seed)
        x.copy_(torch.randn(x.shape, generator=g, device=dev).to(torch.bfloat16))

    fill(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mlp.forward(x, h, y)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph(keep_graph=True)
    with torch.cuda.graph(graph):
        mlp.forward(x, h, y)
    torch.cuda.synchronize()
    assert graph_nodes(graph) == 2
    graph.instantiate()
    for rep in range(3):
        fill(rep + 1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = (bf16_host_bits(h), bf16_host_bits(y))
        mlp.forward(x, h, y)
        torch.cuda.synchronize()
        want = (bf16_host_bits(h), bf16_host_bits(y))
        np.testing.assert_array_equal(got[0], want[0], err_msg=f"replay {rep}: h")
        np.testing.assert_array_equal(got[1], want[1], err_msg=f"replay {rep}: y")
        assert np.any(got[1] != 0)
