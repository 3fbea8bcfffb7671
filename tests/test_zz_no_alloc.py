"""mj_quant_linear_f32_noalloc (the allocation-free variant of QuantLinear's
entry point, its int8 copy of x in a static device array) against
mj_quant_linear_f32 through the C ABI, bit for bit, on two calls in a row
(the second smaller, so stale scratch contents from the first would show),
on both GEMM paths (int8 MFMA and the scalar / legacy-literal kernel), plus
the oracle and the size limit."""
import numpy as np
import pytest
import torch

from momijo_amd import _lib
from _util import to_dev

pytestmark = pytest.mark.gpu

LIMIT = (16 << 20) - 16   # bytes of int8 x the static scratch holds


def _case(oracle, M, N, K, seed):
    x = oracle.randn_f32((M, K), seed=seed) * np.float32(2)
    W = oracle.randn_f32((N, K), std=0.1, seed=seed + 1)
    b = oracle.randu_f32((N,), -0.1, 0.1, seed=seed + 2)
    s_x, s_w = oracle.minmax_scale_symmetric(x), oracle.minmax_scale_symmetric(W)
    return x, oracle.quantize_symmetric_int8(W, s_w), b, s_w, s_x


def _run(fn, dev, x, Wq, b, s_w, s_x, legacy):
    M, K = x.shape
    N = Wq.shape[0]
    tx, tw, tb = to_dev(x, dev), to_dev(Wq, dev), to_dev(b, dev)
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    _lib.call(fn, tx.data_ptr(), tw.data_ptr(), tb.data_ptr(), np.float32(s_w), np.float32(s_x),
              y.data_ptr(), M, N, K, legacy, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("legacy", [0, 1])
def test_noalloc_matches_allocating_entry_point(oracle, dev, legacy):
    # first call: 600 x 4096 int8 of x (2.4 MB of the scratch); second: smaller
    for (M, N, K, seed) in ((600, 300, 4096, 1), (37, 53, 80 if legacy else 96, 7)):
        case = _case(oracle, M, N, K, seed)
        got = _run("mj_quant_linear_f32_noalloc", dev, *case, legacy)
        ref = _run("mj_quant_linear_f32", dev, *case, legacy)
        np.testing.assert_array_equal(got, ref)
        np.testing.assert_array_equal(got, oracle.quant_linear_fw(*case, bool(legacy)))


def test_noalloc_rejects_sizes_beyond_the_scratch(dev):
    lib = _lib.load()
    p = 4096  # never dereferenced: the size check comes first
    M, K = 4097, 4096   # 16 MiB + 4 KiB of int8 x
    st = lib.mj_quant_linear_f32_noalloc(p, p, p, 1.0, 1.0, p, M, 8, K, 0, None)
    assert st == _lib.MJ_ERR_UNSUPPORTED
    assert "static scratch" in lib.mj_last_error().decode()
    assert M * K > LIMIT
