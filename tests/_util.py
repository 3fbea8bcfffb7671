"""Helpers shared by the tests: seeded inputs from the oracle's RNG and the
host/device conversions of bf16 bit patterns."""
import numpy as np
import torch


def to_dev(a: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def bf16_dev(u16: np.ndarray, device) -> torch.Tensor:
    """uint16 bf16 bit patterns -> a torch.bfloat16 device tensor."""
    return torch.from_numpy(np.ascontiguousarray(u16).view(np.int16)).view(torch.bfloat16).to(device)


def bf16_host_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def bf16_host_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def normwise_rel(got: np.ndarray, ref: np.ndarray) -> float:
    """max|got - ref| / max|ref|: the relative error used for bf16 results
    (elementwise relative error is ill-posed near zero)."""
    denom = float(np.max(np.abs(ref)))
    return float(np.max(np.abs(got.astype(np.float64) - ref.astype(np.float64)))) / max(denom, 1e-30)


def assert_close_f32(got: np.ndarray, ref: np.ndarray, atol=1e-5, rtol=1e-5):
    """fp32 bar: |got - ref| <= atol + rtol*|ref| elementwise."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    tol = atol + rtol * np.abs(ref)
    bad = err > tol
    assert not bad.any(), (
        f"{int(bad.sum())} of {bad.size} elements out of tolerance; worst |err|={err.max():.3e}, "
        f"at ref={ref.flat[int(np.argmax(err))]:.6g}")


def slab_rows(M: int, block: int = 128) -> list[int]:
    """One row in every block of `block` rows (at a position that moves from
    block to block), plus the first and last row."""
    rows = {0, M - 1}
    for t in range((M + block - 1) // block):
        rows.add(min(M - 1, t * block + (37 * t + 5) % block))
    return sorted(rows)


def slab_cols(N: int, block: int = 256) -> list[int]:
    """Two columns in every block of `block` columns, plus the first and last."""
    cols = {0, N - 1}
    for t in range((N + block - 1) // block):
        cols.add(min(N - 1, t * block + (91 * t + 11) % block))
        cols.add(min(N - 1, t * block + (131 * t + 200) % block))
    return sorted(cols)


def assert_tiles_covered(M: int, N: int, rows, cols, bm: int = 128, bn: int = 64) -> None:
    """Every bm x bn block of the [M, N] output holds a checked element: the
    row slabs check whole rows and the column slabs whole columns.  (Any
    kernel tile at least bm x bn in size is then checked.)"""
    hit = np.zeros(((M + bm - 1) // bm, (N + bn - 1) // bn), bool)
    for r in rows:
        hit[r // bm, :] = True
    for c in cols:
        hit[:, c // bn] = True
    assert hit.all(), f"{int((~hit).sum())} output blocks unchecked"
