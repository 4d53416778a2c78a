"""Helpers shared by the GPU tests (conversion between torch and the oracle)."""
import numpy as np
import torch


def bits(x: torch.Tensor) -> np.ndarray:
    """bf16 tensor (any device) -> numpy uint16 bit patterns."""
    return x.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def u8(x: torch.Tensor) -> np.ndarray:
    """fp8 / e8m0 / uint8 tensor (any device) -> numpy uint8."""
    x = x.detach().contiguous().cpu()
    if x.dtype != torch.uint8:
        x = x.view(torch.uint8)
    return x.numpy()


def from_bits(b: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).to(device)


def fp8_dev(q: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(q)).to(device).view(torch.float8_e4m3fn)


def assert_close_to_oracle(y: torch.Tensor, ref: np.ndarray, rel_tol: float = 1e-2,
                           rows: np.ndarray | None = None):
    """GEMM tolerance used throughout (fp32 accumulation + bf16/fp32 rounding of
    the output against a float64 dequantised reference):
      * every finite element: |y - ref| <= 2^-7 |ref| + 2^-12 max|ref|
      * normwise:             max|y - ref| / max|ref| <= rel_tol (north star: 1e-2)
      * every non-finite element of ref (NaN, +-inf) is the same in y, and y
        is non-finite nowhere else.
    rows: the rows to compare (a boolean mask over the first axis, or row
    indices), e.g. oracle.rows_in_groups(ends, M) for an output whose rows
    outside every group the kernel leaves untouched; None compares every row,
    so a reference row that holds a NaN is checked, not skipped."""
    yv = y.detach().float().cpu().numpy().astype(np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if rows is not None:
        yv, ref = yv[rows], ref[rows]
    assert yv.shape == ref.shape, f"shape {yv.shape} != reference {ref.shape}"
    if ref.size == 0:
        return
    fin = np.isfinite(ref)
    bad = ~fin & ~((yv == ref) | (np.isnan(yv) & np.isnan(ref)))
    assert not bad.any(), (
        f"non-finite reference not matched at {np.argwhere(bad)[0]}: "
        f"got {yv[tuple(np.argwhere(bad)[0])]}")
    stray = fin & ~np.isfinite(yv)
    assert not stray.any(), f"non-finite output at {np.argwhere(stray)[0]} (reference finite)"
    if not fin.any():
        return
    yv, ref = np.where(fin, yv, 0.0), np.where(fin, ref, 0.0)
    scale = np.abs(ref).max()
    err = np.abs(yv - ref)
    bound = 2.0 ** -7 * np.abs(ref) + 2.0 ** -12 * scale
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    assert np.all(err <= bound), (
        f"elementwise bound violated at {worst}: got {yv[worst]}, ref {ref[worst]}")
    assert err.max() / max(scale, 1e-300) <= rel_tol
