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


def assert_close_to_oracle(y: torch.Tensor, ref: np.ndarray, rel_tol: float = 1e-2):
    """GEMM tolerance used throughout (fp32 accumulation + bf16/fp32 rounding of
    the output against a float64 dequantised reference):
      * every element: |y - ref| <= 2^-7 |ref| + 2^-12 max|ref|
      * normwise:      max|y - ref| / max|ref| <= rel_tol (north star: 1e-2)
    Rows of `ref` that are NaN (outside every group) are skipped."""
    yv = y.detach().float().cpu().numpy().astype(np.float64)
    ok = ~np.isnan(ref).any(axis=tuple(range(1, ref.ndim))) if ref.ndim > 1 else ~np.isnan(ref)
    yv, ref = yv[ok], ref[ok]
    if ref.size == 0:
        return
    scale = np.abs(ref).max()
    err = np.abs(yv - ref)
    bound = 2.0 ** -7 * np.abs(ref) + 2.0 ** -12 * scale
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    assert np.all(err <= bound), (
        f"elementwise bound violated at {worst}: got {yv[worst]}, ref {ref[worst]}")
    assert err.max() / max(scale, 1e-300) <= rel_tol
