"""Shared helpers of the GPU parity tests (device buffers from torch, the HIP
path through the C ABI, the CPU oracle as the checker)."""
import numpy as np
import torch

FP32_TOL = 1e-4   # max relative error, fp32
BF16_TOL = 2e-2   # max relative error, bf16


def require_gpu():
    if not torch.cuda.is_available():
        raise RuntimeError("GPU tests need an MI355X (torch.cuda.is_available() is False)")


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even to bf16, returned as float32 (what the kernels read)."""
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def dev(a: np.ndarray, dtype=torch.float32) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dtype).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def relerr(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(float(np.max(np.abs(b))), 1e-30))


def assert_close(got, ref, tol, what="", floor=None):
    """max|a-b|/max|b| <= tol and, element-wise, |a-b| <= tol*max(|b|, rms(b)),
    or <= floor where an element-wise error model (an array like ref) allows more."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    r = relerr(got, ref)
    assert r <= tol, f"{what}: max relative error {r:.3e} > {tol:.0e}"
    rms = float(np.sqrt(np.mean(ref ** 2))) if ref.size else 0.0
    bound = tol * np.maximum(np.abs(ref), rms)
    if floor is not None:
        bound = np.maximum(bound, floor)
    bad = np.abs(got - ref) > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} elements outside the element-wise bound"
    return r
