import os
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); runs the HIP kernels")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this process")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def assert_close(got: torch.Tensor, ref: torch.Tensor, rtol: float, what: str = "") -> None:
    """|got - ref| <= rtol * |ref| + rtol * max|ref| elementwise (the atol floor keeps
    near-zero elements of a large-magnitude output from failing on rtol alone)."""
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    assert got.shape == ref.shape, f"{what}: shape {tuple(got.shape)} vs {tuple(ref.shape)}"
    assert torch.isfinite(got).all(), f"{what}: non-finite values"
    scale = ref.abs().max().item() if ref.numel() else 0.0
    err = (got - ref).abs()
    bound = rtol * ref.abs() + rtol * scale
    bad = err > bound
    if bad.any():
        i = int(torch.argmax((err - bound).reshape(-1)))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{ref.numel()} elements out of tolerance rtol={rtol}; "
            f"worst at flat index {i}: got {got.reshape(-1)[i].item():.6g}, "
            f"ref {ref.reshape(-1)[i].item():.6g}, max|ref| {scale:.4g}")


def tol(dtype: torch.dtype) -> float:
    return 1e-4 if dtype == torch.float32 else 2e-2
