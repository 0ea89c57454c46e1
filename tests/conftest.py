import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# Parity bar (fp16 I/O, fp32 accumulate) against the fp32 oracle.
ATOL = 2e-3
RTOL = 1e-2


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (gfx950); runs the native kernels")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP device in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def native_lib():
    """The built library (built here once if it is missing)."""
    from custom_inference_engine_amd import _build, _native

    if not os.path.exists(_build.LIB_PATH):
        _build.build()
    return _native.load()


def assert_attn_close(out: torch.Tensor, ref: torch.Tensor, atol: float = ATOL, rtol: float = RTOL,
                      what: str = "") -> float:
    """|out - ref| <= atol + rtol * |ref| elementwise; returns the max abs error."""
    out = out.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert out.shape == ref.shape, (out.shape, ref.shape)
    assert torch.isfinite(out).all(), f"{what}: non-finite output"
    err = (out - ref).abs()
    bound = atol + rtol * ref.abs()
    bad = err > bound
    max_abs = float(err.max()) if err.numel() else 0.0
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} of {err.numel()} elements out of tolerance; "
        f"max abs err {max_abs:.3e} (atol {atol}, rtol {rtol})"
    )
    return max_abs
