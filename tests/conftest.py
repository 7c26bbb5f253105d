import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: long-running CPU oracle case")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def dev():
    """The GPU device; GPU tests fail (not skip) when no GPU is present."""
    import torch
    assert torch.cuda.is_available(), "gpu-marked test run without a visible GPU"
    import evk_amd
    assert evk_amd.available(), "libevkhip.so not built (python -m evk_amd.build)"
    evk_amd.initialize()
    return torch.device("cuda:0")


def to_dev(x: np.ndarray, device):
    """numpy uint16 fp16 bits -> torch fp16 tensor on device."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.uint16).view(np.int16))
    return t.view(torch.float16).to(device)


def from_dev(t) -> np.ndarray:
    """torch fp16/int16 tensor -> numpy uint16 bits."""
    import torch
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.float16:
        t = t.view(torch.int16)
    return t.numpy().view(np.uint16)


def f32(h: np.ndarray) -> np.ndarray:
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def assert_close_f16(got_bits, want_bits, atol=1e-2, rtol=1e-2, what=""):
    g, w = f32(got_bits), f32(want_bits)
    assert g.shape == w.shape, (g.shape, w.shape)
    assert np.all(np.isfinite(g)), f"{what}: non-finite output"
    err = np.abs(g - w)
    lim = atol + rtol * np.abs(w)
    bad = err > lim
    if bad.any():
        i = np.unravel_index(np.argmax(err - lim), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} / {bad.size} outside tol; worst at {i}: "
                             f"got {g[i]} want {w[i]} (max abs err {err.max():.4g})")
