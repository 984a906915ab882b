"""Test setup: the `gpu` marker, import paths, and shared helpers.

GPU tests (marked gpu) call libmdx through its C ABI (via the mdx._C shim) on the ROCm device and
compare against the CPU oracle; everything else runs on the CPU."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "comfy-mono-decode-xpu_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device) and the built libmdx.so")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda", 0)


@pytest.fixture(scope="session")
def C(dev):
    """The product operator surface; its library must load (no silent fallback)."""
    from mdx import _C, _lib
    _lib.lib()
    return _C


def bits(t):
    """A tensor's raw bits as a numpy array (bf16/fp16 -> uint16, f32 -> uint32, ints as is)."""
    import torch
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.numpy()


def assert_bits_equal(got, want, what=""):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    bad = got != want
    if bad.any():
        idx = np.argwhere(bad)[:5]
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} differ; first at {idx.tolist()}: "
                             f"got {got[tuple(idx[0])]} want {want[tuple(idx[0])]}")
