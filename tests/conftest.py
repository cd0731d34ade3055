"""Shared test configuration.

Markers: ``gpu`` -- needs an MI355X (gfx950) and the built HIP library.
Everything unmarked runs on the CPU.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: test needs an MI355X GPU and the built HIP library")


def golden(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def normwise_rel(got, ref):
    """max|got - ref| / max|ref| (max|ref| floored at 1e-30)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if ref.size == 0:
        return 0.0
    return float(np.max(np.abs(got - ref)) / max(float(np.max(np.abs(ref))), 1e-30))


@pytest.fixture(scope="session")
def gpu_ctx():
    """A Context on torch's current stream (torch only provides device memory)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import ferrograd_amd as fa

    ctx, _stream = fa.torch_context(0)
    yield ctx
    ctx.sync()
    ctx.close()
