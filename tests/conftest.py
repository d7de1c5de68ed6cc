import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    """The oracle library (test infrastructure)."""
    from oracle import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def gpu_stream():
    """One stream for the GPU tests, made torch's current stream: tensors the tests create, fill and
    read, and the library's kernels (a context bound to it), are ordered on it."""
    import torch

    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    yield stream
    torch.cuda.synchronize()


@pytest.fixture(scope="module")
def tk(gpu_stream):
    """A library context on the tests' stream."""
    import telmo_amd

    k = telmo_amd.Kernels(0, stream=gpu_stream.cuda_stream)
    yield k
    k.close()
