import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; calls librq.so's C-ABI")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (oracle/oracle.py), built on first use."""
    from oracle import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def gpu():
    """librq on cuda:0. Skips without a GPU; on a GPU box a missing or
    broken librq.so is an error, never a skip."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from rllm_amd.backend import HipBackend

    b = HipBackend(0)
    yield b
    b.synchronize()
    b.close()


@pytest.fixture(params=["dot4", "mfma", "both"])
def gpuk(gpu, request):
    """`gpu` with later uploads laid out for one kernel family (rq_set_kernels;
    "both" holds both layouts and picks per call); tests taking it run once
    per family."""
    gpu.set_kernels(request.param)
    gpu.kernel_family = request.param
    yield gpu
    gpu.set_kernels("auto")
