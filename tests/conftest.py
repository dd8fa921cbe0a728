import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(ROOT, "llm_quantization-kernel_amd")
for p in (ROOT, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture
def emu():
    """Run the ops host logic on the CPU oracle (oracle.emulator injected as the backend)."""
    from crispybits_kernels import ops
    from oracle import emulator
    prev = ops._C
    ops.set_backend(emulator)
    yield "cpu"
    ops.set_backend(prev)


@pytest.fixture
def hip():
    """The gfx950 backend; fails (does not skip) when the library or GPU is missing."""
    import torch
    from crispybits_kernels import ops
    assert ops._CUDA is not None, f"HIP library not loaded: {ops._IMPORT_ERROR}"
    assert torch.cuda.is_available(), "no GPU visible"
    prev = ops._C
    ops.set_backend("cuda")
    yield "cuda"
    ops.set_backend(prev)
