import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built kernel library")


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("GPU tests need a visible MI355X; run them with -m gpu on the GPU box")
    from snowllm_amd import ops  # noqa: F401  (fails loudly if the library is missing)
    return torch.device("cuda")
