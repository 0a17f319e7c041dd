import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
for p in (ROOT / "infer-llm_amd", ROOT / "oracle", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X; runs on the GPU box")


@pytest.fixture(scope="session")
def dev():
    """The GPU. GPU tests fail (not skip) without one: they must run the HIP path."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def oracle_pool():
    """The oracle's worker pool: the reference default (half the hardware
    threads), capped at 8 workers to stay inside one GPU box's CPU share."""
    import oracle

    n = min(oracle.default_workers(), 8)
    return oracle.set_workers(n)
