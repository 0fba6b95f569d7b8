import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "mimo-prismwing_amd", "oracle"):
    path = os.path.join(ROOT, sub)
    if path not in sys.path:
        sys.path.insert(0, path)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def golden_dir():
    return GOLDEN


@pytest.fixture(scope="session")
def rt():
    """One runtime on device 0 for the whole GPU session (the library must be built)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import prismwing_amd as P
    runtime = P.WideMoeRuntime.compile(0)
    yield runtime
    runtime.close()
