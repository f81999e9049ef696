import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
for p in (REPO, HERE):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: takes more than a few seconds")


def _ensure_built():
    """Builds the HIP library, its PyTorch binding and the oracle only if they are missing."""
    import importlib.util

    path = os.path.join(REPO, "bit_reproducible_training_amd", "_build.py")
    spec = importlib.util.spec_from_file_location("_rg_build", path)
    build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(build)
    if not (os.path.exists(build.LIB_PATH) and os.path.exists(build.binding_path())):
        build.build()
    if not os.path.exists(os.path.join(REPO, "oracle", "liboracle.so")):
        from oracle import oracle  # noqa: F401  (builds on import when missing)


_ensure_built()


@pytest.fixture(scope="session")
def torch_gpu():
    import torch

    from bit_reproducible_training_amd import _lib

    if not torch.cuda.is_available():
        pytest.fail("GPU test requested but torch.cuda is not available")
    runtimes = _lib.hip_runtimes_mapped()
    print("HIP runtime(s) mapped:", runtimes, flush=True)
    assert len(runtimes) == 1, "two HIP runtimes in one process: %s" % runtimes
    return torch
