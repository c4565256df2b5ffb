import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")
REF_ADAM = os.path.join(ROOT, "oracle", "_ref", "cpu_adam_ref.so")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU")
    config.addinivalue_line("markers", "slow: long-running GPU test at full layer size")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a host without a GPU")
    return torch.device("cuda", 0)


def load_ref_adam():
    """The reference's CPU Adam compiled from its sources (oracle/_ref), or None."""
    if not os.path.exists(REF_ADAM):
        return None
    import importlib.util

    import torch  # noqa: F401  (the extension links libtorch)

    spec = importlib.util.spec_from_file_location("cpu_adam_ref", REF_ADAM)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod
