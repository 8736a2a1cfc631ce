import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libkanso_hip.so)")


@pytest.fixture(scope="session")
def ctx():
    """One kanso context on cuda:0 for the whole GPU session."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    import kanso_infer_amd as K
    c = K.Context(0)
    yield c
    c.close()
