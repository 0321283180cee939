import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The HIP device; GPU tests fail (never skip to a fallback) without the library."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from qwen3_engine_from_scratch_amd import _lib

    _lib.load()
    return torch.device("cuda:0")


def announce(msg: str) -> None:
    """Names the case on stdout before a GPU step, flushed, so a log that ends
    abruptly still says what was running."""
    sys.stdout.write(f"[case] {msg}\n")
    sys.stdout.flush()


os.environ.setdefault("PYTHONUNBUFFERED", "1")
