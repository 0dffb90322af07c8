import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an AMD GPU and the built libtropnn_hip.so")
    config.addinivalue_line("markers", "slow: minutes of CPU work; skipped unless TROPNN_SLOW_TESTS=1")
