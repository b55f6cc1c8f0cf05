"""Test configuration: import paths, the ``gpu`` marker, oracle registration.

``-m "not gpu"`` runs on any machine (oracle vs golden vectors, host logic,
the C-ABI library's exports); ``-m gpu`` needs a HIP device and runs the HIP
implementation against the oracle.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "ace-kernels_amd", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a HIP (MI355X) device and libace_hip.so")


def pytest_collection_modifyitems(config: pytest.Config, items) -> None:
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP device")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session", autouse=True)
def _register_oracle_impls():
    """The oracle's reference loss as registry impl ``reference`` (tests only)."""
    from oracle.reference import register_reference
    from oracle.v2 import register_v2

    register_reference()
    register_v2()
