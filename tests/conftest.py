"""Shared pytest setup: import paths, the `gpu` marker and device fixtures.

Tests marked `gpu` need a HIP device and the built library; they fail (not skip) when either is
missing, so a GPU run can never pass on a host-only path.
"""

from __future__ import annotations

import pathlib
import sys

import pytest

REPO = pathlib.Path(__file__).resolve().parents[1]
for p in (REPO, REPO / "plastic-infer_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a HIP (ROCm) device and the built library")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available() or torch.version.hip is None:
        pytest.fail("this test needs a HIP device (run the gpu-marked tests on an MI355X)")
    from plastic_infer import _native

    _native.load()
    d = torch.device("cuda", 0)
    torch.cuda.set_device(d)
    return d
