"""Shared pytest setup: the ``gpu`` marker and import paths.

GPU tests (``-m gpu``) run the HIP library on an MI355X and compare it with
the CPU oracle in ``oracle/`` (test infrastructure only).  Everything else runs
on the CPU.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    name = torch.cuda.get_device_properties(0).gcnArchName
    assert name.startswith("gfx950"), f"tests target gfx950, found {name}"
    return torch.device("cuda:0")
