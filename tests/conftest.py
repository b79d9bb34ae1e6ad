"""Shared pytest setup: import paths, the `gpu` marker, device fixtures."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (str(ROOT / "convrot-mlx_amd"), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device) and the built HIP library")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm device visible")
    from convrot_mlx_amd import _native

    _native.load()  # fail loudly if the HIP library is missing
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle

    oracle.build()
    return oracle


@pytest.fixture
def tuning():
    """set(name, value) forces a kernel / plan choice of the HIP library for one test
    (convrot_set_tuning); every override is restored to automatic at teardown."""
    from convrot_mlx_amd import _native

    used = set()

    class _Tuning:
        def set(self, name, value):
            used.add(name)
            _native.set_tuning(name, value)

    yield _Tuning()
    for name in used:
        _native.set_tuning(name, None)


@pytest.fixture
def fp6_form():
    """set(form) picks the FP6 weight form ConvRotLinear caches for one test
    (set_fp6_weight_form); "auto" is restored at teardown."""
    from convrot_mlx_amd import core

    yield core.set_fp6_weight_form
    core.set_fp6_weight_form("auto")
