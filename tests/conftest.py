"""Shared test setup.

Tiers: tests marked ``gpu`` run the HIP path on an MI355X and compare it with
the CPU oracle (``oracle/``); everything else runs on CPU (oracle vs golden
fixtures, host logic, C-ABI loading and argument validation).
"""
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PACKAGE_ROOT = ROOT / "parrot-h200-worker_amd"
GOLDEN = ROOT / "tests" / "golden"
for p in (str(ROOT), str(PACKAGE_ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm) GPU and the built HIP library")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def golden():
    def load(name):
        return np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    return load


@pytest.fixture(scope="session")
def tiny_cfg():
    from oracle.parrot_fp32 import tiny_config
    return tiny_config()


def tiny_model_config(**overrides):
    from oracle.parrot_fp32 import tiny_config
    from parrot import ModelConfig
    fields = dict(vars(tiny_config()))
    fields.update(overrides)
    return ModelConfig(**fields)
