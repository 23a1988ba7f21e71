"""Shared test setup.

* ``gpu`` marks tests that need a GPU (run on the MI355X box with
  ``pytest -m gpu``); everything else runs on the CPU.
* The package directory ``tensorplay-mlu_amd`` is imported under that name
  with importlib; the oracle (test infrastructure) as ``oracle.binding``.
"""

import importlib
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture(scope="session")
def amd():
    """The device backend package, loaded (raises if the library is not built)."""
    pkg = importlib.import_module("tensorplay-mlu_amd")
    pkg.load()
    return pkg


@pytest.fixture(scope="session")
def ops(amd):
    return importlib.import_module("tensorplay-mlu_amd.ops")


@pytest.fixture(scope="session")
def dev(amd):
    """DeviceTensor class; also checks a GPU is there (GPU tests only)."""
    tensor = importlib.import_module("tensorplay-mlu_amd.tensor")
    runtime = importlib.import_module("tensorplay-mlu_amd.runtime")
    assert runtime.is_available(), "no GPU visible to the HIP runtime"
    return tensor.DeviceTensor


@pytest.fixture(scope="session")
def orc():
    from oracle import binding

    binding.lib()
    return binding


def rng(seed=0):
    return np.random.default_rng(seed)
