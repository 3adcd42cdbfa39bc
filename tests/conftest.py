"""Shared pytest setup: the `gpu` marker, the package loader and the oracle fixtures."""
import importlib.util
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")


def load_package():
    """Loads quanta.cpp_amd/ (not an importable identifier) as module `quanta_cpp_amd`."""
    if "quanta_cpp_amd" in sys.modules:
        return sys.modules["quanta_cpp_amd"]
    pkg_dir = os.path.join(ROOT, "quanta.cpp_amd")
    spec = importlib.util.spec_from_file_location("quanta_cpp_amd", os.path.join(pkg_dir, "__init__.py"),
                                                  submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["quanta_cpp_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def load_synth():
    load_package()
    import quanta_cpp_amd.synth as synth  # noqa: E402
    return synth


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def qh():
    return load_package()


@pytest.fixture(scope="session")
def synth():
    return load_synth()


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    if o.oracle is None:
        pytest.fail("oracle/liboracle.so is not built (make -C oracle)")
    return o.oracle


@pytest.fixture(scope="session")
def gpu(qh):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    qh.init(0)
    return torch.device("cuda:0")


def bits(a: np.ndarray) -> np.ndarray:
    """Bit patterns of a float32 array, for exact comparisons (NaN-safe)."""
    return np.ascontiguousarray(a, np.float32).view(np.uint32)
