"""Shared test setup.

* registers the ``gpu`` marker (tests that need an MI355X);
* loads the product package from the ``vlx-tee_amd`` directory as ``vlx_tee_amd``;
* exposes the CPU oracle (oracle/oracle.py) that GPU results are compared with.
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X)")


def load_package():
    name = "vlx_tee_amd"
    if name in sys.modules:
        return sys.modules[name]
    root = REPO / "vlx-tee_amd"
    spec = importlib.util.spec_from_file_location(name, root / "__init__.py",
                                                  submodule_search_locations=[str(root)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def pkg():
    return load_package()


@pytest.fixture(scope="session")
def O():
    from oracle import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def ref(O):
    m = O.ref_module()
    if m is None:
        pytest.skip("compiled reference (oracle/_ref) not available")
    return m


@pytest.fixture(scope="session")
def hip(pkg):
    """The HIP drop-in module; GPU tests fail loudly if it cannot load."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    import vlx_tee_amd.native_hip_codec as H

    H.N.lib()
    return H
