import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the C-ABI library")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as o
    o.build()
    return o


def load_mi355():
    """Load the sam3.cpp_amd package (directory name is not an identifier)."""
    import importlib.util
    name = "sam3_cpp_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(ROOT, "sam3.cpp_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def mi():
    return load_mi355()


@pytest.fixture(scope="session")
def ctx(mi):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    c = mi.Context(0)
    yield c
    c.close()
