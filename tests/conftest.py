import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "candle-rocm-vulkan_amd")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def load_cqkv():
    """The package front end (candle-rocm-vulkan_amd/cqkv.py) as module `cqkv`."""
    if "cqkv" in sys.modules:
        return sys.modules["cqkv"]
    spec = importlib.util.spec_from_file_location("cqkv", os.path.join(PKG, "cqkv.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["cqkv"] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def cq():
    return load_cqkv()


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
