"""Shared fixtures.  `gpu`-marked tests run on an MI355X and call libmq4.so
through its C ABI; the rest run on the CPU (oracle, host logic, ABI surface)."""
import importlib.util
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _load(name, path):
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def O():
    """The CPU oracle (test infrastructure)."""
    return _load("mq4_oracle", os.path.join(ROOT, "oracle", "oracle.py"))


@pytest.fixture(scope="session")
def mq4():
    import __graft_entry__
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def dev():
    import torch
    assert torch.cuda.is_available(), "gpu tests need a GPU"
    return torch.device("cuda:0")


def to_host_u16(t):
    """bf16 device tensor -> numpy uint16 bit patterns."""
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def to_dev_bf16(a, dev):
    import torch
    a = np.ascontiguousarray(a, dtype=np.uint16)
    return torch.from_numpy(a.view(np.int16)).to(dev).view(torch.bfloat16)
