import importlib
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def load_pkg():
    """The product package lives in the directory ``rwkv-rs_amd``; its name is
    not a Python identifier, so it is imported by string. RWKV_AMD_TEST_LIB
    points the tests at another build of the library (the sanitizer build of
    ``rwkv-rs_amd/build.py --sanitize``)."""
    pkg = importlib.import_module("rwkv-rs_amd")
    other = os.environ.get("RWKV_AMD_TEST_LIB")
    if other:
        native = importlib.import_module("rwkv-rs_amd._native")
        native.LIB_PATH = other
    return pkg


@pytest.fixture(scope="session")
def pkg():
    return load_pkg()


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.build()
    return o


def rel_l2(got, want):
    import numpy as np
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    den = np.linalg.norm(want.ravel())
    num = np.linalg.norm((got - want).ravel())
    if den == 0.0:
        return float(num)
    return float(num / den)


NAMES = ("w", "r", "k", "v", "a", "b")
GRAD_NAMES = ("weight_decay_grad", "receptance_grad", "key_grad", "value_grad",
              "removal_grad", "replacement_grad")


def announce(*parts):
    """Name the case before a GPU step, so that a crash still identifies it."""
    print("[gpu-case]", *parts, flush=True)


def to_dev(x, dtype=None):
    import numpy as np
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()
    return t.to(dtype) if dtype is not None else t


def to_np(t):
    return t.detach().float().cpu().numpy()
