import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs the HIP kernels through the C ABI)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def golden_elem():
    return np.load(os.path.join(GOLDEN, "elem_quant.npz"))


@pytest.fixture(scope="session")
def golden_mxfp():
    return np.load(os.path.join(GOLDEN, "mxfp_quant.npz"))


@pytest.fixture(scope="session")
def golden_hbq():
    return np.load(os.path.join(GOLDEN, "hbq_quant.npz"))


@pytest.fixture(scope="session")
def golden_compiled():
    """use_quant_kernel=True / activate_dynamo=True fixtures: the torch.compile'd element quantizer."""
    return np.load(os.path.join(GOLDEN, "compiled_quant.npz"))


@pytest.fixture(scope="session")
def golden_extra():
    """The MXFP per-tensor scale branch and PoT HBQ on the weight and bf16 inputs."""
    return np.load(os.path.join(GOLDEN, "extra_quant.npz"))
