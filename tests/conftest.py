import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "spectral-deflation_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI)")


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    return {
        "inputs": np.load(os.path.join(GOLDEN, "inputs.npz")),
        "eager": np.load(os.path.join(GOLDEN, "ref_eager.npz")),
        "compiled": np.load(os.path.join(GOLDEN, "ref_compiled.npz")),
    }


def bf16_from_bits(a):
    import numpy as np
    import torch
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def bits_of(t):
    import numpy as np
    import torch
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
