import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

# the package directory name is not an identifier: load it as kt_prefill_lend_amd
import importlib.util  # noqa: E402

_spec = importlib.util.spec_from_file_location(
    "kt_prefill_lend_amd", ROOT / "kt-prefill-lend_amd" / "__init__.py",
    submodule_search_locations=[str(ROOT / "kt-prefill-lend_amd")])
if "kt_prefill_lend_amd" not in sys.modules:
    _mod = importlib.util.module_from_spec(_spec)
    sys.modules["kt_prefill_lend_amd"] = _mod
    _spec.loader.exec_module(_mod)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda", 0)


def to_dev(a: np.ndarray, dev, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.to(dev)


def bf16_tensor(bits: np.ndarray, dev):
    import torch

    return to_dev(bits.astype(np.uint16).view(np.int16), dev).view(torch.bfloat16)


def bf16_bits_of(t) -> np.ndarray:
    import torch

    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
