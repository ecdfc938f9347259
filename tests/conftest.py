"""Shared test set-up.

`-m "not gpu"` runs the CPU suite: the oracle against the reference's golden
vectors and independent witnesses, host-side validation, and the C ABI's
exports.  `-m gpu` runs the parity tests proper, through the C ABI, on a GPU.
"""
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "uor-matmul_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import uor_gfx950
    uor_gfx950.lib()
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def uor():
    import torch  # noqa: F401  (binds the library to torch's HIP runtime)
    import uor_gfx950
    return uor_gfx950
