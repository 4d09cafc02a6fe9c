import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "katali-lab_amd", "tests"):
    p = os.path.join(REPO, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def refcpu():
    from oracle import RefCPU, ref_available
    if not ref_available():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    return RefCPU()


@pytest.fixture(scope="session")
def hip():
    """The HIP library on a real device; GPU tests fail (not skip) when the
    library or the device is missing, so a silent fallback cannot pass."""
    from katali_hip import KataliHip
    h = KataliHip()
    assert h.probe(), f"no usable gfx950 device: {h.status()}"
    print(f"[katali_hip] {h.status()}", flush=True)
    return h


@pytest.fixture
def two_launch_layer(monkeypatch):
    """The single-token layer as kernels A and B (KATALI_HIP_XCD=0): for tests
    whose other path (batched, normed, allocation-free) must match those two
    kernels bit for bit. The XCD-sliced layer that eight-slot shapes take by
    default sums each down row over its own lane split and is tested against
    kernels A and B and the oracle on its own."""
    monkeypatch.setenv("KATALI_HIP_XCD", "0")
