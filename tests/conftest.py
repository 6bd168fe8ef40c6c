import os
import sys

import pytest

import sys
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built qwn_hip library")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    return oracle.load()


@pytest.fixture(scope="session")
def ref_lib():
    import oracle
    ref = oracle.load_ref()
    if ref is None:
        pytest.skip("oracle/_ref (reference CPU kernels built in place) is not available")
    return ref


@pytest.fixture(scope="session")
def hip_lib():
    # torch first: its bundled HIP runtime has the same soname as the one the
    # library links, so loading torch first makes both share one runtime and
    # torch device tensors usable as the library's device buffers.
    import torch  # noqa: F401
    from qwanto_amd import abi
    return abi.load()


@pytest.fixture(scope="session")
def gpu_ctx(hip_lib):
    from qwanto_amd import abi
    if not hip_lib.devices():
        pytest.fail("no GPU visible to qwn_hip (gpu tests must run on the GPU host)")
    ctx = abi.Context(hip_lib, device=0)
    yield ctx
    ctx.close()
