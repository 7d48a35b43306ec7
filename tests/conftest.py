"""Shared fixtures. GPU tests are marked `gpu`; everything else runs on the CPU.

The oracle (oracle/) is test infrastructure: only the checker side of a test
touches it. The product libraries are loaded from mynah-asr_amd/lib.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "mynah-asr_amd"))

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    import oracle
    if not os.path.exists(oracle.LIB_PATH):
        oracle.build(ref=False)
    return oracle.Oracle()


@pytest.fixture(scope="session")
def ingot_ref():
    import oracle
    if not oracle.IngotRef.available():
        pytest.skip("oracle/_ref not built (needs the reference tree at build time)")
    return oracle.IngotRef()


@pytest.fixture(scope="session")
def lib():
    import mynah_hip
    return mynah_hip.HipLib()


@pytest.fixture(scope="session")
def gpu(lib):
    """The HIP library on a machine that must have the GPU: fail, never skip."""
    if not lib.available():
        raise RuntimeError("gpu-marked test on a machine without a usable gfx950 device: "
                           + lib.last_error())
    return lib
