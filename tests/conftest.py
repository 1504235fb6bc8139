import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(REPO, "microscaling-quant_amd")
for p in (PKG_ROOT, REPO):
    if p not in sys.path:
        sys.path.insert(0, p)

HOST_DIR = os.path.join(REPO, "tests", "host")
HOST_LIB = os.path.join(HOST_DIR, "_build", "libmxq_numerics_host.so")


def build_host_lib() -> str:
    """g++ build of the kernels' numerics header for host-side tests (seconds)."""
    os.makedirs(os.path.dirname(HOST_LIB), exist_ok=True)
    src = os.path.join(HOST_DIR, "numerics_host.cpp")
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
           "-I", os.path.join(PKG_ROOT, "csrc"), "-I", os.path.join(REPO, "include"), src, "-o", HOST_LIB]
    subprocess.run(cmd, check=True)
    return HOST_LIB


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (gfx950) and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running")


@pytest.fixture(scope="session")
def host_lib():
    import ctypes
    deps = [os.path.join(HOST_DIR, "numerics_host.cpp"), os.path.join(PKG_ROOT, "csrc", "mxq_numerics.h")]
    if not os.path.exists(HOST_LIB) or any(os.path.getmtime(d) > os.path.getmtime(HOST_LIB) for d in deps):
        build_host_lib()
    return ctypes.CDLL(HOST_LIB)


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("a gpu-marked test ran where no GPU is visible")
    return torch.device("cuda", 0)
