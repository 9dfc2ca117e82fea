import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def _ensure_built():
    need = [
        os.path.join(ROOT, "foundry_amd", "_build", "libfoundry_restore.so"),
        os.path.join(ROOT, "foundry_amd", "_build", "libfdy_synth.so"),
        os.path.join(ROOT, "oracle", "_build", "liboracle.so"),
    ]
    if not all(os.path.exists(p) for p in need):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
        subprocess.run(["make", "-s", "-j8", "-C", os.path.join(ROOT, "foundry_amd", "csrc")], check=True)


_ensure_built()


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    torch.cuda.init()
    return torch
