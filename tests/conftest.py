import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "vllm-gr-ehaleva_amd")
for p in (ROOT, PKG_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and the built library")


def _lib_path():
    return os.path.join(PKG_DIR, "vllm_gr_amd", "_lib", "libgr_beam.so")


@pytest.fixture(scope="session")
def built_lib():
    """The HIP library; built here when missing (tests never fall back)."""
    if not os.path.exists(_lib_path()):
        import importlib.util
        spec = importlib.util.spec_from_file_location("gr_build", os.path.join(PKG_DIR, "build.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    from vllm_gr_amd import _C
    return _C.lib()


@pytest.fixture(scope="session")
def device(built_lib):
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a HIP device")
    return torch.device("cuda:0")
