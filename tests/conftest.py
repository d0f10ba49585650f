# SPDX-License-Identifier: Unlicense
import importlib.util
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "i.coregistration.opencl_amd"
sys.path.insert(0, str(Path(__file__).resolve().parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


def load_package():
    """The binding module (the package directory name has dots)."""
    if "icoreg_amd" in sys.modules:
        return sys.modules["icoreg_amd"]
    spec = importlib.util.spec_from_file_location(
        "icoreg_amd", PKG_DIR / "__init__.py", submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["icoreg_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def ic():
    return load_package()


@pytest.fixture(scope="session")
def dev(ic):
    d = ic.Device("auto")
    print(f"\n[device] {d.name} {d.arch} CUs={d.ocl.cu_count}", flush=True)
    yield d
    d.close()


@pytest.fixture(scope="session")
def orc():
    from oracle_lib import oracle
    return oracle()
