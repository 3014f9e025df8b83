import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP path through the C ABI")


def _ensure_built():
    lib = os.path.join(ROOT, "furnace_amd", "lib", "libfurnace_hip.so")
    orc = os.path.join(ROOT, "oracle", "liboracle.so")
    if not os.path.exists(lib):
        from furnace_amd import _build
        _build.build()
    if not os.path.exists(orc):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True)


_ensure_built()


@pytest.fixture(scope="session")
def hip():
    """HIP runtime access for GPU tests; skips when no device is visible."""
    import furnace_amd as fa
    h = fa.Hip()
    if h.device_count() == 0:
        pytest.skip("no HIP device visible")
    return h


@pytest.fixture(scope="session")
def tmpdir_models(tmp_path_factory):
    return str(tmp_path_factory.mktemp("models"))
