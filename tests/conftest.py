import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")
    config.addinivalue_line("markers", "slow: long CPU-only check (set LLAMD_SLOW=1)")
    # Build what is missing (the driver builds beforehand; this only covers a
    # fresh checkout). Never rebuilds an existing library.
    if not (ROOT / "oracle" / "libllamd_oracle.so").exists():
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
    if not (ROOT / "llamd_rs_amd" / "libllamd_hip.so").exists():
        subprocess.run([sys.executable, str(ROOT / "llamd_rs_amd" / "build.py")], check=True)


@pytest.fixture(scope="session")
def gpu():
    """Skip loudly when there is no device, like the reference's skip()."""
    from llamd_rs_amd import rocm
    if not rocm.available():
        if os.path.exists("/dev/kfd"):
            pytest.fail("a ROCm driver is present but no device is visible to libllamd_hip.so")
        pytest.skip("no ROCm device in this container")
    return rocm
