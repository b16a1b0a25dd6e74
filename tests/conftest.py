import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "synthesize.cpp_amd")
ORACLE = os.path.join(ROOT, "oracle")
GOLDEN = os.path.join(ROOT, "tests", "golden")

for p in (ROOT, PKG, ORACLE):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


def _ensure_oracle():
    so = os.path.join(ORACLE, "libggml_cpu_ref.so")
    if not os.path.exists(so):
        subprocess.run(["make", "-C", ORACLE], check=True, stdout=subprocess.DEVNULL)


_ensure_oracle()


@pytest.fixture(scope="session")
def gpu():
    """The HIP binding with torch's device plumbing; skips nothing: a GPU test
    run without a GPU or without the built library fails loudly."""
    import torch  # noqa: F401  (loads the HIP runtime the library shares)
    import synth_hip

    if not torch.cuda.is_available():
        pytest.fail("gpu-marked test run without a visible GPU")
    synth_hip.load()
    return synth_hip
