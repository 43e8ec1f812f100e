"""Shared test setup.

- puts the repository root (for ``oracle``) and the package directory
  ``hawkpoint-npu-llm_amd`` (for ``runtime``, as the reference's tests put
  ``npu_llm`` on the path) on ``sys.path``;
- registers the ``gpu`` marker: GPU tests run with ``-m gpu`` on an MI355X and
  call the product through libhk.so's C ABI;
- never imports torch: the product has its own HIP runtime binding, and a
  second HIP runtime in the process would be a hazard.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "hawkpoint-npu-llm_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libhk.so")


@pytest.fixture(scope="session")
def hk_lib():
    from runtime import hip

    hip.init(0)
    return hip.lib()


def announce(message):
    """Print and flush a line that names the GPU case about to run."""
    print(message, flush=True)
    sys.stderr.write(message + "\n")
    sys.stderr.flush()
