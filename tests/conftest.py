"""pytest configuration: the `gpu` marker and import paths.

GPU tests are marked ``@pytest.mark.gpu`` and run on a real MI355X; every
other test runs on the CPU.  The package directory
(``gqa-flash-attn-rtx3060_amd/``, which holds ``gqa_kernels``) and the repo
root (for ``oracle``) are put on sys.path so the tests import the drop-in as
``from gqa_kernels import gqa_flash_attn``, like the reference's own tests.
"""
import sys
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent
PKG_DIR = REPO / "gqa-flash-attn-rtx3060_amd"
for p in (str(PKG_DIR), str(REPO)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")
