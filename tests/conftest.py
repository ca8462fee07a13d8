"""pytest configuration: import paths, the `gpu` marker, and the built library.

`-m gpu` tests need a HIP device (an MI355X); everything else runs on CPU.
The C-ABI library and the torch extension are built in-tree once per session
when they are missing (the GPU box receives them prebuilt).
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(ROOT, "cuda-pa-int8_amd")
for p in (ROOT, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X, gfx950)")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP device in this process")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def built():
    """Paths of the built library and extension (built here if absent)."""
    from pa_int8 import _build

    lib = os.path.join(_build.LIB_DIR, _build.LIB_NAME)
    ext = os.path.join(_build.LIB_DIR, _build.EXT_NAME)
    if not (os.path.exists(lib) and os.path.exists(ext)):
        _build.build()
    return lib, ext
