"""Shared pytest setup: the ``gpu`` marker and import paths.

GPU tests carry ``@pytest.mark.gpu`` and run only on a machine with a ROCm GPU
(``pytest -m gpu``); everything else runs on the CPU (``pytest -m "not gpu"``).
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_PARENT = os.path.join(ROOT, "01-glm53-ascend_amd")
for p in (ROOT, PKG_PARENT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X / gfx950)")


def pytest_collection_modifyitems(config, items):
    # A GPU test selected on a machine without a GPU should fail loudly, not
    # skip: the round-end run happens on a GPU box and a skip would hide a
    # missing device. Only mark the reason here.
    for item in items:
        if "gpu" in item.keywords:
            item.user_properties.append(("needs", "gpu"))


@pytest.fixture(scope="session")
def gpu_ops():
    """The native op library, loaded; fails (never skips) if it is missing."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    import sgl_glm53_ascend_ops  # noqa: F401  loads the native libraries

    return torch.ops.sgl_glm53_ascend
