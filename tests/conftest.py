import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library's kernels)")


def pytest_collection_modifyitems(config: pytest.Config, items: list[pytest.Item]) -> None:
    """GPU tests need a visible GPU: skip them (with the reason) where the built library sees none, unless
    ARTLITE_REQUIRE_GPU is set. A missing library is no reason to skip: the GPU tests then fail loudly."""
    if os.environ.get("ARTLITE_REQUIRE_GPU"):
        return
    from artlite_amd import _hip

    if not _hip.LIB_PATH.exists() or _hip.device_count() > 0:
        return
    skip = pytest.mark.skip(reason="no GPU visible (or libartlite_moe.so not built)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
