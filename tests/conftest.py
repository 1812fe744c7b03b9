"""pytest configuration: the `gpu` marker and import paths.

`-m gpu` tests run the HIP path on a real GPU and compare it with the CPU
oracle; everything else runs on the CPU.
"""

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "breeze-tts-2_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libbzgemv.so")


def pytest_collection_modifyitems(config, items):
    import pytest
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
