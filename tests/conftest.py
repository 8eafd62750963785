"""Shared test setup: import paths for the drop-in modules and the oracle, and the `gpu` marker.

Tests marked `gpu` need an MI355X (run with `-m gpu`); everything else runs on the CPU.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "ming-voice_amd")
for p in (PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (MI355X / gfx950) and the built HIP library")


import pytest  # noqa: E402


@pytest.fixture(autouse=True)
def _prefill_on_the_row_layout(monkeypatch):
    """Prefill calls read the expert stacks themselves unless a test passes copies or turns the registry on: the row
    layout stays covered, and tests of the copy registry set fused_moe.PREFILL_COPIES themselves."""
    import fused_moe
    monkeypatch.setattr(fused_moe, "PREFILL_COPIES", "off")
    yield
    fused_moe.release_prefill_copies()
