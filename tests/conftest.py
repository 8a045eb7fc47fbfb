"""Shared pytest setup: markers, import paths, device detection."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "enginesmith-qwen35-08b-long-decode-m5max-round005_amd")
for p in (PKG, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: long-running case")


_gpu = None


def gpu_available() -> bool:
    global _gpu
    if _gpu is None:
        import esdecode
        _gpu = esdecode.device_count() > 0
    return _gpu


def pytest_runtest_setup(item):
    if item.get_closest_marker("gpu") is not None and not gpu_available():
        pytest.skip("no GPU visible to the HIP runtime")
