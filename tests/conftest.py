"""Shared pytest configuration.

Tests marked ``gpu`` need an MI355X (gfx950) and the built libraries; the rest
run on the CPU (oracle vs golden fixtures, host logic, C-ABI exports).
"""
import os
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (REPO, os.path.join(REPO, "pytorch-vulkan_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built gfx950 libraries")
