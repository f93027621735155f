"""Test configuration: the `gpu` marker and the repository root on sys.path.

Tests marked `gpu` need an AMD Instinct GPU and call the HIP path through the C ABI (libveckern.so). Everything
else runs on the CPU: the oracle against golden vectors and the reference's own compiled CPU code, host-side
planning logic, and that the C-ABI library loads and exports every declared symbol.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU; exercises the HIP path through the C ABI")
