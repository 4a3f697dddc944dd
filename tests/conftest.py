"""Shared pytest setup: the `gpu` marker, repo paths, and a device fixture.

GPU tests call the product through the C ABI (libnmx.so / libpinfer.so) and compare with the
oracle (a scalar C restatement of the reference, oracle/). They never fall back to the CPU:
if the native library or the GPU is missing, they fail.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libnmx.so)")


@pytest.fixture(scope="session")
def dev():
    from nibblemac_amd.nmx import Device

    d = Device(0)
    print(f"[gpu] {d.name}", flush=True)
    yield d
    d.close()
