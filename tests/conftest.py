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


@pytest.fixture(scope="session")
def agree_model(tmp_path_factory):
    """(path, prompt): a small synthetic model (the 0.8B layer pattern) whose MTP drafts are
    often accepted, and a 24-token prompt. Generating 64 tokens at k = 4 from that prompt, the
    reference engine accepts 46 of 66 drafts, so rounds with every draft accepted and rounds
    with a rejection both occur: multi-token commits of the KV rows and deferred DeltaNet
    replays (pend / keep) of 1..k rows."""
    import numpy as np

    from nibblemac_amd import pqfile

    w = pqfile.agreeing_norm(pqfile.SMALL.hidden)
    d = tmp_path_factory.mktemp("agree")
    path = pqfile.write_model(d / "agree.pq", pqfile.SMALL, seed=3, random_norms=True,
                              overrides={"norm.weight": w, "mtp.norm.weight": w})
    return path, np.random.default_rng(2).integers(0, 2047, 24)
