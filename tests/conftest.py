"""Shared test setup: import paths, the `gpu` marker and device gating."""

from __future__ import annotations

import os
import sys
import warnings

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(REPO, "llm-serving-runtime_amd")
for p in (REPO, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


class ParityReport(UserWarning):
    """Figures a passing parity test reports (token flips, margins, errors). Emitted as a
    warning so that pytest's warnings summary carries them in a ``-q`` run's log."""


def report(msg: str) -> None:
    print(msg, flush=True)
    warnings.warn(msg, ParityReport, stacklevel=2)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X, gfx950) and the built libmxdecode.so")


def _gpu_ready() -> tuple[bool, str]:
    """GPU tests are skipped only when no device is visible. With a device, a
    missing or broken libmxdecode.so makes them fail (no silent fallback)."""
    import torch

    if not torch.cuda.is_available():
        return False, "no ROCm device visible"
    return True, ""


def pytest_collection_modifyitems(config, items):
    gpu_items = [it for it in items if "gpu" in it.keywords]
    if not gpu_items:
        return
    ok, why = _gpu_ready()
    if ok:
        return
    skip = pytest.mark.skip(reason=why)
    for it in gpu_items:
        it.add_marker(skip)
