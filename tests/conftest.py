# SPDX-License-Identifier: MIT
"""Markers and shared helpers.

`gpu` tests need an MI355X (gfx950); they are deselected on the CPU-only
container (`-m "not gpu"`) and skipped if collected without a GPU. On a GPU
box a missing or unbuilt library fails them loudly: libstrix_amd has no
fallback path.
"""

import os
import sys

import pytest
import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X)")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def peak_rel_err(out: torch.Tensor, ref: torch.Tensor) -> float:
    """max |out - ref| / max |ref|: the "max relative error" of the accuracy
    bar (the reference's tests compare against atol = tol * peak, e.g.
    tests/test_fp8.py:77-78)."""
    out = out.detach().float().cpu()
    ref = ref.detach().float().cpu()
    peak = ref.abs().max().item()
    return (out - ref).abs().max().item() / (peak if peak > 0 else 1.0)
