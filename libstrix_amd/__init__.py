# SPDX-License-Identifier: MIT
"""gfx950 (MI355X) quantized-GEMM kernels, exposed as torch.ops.strix.*.

The MI355X counterpart of the reference's `strix` package
(python/strix/__init__.py): importing it registers the torch.ops.strix.*
schemas (libstrix_amd.ops) over the C-ABI library libstrix_amd/_strix_amd.so
and exports the kernel-table query API. `is_supported_device()` is the gfx950
gate (the reference gates on gfx1151, python/strix/__init__.py:510-513).
"""

from __future__ import annotations

import torch

from libstrix_amd import torch_ops as _torch_ops  # noqa: F401  (registers torch.ops.strix.*)
from libstrix_amd._lib import available as library_available
from libstrix_amd.registry import Range, explain, geometries, kernels, ops, select, selections


def is_supported_device() -> bool:
    if not torch.cuda.is_available() or torch.version.hip is None:
        return False
    return torch.cuda.get_device_properties(0).gcnArchName.split(":")[0] == "gfx950"


__all__ = [
    "Range",
    "explain",
    "geometries",
    "is_supported_device",
    "kernels",
    "library_available",
    "ops",
    "select",
    "selections",
]
