# SPDX-License-Identifier: MIT
"""The C-ABI library: it loads, exports every symbol include/strix_amd.h
declares, and rejects bad arguments with the reference's messages before any
HIP call (so these run without a GPU)."""

import ctypes
import re
from pathlib import Path

import pytest

from libstrix_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "strix_amd.h"


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:const\s+)?[\w]+\s*\*?\s*(strix_\w+)\s*\(", text, flags=re.M))


def test_library_loads_and_reports_abi():
    lib = _lib.load()
    assert lib.strix_abi_version() == 1


def test_every_declared_symbol_is_exported_and_bound():
    names = declared_functions()
    assert len(names) >= 15
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for n in sorted(names):
        assert hasattr(lib, n), f"{n} declared in strix_amd.h but not exported"
    assert names == set(_lib.SIGNATURES), "ctypes signatures drift from the header"


@pytest.mark.parametrize(
    "fn,args,msg",
    [
        ("strix_fp8_w8a8_block_gemm", (0, 96, 0, 1, 0, 96, 0, 1, 0, 96, 0, 4, 96, 96, -1, 0), "K must be a multiple of 128"),
        ("strix_fp8_w8a8_block_gemm", (0, 128, 0, 1, 0, 128, 0, 1, 0, 128, 7, 4, 128, 128, -1, 0), "output must be"),
        ("strix_w8a8_int8_gemm", (0, 64, 0, 0, 64, 0, 0, 64, 0, 4, 64, 64, -1, 0), "K must be a multiple of 128"),
        ("strix_int8_quant_per_token", (0, 5, 64, 0, 64, 0, 1, 64, 0), "float16 or bfloat16"),
        ("strix_fp8_quant_group128", (0, 0, 100, 0, 100, 0, 1, 1, 100, 0), "K must be a multiple of 8"),
        ("strix_moe_route_topk", (0, 2, 4096, 1, 4096, 8, 1, 0, 0, 8, 0), "1 <= E <= 1024"),
        ("strix_moe_align", (0, 16, 4, 16, 0, 10, 0, 10, 0, 0, 0, 0), "sorted_ids needs"),
        ("strix_moe_sum", (0, 0, 100, 1, 8, 100, 0, 0, 100, 0), "multiples of 8"),
        ("strix_probe_mfma", (1, 0, 0, 0, 100, 0), "multiple of 128"),
        # Operands whose rows span more than 4 GiB overflow the kernels' 32-bit row offsets.
        ("strix_fp8_w8a8_block_gemm", (0, 5120, 0, 40, 0, 5120, 0, 40, 0, 128, 0, 900000, 128, 5120, -1, 0),
         "more than 4 GiB"),
        ("strix_w8a8_int8_gemm", (0, 5120, 0, 0, 5120, 0, 0, 128, 0, 900000, 128, 5120, -1, 0),
         "more than 4 GiB"),
        ("strix_w16_gemm", (1, 0, 2560, 0, 3, 160, 1, 32, 1, 0, 0, 5120, 0, 0, 0, 128, 0, 450000, 128, 5120, -1,
                            0), "more than 4 GiB"),
    ],
)
def test_argument_errors_without_gpu(fn, args, msg):
    with pytest.raises(RuntimeError, match=msg):
        _lib.call(fn, *args)


def test_align_capacity_queries():
    assert _lib.query("strix_moe_align_sorted_capacity", 32768, 128, 128) == 32768 + 128 * 127
    assert _lib.query("strix_moe_align_workspace_bytes", 32768, 128) == 128 * 128 * 4
