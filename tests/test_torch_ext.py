# SPDX-License-Identifier: MIT
"""The C++ registration of the hot-path ops (libstrix_amd/_strix_torch.so):
it is built, it loaded, its schemas are the strings the Python layer records
(the reference's schemas byte for byte where the op is the reference's), and
its argument checks raise the same errors without a GPU."""

import pytest
import torch

import libstrix_amd  # noqa: F401
from libstrix_amd import torch_ops as T

HOT = {"int8_quant_per_token", "fp8_quant_group128", "w8a8_scaled_mm", "fp8_w8a8_block_gemm",
       "fp8_w8a8_block_gemm_kmajor", "weight8_kmajor", "moe_route_topk", "moe_align", "moe_align_quant",
       "moe_route_align", "moe_route_align_quant", "moe_sum", "moe_weighted_sum", "moe_gemm_fp8_w8a8",
       "moe_gemm_mxfp4", "moe_gemm_w4a16_zp"}


def test_extension_built_and_loaded():
    assert T.TORCH_EXT.exists(), "python libstrix_amd/build.py builds _strix_torch.so"
    assert HOT <= T.NATIVE_OPS


def test_every_schema_matches_its_registration():
    for name, text in T.SCHEMAS.items():
        registered = str(getattr(torch.ops.strix, name).default._schema)
        assert registered == str(torch._C.parse_schema("strix::" + text)), name


def test_native_ops_have_fake_kernels():
    x = torch.empty(4, 256, dtype=torch.bfloat16, device="meta")
    q, s = torch.ops.strix.fp8_quant_group128(x)
    assert q.shape == (4, 256) and q.dtype == torch.float8_e4m3fn and s.shape == (4, 2)
    ids, w, si, ei, npp = torch.ops.strix.moe_route_align(torch.empty(3, 16, device="meta"), 2, 16)
    assert ids.shape == (3, 2) and si.numel() == 6 + 16 * 15


def test_native_checks_raise_before_launch():
    # A CUDA-key impl is reached only for device tensors; the checks of the
    # ctypes rendering (the same messages) are exercised on the CPU instead.
    with pytest.raises(RuntimeError, match="must be 2-D and contiguous"):
        T.fp8_quant_group128(torch.zeros(4, dtype=torch.bfloat16))
