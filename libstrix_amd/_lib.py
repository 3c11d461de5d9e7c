# SPDX-License-Identifier: MIT
"""ctypes binding of the C ABI in include/strix_amd.h (libstrix_amd/_strix_amd.so).

Every entry point returns a status code; `call` turns a non-zero status into
a RuntimeError carrying the library's message, the way the reference's
TORCH_CHECK surfaces as RuntimeError (csrc/gemm/mxfp4_wmma_gemm.hip:291-295).
There is no fallback: when the library is missing, any op call raises.
"""

from __future__ import annotations

import ctypes
from ctypes import c_char_p, c_int, c_int64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).with_name("_strix_amd.so")

# dtype codes (STRIX_BF16 ... in include/strix_amd.h)
BF16, F16, F32, I32 = 0, 1, 2, 3
ACT_SILU, ACT_GELU_TANH = 0, 1

P = c_void_p
I = c_int
L = c_int64

# Trailing arguments shared by the 16-bit MoE GEMMs (STRIX_MOE16_PARAMS).
MOE16 = [P, L, I, P, L, I, P, L, P, L, P, P, L, L, L, I, I, L, L, P]

# scale dtype codes of the 16-bit GEMMs
S_F32, S_BF16, S_F16, S_E8M0 = 0, 1, 2, 3
# weight format codes of strix_w16_gemm / strix_dequant_bf16
FMT_MXFP4, FMT_INT4_SYM, FMT_FP8, FMT_INT8, FMT_INT4_EX, FMT_U8B128 = 1, 3, 4, 5, 6, 7

# name -> argument types (all return int unless listed in _RESTYPE)
SIGNATURES: dict[str, list] = {
    "strix_abi_version": [],
    "strix_last_error": [],
    "strix_int8_quant_per_token": [P, I, L, P, L, P, L, L, P],
    "strix_int8_quant_group128": [P, I, L, P, L, P, L, L, L, P],
    "strix_fp8_quant_group128": [P, I, L, P, L, P, L, L, L, P],
    "strix_int8_dequant_group128": [P, L, P, L, P, I, L, L, L, P],
    "strix_w16_gemm": [I, P, L, P, I, L, L, L, L, P, I, L, P, L, P, L, I, L, L, L, I, P],
    "strix_fp8_w8a8_block_gemm": [P, L, P, L, P, L, P, L, P, L, I, L, L, L, I, P],
    "strix_weight8_kmajor": [P, L, L, L, L, P, P],
    "strix_fp8_w8a8_block_gemm_kmajor": [P, L, P, L, P, P, L, P, L, I, L, L, L, I, P],
    "strix_w8a8_int8_gemm": [P, L, P, P, L, P, P, L, I, L, L, L, I, P],
    "strix_w8a8_int8_group_gemm": [P, L, P, L, P, L, I, P, L, L, P, L, I, L, L, L, I, P],
    "strix_w4a8_gemm": [P, L, P, L, P, L, I, P, L, L, P, L, I, L, L, L, P],
    "strix_moe_gemm_w4a8": [P, L, I, P, L, P, L, P, L, L, P, L, L, P, L, P, L, P, P, L, L, L, I, I, L, L, P],
    "strix_moe_gemm_fp8_w8a8": [P, L, I, P, L, P, L, P, L, L, P, L, L, P, L, P, L, P, P, L, L, L, I, I, L, L, P],
    "strix_moe_gemm_fp8_w8a8_kmajor": [P, L, I, P, L, P, L, P, P, L, L, P, L, P, L, P, P, L, L, L, I, I, L, L, P],
    "strix_moe_gemm_mxfp4": [P, L, L, P, L, L] + MOE16,
    "strix_moe_gemm_w4a16_zp": [P, L, L, P, I, L, L, P, L, L, L] + MOE16,
    "strix_moe_gemm_w4a16": [P, L, L, P, I, L, L, L] + MOE16,
    "strix_moe_gemm_bf16": [P, L, L] + MOE16,
    "strix_moe_gemm_fp8_w8a16": [P, L, L, P, I, L, L, L, I] + MOE16,
    "strix_moe_gemm_w8a16": [P, L, L, P, I, L, L] + MOE16,
    "strix_mxfp4_gemm": [P, L, P, L, P, I, L, P, L, P, L, I, L, L, L, I, P],
    "strix_fp8_w8a16_gemm": [P, L, P, L, I, P, I, L, P, L, I, L, L, L, I, P],
    "strix_dequant_bf16": [I, P, L, P, I, L, L, L, P, L, L, L, P],
    "strix_moe_route_topk": [P, I, L, L, L, L, I, P, P, L, P],
    "strix_moe_align_sorted_capacity": [L, L, L],
    "strix_moe_align_workspace_bytes": [L, L],
    "strix_moe_align": [P, L, L, L, P, L, P, L, P, P, L, P],
    "strix_moe_align_noalloc_max_bytes": [],
    "strix_moe_align_noalloc": [P, L, L, L, P, L, P, L, P, P],
    "strix_moe_align_quant": [P, L, L, L, P, L, P, L, P, P, L, P, I, L, P, L, P, L, L, L, P],
    "strix_moe_route_align": [P, I, L, L, L, L, I, P, P, L, P, L, P, L, P, P, L, P],
    "strix_moe_route_align_quant": [P, I, L, L, L, L, I, P, P, L, P, L, P, L, P, P, L, P, I, L, P, L, P, L, L, P],
    "strix_moe_sum": [P, I, L, L, L, L, P, P, L, P],
    "strix_probe_mfma": [I, P, P, P, L, P],
    "strix_probe_g2l": [P, P, P],
    "strix_probe_cvt": [P, L, P, P, P, P, L, P],
}
_RESTYPE = {
    "strix_last_error": c_char_p,
    "strix_moe_align_sorted_capacity": c_int64,
    "strix_moe_align_workspace_bytes": c_int64,
    "strix_moe_align_noalloc_max_bytes": c_int64,
}

_lib: ctypes.CDLL | None = None
_load_error: str | None = None


def load() -> ctypes.CDLL:
    """Loads the shared library once; raises if it is missing or incomplete."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        _load_error = (
            f"{LIB_PATH} is not built: run `python libstrix_amd/build.py` "
            "(libstrix_amd has no CPU or PyTorch fallback)"
        )
        raise RuntimeError(_load_error)
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError names a missing export
        fn.argtypes = argtypes
        fn.restype = _RESTYPE.get(name, c_int)
    _lib = lib
    return lib


def available() -> bool:
    try:
        load()
        return True
    except (RuntimeError, OSError, AttributeError):
        return False


def last_error() -> str:
    msg = load().strix_last_error()
    return msg.decode() if msg else ""


def call(name: str, *args) -> None:
    rc = getattr(load(), name)(*args)
    if rc != 0:
        raise RuntimeError(last_error() or f"{name} failed with status {rc}")


def query(name: str, *args) -> int:
    return int(getattr(load(), name)(*args))
