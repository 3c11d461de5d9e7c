# SPDX-License-Identifier: MIT
"""CPU oracle for the quantized-GEMM hot path. TEST INFRASTRUCTURE ONLY.

A CPU restatement (torch on the CPU, numpy for exact integer work) of the
reference's own PyTorch references: quantize or decode the long way, then an
fp32 matmul, per-expert loops for MoE. Each function cites the reference
file:line it follows.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or the timed CPU baseline),
never as the thing measured or shipped: the libstrix_amd product path has no
CPU fallback and never imports it.

Parity pinning: every function here is checked by tests/test_oracle_*.py
against known answers, first-principles restatements, brute force on tiny
inputs, or invariants chosen so that a plausible mistake fails; see the
"pinned by" line of each docstring.
"""

from oracle.quant import (  # noqa: F401
    e4m3_decode,
    u8b128_decode,
    wna16_ex_decode,
    wna16_ex_pack,
    wna16_ex_unpack,
    fp8_quant_group128,
    int8_quant_group128,
    int8_quant_per_token,
    mxfp4_decode,
    wna16_sym_decode,
    wna16_zp_decode,
)
from oracle.gemm import (  # noqa: F401
    fp8_block_dequant,
    fp8_block_gemm,
    w8a8_int8_acc,
    w8a8_int8_gemm,
    w8a8_int8_group_gemm,
)
from oracle.moe import (  # noqa: F401
    align,
    fused_moe,
    moe_expert_gemm,
    moe_sum,
    route_topk,
)
