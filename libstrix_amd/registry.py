# SPDX-License-Identifier: MIT
"""Kernel table: each gfx950 entry point, the op it implements and its geometry.

Same query API and semantics as the reference's table
(python/strix/registry.py:65-964): `select(op, **geometry)` returns the first
row of `op` whose constraints all hold, or None (the caller keeps its own
path); `explain` gives every row's verdict with a reason; `geometries` lists
shape points; `selections` records every query; `kernels` and `ops` list the
table. Constraint forms: a scalar is one required value, a tuple the allowed
set, `Range` a bound. The rows are re-derived for gfx950 tiles.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

import torch

_DTYPE_NAMES = {
    torch.bfloat16: "bf16",
    torch.float16: "fp16",
    torch.float32: "fp32",
    torch.float8_e4m3fn: "fp8_e4m3",
    torch.int8: "int8",
    torch.uint8: "uint8",
    torch.int32: "int32",
}
_POINT_TYPES = (int, bool, str)


def _norm(v: Any) -> Any:
    """Canonical form of a geometry value: torch dtypes (or 'torch.x' strings) by short name."""
    if isinstance(v, torch.dtype):
        return _DTYPE_NAMES.get(v, str(v))
    if isinstance(v, str) and v.startswith("torch."):
        dt = getattr(torch, v[len("torch."):], None)
        return _DTYPE_NAMES.get(dt, v) if isinstance(dt, torch.dtype) else v
    return v


@dataclass(frozen=True)
class Range:
    """Inclusive integer bound: Range(lo=6) is 6 or more, Range(hi=5) at most 5."""

    lo: int | None = None
    hi: int | None = None

    def covers(self, got: Any) -> bool:
        if isinstance(got, bool) or not isinstance(got, int):
            return False
        return (self.lo is None or got >= self.lo) and (self.hi is None or got <= self.hi)

    def __str__(self) -> str:
        if self.lo is not None and self.hi is not None:
            return f"in {self.lo}..{self.hi}"
        return f">= {self.lo}" if self.lo is not None else f"<= {self.hi}"


def _matches(want: Any, got: Any) -> bool:
    if isinstance(want, Range):
        return want.covers(got)
    if isinstance(want, tuple):
        return got in want
    return got == want


def _describe(want: Any) -> str:
    if isinstance(want, Range):
        return str(want)
    if isinstance(want, tuple):
        return f"in {want}"
    return f"== {want}"


@dataclass(frozen=True)
class Kernel:
    name: str
    op: str
    doc: str
    constraints: dict[str, Any] = field(default_factory=dict)
    spec: dict[str, Any] = field(default_factory=dict)

    def check(self, geometry: dict[str, Any]) -> str | None:
        """None when `geometry` satisfies every constraint, else the first failure."""
        for key, want in self.constraints.items():
            if key not in geometry:
                return f"{key} not given"
            got = _norm(geometry[key])
            if not _matches(want, got):
                return f"{key}={got}, needs {_describe(want)}"
        return None

    def accepts(self, partial: dict[str, Any]) -> bool:
        """Whether every given key is constrained by this row and satisfied."""
        return all(k in self.constraints and _matches(self.constraints[k], _norm(v)) for k, v in partial.items())


_BF16 = {"dtype": "bf16"}
_MOE_TILES = {"block_m": (16, 32, 64, 128, 256)}

KERNELS: list[Kernel] = [
    # ------------------------------------------------------------ quantizers
    Kernel(
        "int8_quant_per_token",
        "int8_quant",
        "per-token symmetric int8: s = max|x|/127 (1 for a zero row), q = clamp(rint(x / s), -127, 127); "
        "one 256-thread block per row, two passes (the second from L2)",
        {"dtype": ("bf16", "fp16"), "granularity": "token"},
    ),
    Kernel(
        "moe_act_quant_i8",
        "moe_act_quant_i8",
        "per (row, 128-element group) int8: s = max|x|/127 (1 for an all-zero group), "
        "q = clamp(rint(x / s), -127, 127). bf16 in, int8 + fp32 scales out",
        {**_BF16, "out_dtype": "int8", "group_size": (128,)},
        {"threads": 256, "lanes_per_group": 16},
    ),
    Kernel(
        "fp8_quant_group128",
        "fp8_quant",
        "per (row, 128-element group) e4m3fn: s = max|x|/448 (1 for an all-zero group), q = e4m3_rne(x / s)",
        {"dtype": ("bf16", "fp16"), "group_size": 128},
        {"lanes_per_group": 8},
    ),
    # ------------------------------------------------------------ int8 dense
    Kernel(
        "w8a8_scaled_mm",
        "w8a8_int8",
        "INT8 W8A8, per-token activation scales and per-channel weight scales: i8 16x16x64 MFMA, exact "
        "int32 accumulator over all of K, epilogue (acc * sa) * sw to bf16. M <= 64 streams the weights "
        "once with the K loop split across the block's waves; larger M runs the LDS-tiled kernel. "
        "K % 128 == 0",
        {"weight_dtype": "int8", "granularity": "token", "dtype": ("bf16", "fp16")},
        {"tiles": "stream 16/32/64 x 16, tiled 256x64, 128x256"},
    ),
    Kernel(
        "w8a8_scaled_mm_cfg",
        "w8a8_int8_tile_sweep",
        "w8a8_scaled_mm pinned to one tile config (0..12), for tile sweeps",
        {"weight_dtype": "int8", "granularity": "token"},
    ),
    Kernel(
        "w8a8_wmma_gemm",
        "w8a16",
        "prefill GEMM: int8 activations quantized per (row, 128-element group) inside the op, i8 MFMA, "
        "fp32 group-scale fold, uint8b128 weights flipped to signed on the fly. K % 128 == 0",
        {"weight_bits": 8, "group_size": (0, 128), "rows": Range(lo=6), "dtype": ("bf16", "fp16")},
    ),
    Kernel(
        "w8a8_wmma_gemm_cfg",
        "w8a8_tile_sweep",
        "the W8A8 group GEMM pinned to one tile config (0..12), same math and activation quantize",
        {"weight_bits": 8, "rows": Range(lo=1), "dtype": ("bf16", "fp16")},
        {"cfgs": "0 stream 16 | 1 stream 32 | 2 stream 64 | 3 tiled 128x128 | 4 tiled 256x64 | "
                 "5 tiled 256x256 | 6 tiled 128x256"},
    ),
    # ------------------------------------------------------------ fp8 dense
    Kernel(
        "fp8_w8a8_block_gemm",
        "fp8_w8a8",
        "FP8-block W8A8: e4m3 activations with 1x128 fp32 scales, e4m3 weights with 128x128 fp32 block "
        "scales, native e4m3 16x16x128 MFMA (one instruction per scale block) and an fp32 fold "
        "acc += part * sa * sw per 128-K block. M <= 64 streams the weights (decode), larger M uses "
        "direct global->LDS copies into a fragment-native layout. K % 128 == 0",
        {"weight_dtype": "fp8_e4m3", "activation_dtype": "fp8_e4m3", "group_size": 128},
        {"tiles": "stream 16/32/64 x 16 (8 waves split K), tiled 256x64 (M <= 256), 128x256"},
    ),
    Kernel(
        "fp8_w8a8_block_gemm_cfg",
        "fp8_w8a8_tile_sweep",
        "fp8_w8a8_block_gemm pinned to one tile config (0..12)",
        {"weight_dtype": "fp8_e4m3", "activation_dtype": "fp8_e4m3", "group_size": 128},
    ),
    Kernel(
        "weight8_kmajor",
        "weight8_kmajor",
        "8-bit weights [E, N, K] -> K-block-major [E, K/128, N, 128]: one contiguous run per 128-K block, "
        "so the blocks the GEMM streams at one moment lie together in memory. K % 128 == 0",
        {"weight_dtype": ("fp8_e4m3", "int8", "uint8"), "group_size": 128},
    ),
    Kernel(
        "fp8_w8a8_block_gemm_kmajor",
        "fp8_w8a8_kmajor",
        "fp8_w8a8_block_gemm on K-block-major weights: the same kernels and tiles, bit-identical output",
        {"weight_dtype": "fp8_e4m3", "activation_dtype": "fp8_e4m3", "group_size": 128},
    ),
    # ------------------------------------------------------------ moe
    Kernel(
        "moe_route_topk",
        "moe_route",
        "router: fp32 softmax -> top-k by logit (ties to the lower expert id) -> optional renormalize; "
        "one wave per token",
        {"logits_dtype": ("fp32", "bf16"), "num_experts": Range(hi=1024)},
    ),
    Kernel(
        "moe_align",
        "moe_align_small",
        "moe_align_block_size contract in one 1024-thread block: LDS histogram, block scan, stable "
        "scatter by rank (up to 1024 slots)",
        {"num_experts": Range(lo=1, hi=1024), "num_slots": Range(hi=1024)},
    ),
    Kernel(
        "moe_align",
        "moe_align",
        "moe_align_block_size contract: stable counting sort of slot ids by expert (bit-exact, no "
        "atomics on global memory), each expert padded to block_m with id T*top_k",
        {"num_experts": Range(lo=1, hi=1024)},
    ),
    Kernel(
        "moe_route_align",
        "moe_route_align_small",
        "router top-k and align in one 1024-thread block launch (T <= 16, T * top_k <= 1024); the same "
        "outputs as moe_route_topk then moe_align",
        {"logits_dtype": ("fp32", "bf16"), "num_experts": Range(hi=1024), "tokens": Range(lo=1, hi=16),
         "num_slots": Range(hi=1024)},
    ),
    Kernel(
        "moe_align_quant",
        "moe_align_quant_small",
        "moe_align_small plus the tokens' e4m3 1x128 quantization in the same single-block launch",
        {"dtype": ("bf16", "fp16"), "num_experts": Range(hi=1024), "num_slots": Range(hi=1024),
         "tokens": Range(hi=64), "group_size": 128},
    ),
    Kernel(
        "moe_align_quant",
        "moe_align_then_quant",
        "moe_align then fp8_quant_group128 (above 1024 slots or 64 tokens)",
        {"dtype": ("bf16", "fp16"), "num_experts": Range(hi=1024), "group_size": 128},
    ),
    Kernel(
        "moe_route_align_quant",
        "moe_route_align_quant_small",
        "moe_route_align_small plus the tokens' e4m3 1x128 quantization, done by the waves the router leaves "
        "idle: router, align and quantizer in one launch",
        {"logits_dtype": ("fp32", "bf16"), "dtype": ("bf16", "fp16"), "num_experts": Range(hi=1024),
         "tokens": Range(lo=1, hi=16), "num_slots": Range(hi=1024), "group_size": 128},
    ),
    Kernel(
        "moe_route_align_quant",
        "moe_route_align_then_quant",
        "moe_route_align then fp8_quant_group128 (above 16 tokens or 1024 slots)",
        {"logits_dtype": ("fp32", "bf16"), "dtype": ("bf16", "fp16"), "num_experts": Range(hi=1024),
         "group_size": 128},
    ),
    Kernel(
        "moe_route_align",
        "moe_route_then_align",
        "moe_route_topk (one wave per token, grid-wide) then moe_align",
        {"logits_dtype": ("fp32", "bf16"), "num_experts": Range(hi=1024)},
    ),
    Kernel(
        "moe_sum",
        "moe_sum",
        "out[t] = sum_j y[t, j] over top-k slots, fp32 in slot order",
        {"dtype": ("bf16", "fp16")},
    ),
    Kernel(
        "moe_weighted_sum",
        "moe_sum",
        "out[t] = sum_j w[t, j] * y[t, j] (the top-k weighted combine when w2 does not apply weights)",
        {"dtype": ("bf16", "fp16"), "weighted": True},
    ),
    Kernel(
        "moe_gemm_fp8_w8a8",
        "moe_gemm_fp8_w8a8",
        "FP8-block W8A8 expert GEMM over aligned sorted ids: e4m3 activations (1x128 scales) x e4m3 "
        "experts [E, N, K] with [E, N/128, K/128] scales, e4m3 MFMA, gated act*mul epilogue for w13 "
        "(c gets N/2 columns) or top-k weight for w2. block_m 16/32 stream the experts, 64+ tile",
        {"silu_mul": (True, False), "weight_dtype": "fp8_e4m3", "activation": ("silu", "gelu_tanh"),
         "quant": "fp8_w8a8"},
        _MOE_TILES,
    ),
    # ------------------------------------------------ 16-bit MFMA over dequantized weights
    Kernel(
        "moe_gemm_mxfp4",
        "moe_gemm_mxfp4",
        "MXFP4 expert GEMM: e2m1 nibbles [E, N, K/2] (low nibble = even k) with e8m0 [E, N, K/32] decoded "
        "exactly to bf16 once per block into LDS, bf16 16x16x32 MFMA, bf16 activations (W4A16); fused "
        "act*mul (w13) or top-k weight (w2). K % 64 == 0 (2880 is fine), ragged N",
        {"silu_mul": (True, False), "dtype": "bf16", "weight_dtype": "uint8", "weight_bits": 4, "quant": "mxfp4",
         "group_size": 32, "activation": ("silu", "gelu_tanh")},
        _MOE_TILES,
    ),
    Kernel(
        "moe_gemm_w4a16_zp",
        "moe_gemm_w4a16",
        "WNA16 expert GEMM with zero points (AWQ-style): uint4 [E, N, K/8] int32 words (k = 8w + j in "
        "nibble j), bf16/fp16 scales and uint4 zero points [E, N/2, K/G]; (q - z) * s decoded to bf16 in LDS",
        {"silu_mul": (True, False), "dtype": "bf16", "weight_bits": 4, "quant": "wna16", "has_zp": True,
         "group_size": (32, 64, 128), "activation": ("silu", "gelu_tanh")},
        _MOE_TILES,
    ),
    Kernel(
        "moe_gemm_w4a16",
        "moe_gemm_w4a16",
        "WNA16 symmetric expert GEMM over vLLM's Triton layout: uint8 [E, N, K/2] (low nibble = even k), "
        "(q - 8) * s decoded to bf16 in LDS",
        {"silu_mul": (True, False), "dtype": "bf16", "weight_dtype": "uint8", "weight_bits": 4, "quant": "wna16",
         "has_zp": False, "group_size": (32, 64, 128), "activation": ("silu", "gelu_tanh")},
        _MOE_TILES,
    ),
    Kernel(
        "moe_gemm_bf16",
        "moe_gemm",
        "unquantized bf16 expert GEMM: both operands by direct global->LDS copy, bf16 MFMA, same fused "
        "epilogues",
        {"silu_mul": (True, False), **_BF16, "weight_dtype": "bf16", "quant": "none",
         "activation": ("silu", "gelu_tanh")},
        _MOE_TILES,
    ),
    Kernel(
        "moe_gemm_w8a16",
        "moe_gemm_w8a16",
        "int8 experts [E, N, K] with per-channel scales ([E, N] or [E, N, 1]), int8 * scale decoded to bf16 in "
        "LDS, bf16 activations (W8A16)",
        {"silu_mul": (True, False), **_BF16, "weight_dtype": "int8", "weight_bits": 8, "quant": "int8",
         "group_size": (0,), "activation": ("silu", "gelu_tanh")},
        _MOE_TILES,
    ),
    Kernel(
        "moe_gemm_fp8",
        "moe_gemm_fp8",
        "e4m3 experts with 128x128 block scales [E, N/128, K/128] or per-channel scales, decoded with the "
        "scale to bf16 in LDS, bf16 activations (W8A16)",
        {"silu_mul": (True, False), **_BF16, "weight_dtype": "fp8_e4m3", "weight_bits": 8, "quant": "fp8",
         "group_size": (0, 128), "activation": ("silu", "gelu_tanh")},
        _MOE_TILES,
    ),
    Kernel(
        "moe_gemm_fp8_raw",
        "moe_gemm_fp8",
        "the same with fp16 activations: weights decoded to fp16, f16 MFMA; fp16 or bf16 output (the c tensor's "
        "dtype)",
        {"silu_mul": (True, False), "dtype": "fp16", "weight_dtype": "fp8_e4m3", "weight_bits": 8, "quant": "fp8",
         "group_size": (0, 128), "activation": ("silu", "gelu_tanh")},
        _MOE_TILES,
    ),
    Kernel(
        "mxfp4_wmma_gemm",
        "mxfp4",
        "dense MXFP4 W4A16: packed e2m1 [N, K/2] + e8m0 [N, K/32], read in place (decode in registers for "
        "M <= 64, decoded into LDS once per block otherwise), bf16 MFMA, optional [N] or [M, N] bias. K % 64 == 0",
        {"weight_bits": 4, "group_size": 32, "dtype": ("bf16", "fp16"), "scale_dtype": "e8m0"},
        {"tiles": "stream 16/32/64 rows, tiled 128x128"},
    ),
    Kernel(
        "mxfp4_wmma_gemm_cfg",
        "mxfp4_tile_sweep",
        "mxfp4_wmma_gemm pinned to one tile config: 0 stream16 | 1 stream32 | 2 stream64 | 3 tiled 128x128 | "
        "4 tiled 256x128 | 5 tiled 64x128",
        {"weight_bits": 4, "group_size": 32, "dtype": ("bf16", "fp16")},
    ),
    Kernel(
        "mxfp4_dequant",
        "mxfp4_dequant",
        "MXFP4 [N, K/2] + e8m0 [N, K/32] -> bf16 [N, K], exact (e2m1 times a power of two), zero blocks for "
        "an e8m0 byte of 0",
        {"weight_bits": 4, "group_size": 32, "dtype": "bf16"},
        {"threads": 256},
    ),
    Kernel(
        "fp8_wmma_gemm",
        "fp8",
        "dense FP8 W8A16: e4m3 [N, K] with 128x128 block or per-channel scales decoded to bf16, bf16 MFMA",
        {"weight_bits": 8, "weight_dtype": "fp8_e4m3", "group_size": (0, 128), "rows": Range(lo=1), "dtype": "bf16"},
    ),
    Kernel(
        "fp8_wmma_gemm_raw",
        "fp8",
        "dense FP8 W8A16 with fp16 activations: e4m3 decoded with its scale to fp16, f16 MFMA, bf16 output",
        {"weight_bits": 8, "weight_dtype": "fp8_e4m3", "group_size": (0, 128), "rows": Range(lo=1), "dtype": "fp16"},
    ),
    Kernel(
        "fp8_wmma_gemm_cfg",
        "fp8_tile_sweep",
        "fp8_wmma_gemm pinned to one tile config (0..7)",
        {"weight_bits": 8, "weight_dtype": "fp8_e4m3", "group_size": (0, 128), "dtype": "bf16"},
    ),
    Kernel(
        "fp8_wmma_gemm_raw_cfg",
        "fp8_tile_sweep",
        "fp8_wmma_gemm_raw pinned to one tile config (0..7)",
        {"weight_bits": 8, "weight_dtype": "fp8_e4m3", "group_size": (0, 128), "dtype": "fp16"},
    ),
    Kernel(
        "fp8_dequant",
        "fp8_dequant",
        "float8_e4m3fn [N, K] + 128x128 block or per-channel scales -> bf16 [N, K] (exact decode, one "
        "rounding at the scale multiply)",
        {"weight_bits": 8, "weight_dtype": "fp8_e4m3", "group_size": (0, 128), "dtype": "bf16"},
        {"threads": 256},
    ),
    # ------------------------------------------------------------ weight-only decode ops
    Kernel(
        "w8a16_skinny_gemm",
        "w8a16",
        "decode GEMM (M <= 8) on the raw uint8b128 weight bytes with per-channel or 32/64/128 group scales in "
        "the activation dtype: weights decoded to bf16/fp16 in registers, 16x16x32 MFMA, no activation "
        "quantize. K % 64 == 0",
        {"weight_bits": 8, "group_size": (0, 32, 64, 128), "rows": Range(hi=8), "dtype": ("bf16", "fp16")},
        {"kernel": "stream16 (M <= 32 path of strix_w16_gemm)"},
    ),
    Kernel(
        "w8a16_gemm",
        "w8a16",
        "the same uint8b128 W8A16 contraction at any M (bf16/fp16 activations as given, weights decoded "
        "exactly): the prefill path of layers whose 32/64-element groups the W8A8 op does not take. "
        "K % 64 == 0",
        {"weight_bits": 8, "group_size": (0, 32, 64, 128), "dtype": ("bf16", "fp16")},
        {"kernel": "stream16 to 64 rows, tiled16 above"},
    ),
    Kernel(
        "fp8_skinny_gemm",
        "fp8",
        "decode GEMM (M <= 8) on float8_e4m3fn weights with fp32 scales per (row, 128-K block) [N, K/128] or "
        "per channel [N]; e4m3 -> fp32 with gfx950's v_cvt_pk_f32_fp8, bf16 MFMA. K % 64 == 0",
        {"weight_bits": 8, "weight_dtype": "fp8_e4m3", "group_size": (0, 128), "rows": Range(hi=8),
         "dtype": ("bf16", "fp16")},
        {"kernel": "stream16"},
    ),
    Kernel(
        "mxfp4_gemv",
        "mxfp4_gemv",
        "MXFP4 W4A16 for M <= 8: the packed e2m1 stream decoded in registers, one 16-row subtile per wave "
        "with K split across the block, bf16 MFMA",
        {"weight_bits": 4, "group_size": 32, "dtype": "bf16", "m_max": 8},
        {"kernel": "stream16"},
    ),
    Kernel(
        "w4a16_wmma_gemm",
        "w4a16",
        "uint4b8 weights in the RDNAHybridW4A16 word order (nibble j of each 32-bit word is k = 0 2 4 6 1 3 5 7) "
        "with bf16 group scales: decoded to bf16 in registers (M <= 32) or into LDS by producer waves while "
        "consumer waves run bf16 MFMA (prefill). K % 64 == 0, group % 32 == 0",
        {"weight_bits": 4, "group_size": (32, 64, 128), "rows": Range(lo=1), "dtype": "bf16",
         "scale_dtype": "bf16"},
    ),
    Kernel(
        "w4a16_dequant",
        "w4a16_dequant",
        "RDNAHybridW4A16 int4 [N, K/2] + bf16 group scales -> bf16 [N, K], exact bf16 of (u4 - 8) * scale",
        {"weight_bits": 4, "group_size": (32, 64, 128), "dtype": "bf16"},
        {"threads": 256},
    ),
    Kernel(
        "w4a8_wmma_gemm",
        "w4a16",
        "uint4b8 RDNAHybridW4A16 weights x activations quantized to int8 per (row, 128-group) in the op: "
        "nibbles widened to int8 in the tile, int8 MFMA, an exact int32 sum per 128-group folded in fp32 "
        "with both scales (weight group 0 or 128); 32-element weight groups dequantize the int8 activations "
        "for the int4 bf16-MFMA GEMM. K % 128 == 0",
        {"weight_bits": 4, "group_size": (0, 32, 128), "rows": Range(lo=1), "dtype": "bf16"},
    ),
    Kernel(
        "moe_gemm_w4a8",
        "moe_gemm_w4a8",
        "expert GEMM over the WNA16 int4 layout (low nibble = even k, q - 8, bf16/fp16 scales per 128-K group) "
        "with int8 activations per (row, 128-group): nibbles widened to int8 in the tile, int8 MFMA, an "
        "exact int32 sum per 128-group folded in fp32 with both scales, fused act*mul / top-k weight "
        "epilogues; tiles 64x128, 64x256, 128x128, 256x256",
        {"silu_mul": True, **_BF16, "activation_dtype": "int8", "weight_dtype": "uint8", "weight_bits": 4,
         "quant": "wna16", "group_size": (128,), "activation": ("silu", "gelu_tanh"), "block_m": (64, 128, 256)},
    ),
]

_selections: dict[tuple, dict[str, Any]] = {}


def ops() -> dict[str, list[str]]:
    """op -> names of the kernels implementing it, in priority order."""
    out: dict[str, list[str]] = {}
    for k in KERNELS:
        names = out.setdefault(k.op, [])
        if k.name not in names:
            names.append(k.name)
    return out


def geometries(op: str, *keys: str, **where: Any) -> set[tuple]:
    """Shape points of `op` as tuples of `keys`; `where` narrows the rows first.

    A row whose constraint for one of the keys is a set or a Range is not a
    point and contributes nothing."""
    points = set()
    for k in KERNELS:
        if k.op != op or not k.accepts(where):
            continue
        vals = []
        for key in keys:
            want = k.constraints.get(key)
            if not isinstance(want, _POINT_TYPES):
                break
            vals.append(_norm(want))
        else:
            points.add(tuple(vals))
    return points


def explain(op: str, **geometry: Any) -> list[dict[str, Any]]:
    verdicts = []
    for k in KERNELS:
        if k.op == op:
            reason = k.check(geometry)
            verdicts.append({"name": k.name, "ok": reason is None, "reason": reason})
    return verdicts


def select(op: str, **geometry: Any) -> str | None:
    rows = explain(op, **geometry)
    hit = next((r["name"] for r in rows if r["ok"]), None)
    key = (op, tuple(sorted((k, _norm(v)) for k, v in geometry.items())))
    rec = _selections.get(key)
    if rec is None:
        reason = None if hit else ("; ".join(r["reason"] for r in rows) or "no kernel")
        rec = _selections[key] = {"op": op, "query": dict(key[1]), "kernel": hit, "reason": reason, "count": 0}
    rec["count"] += 1
    return hit


def selections() -> list[dict[str, Any]]:
    return list(_selections.values())


def kernels() -> list[dict[str, Any]]:
    return [
        {"name": k.name, "op": k.op, "doc": k.doc, "constraints": dict(k.constraints), "spec": dict(k.spec)}
        for k in KERNELS
    ]
