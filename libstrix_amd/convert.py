# SPDX-License-Identifier: MIT
"""Load-time converters from checkpoint layouts to the kernels' layouts.

AWQ (the AutoAWQ GEMM format) stores int4 weights transposed and packed
along the output dimension, with its own nibble order:

    qweight  int32 [..., K, N/8]    nibble i of word w = column 8w + AWQ_ORDER[i]
    qzeros   int32 [..., K/G, N/8]  the same packing of the uint4 zero points
    scales   fp16/bf16 [..., K/G, N]

value = (q - z) * s. The WNA16 zero-point kernels (`moe_gemm_w4a16_zp`) read

    b        int32 [..., N, K/8]    nibble j of word w = k 8w + j (byte-identical
                                    to uint8 [..., N, K/2], low nibble = even k)
    scales   [..., N, K/G]
    zeros    uint8 [..., N/2, K/G]  two uint4 per byte along N, even n low

The reference rejects zero points outright (python/strix_vllm/linear.py:
173-174, python/strix_vllm/moe.py:376), so it has no such converter. Leading
dims (experts) pass through. Every step is a torch view or elementwise op on
the tensors' own device, run once per checkpoint, never per forward.

The other load-time transforms live beside their layers:
`vllm_plugin.int8.prepare_weights` (compressed-tensors int8),
`vllm_plugin.fp8.prepare_block` (FP8 block scales, K-block-major re-layout),
`vllm_plugin.fp8.prepare_channel`, `vllm_plugin.linear.prepare_w8`
(uint8b128); Quark MXFP4 `u8 [N, K/2]` + `e8m0 [N, K/32]` is the kernels'
layout as loaded (`vllm_plugin.mxfp4.check_weights`).
"""

from __future__ import annotations

import torch

# AutoAWQ's pack order: nibble i (bits 4i..4i+3) of a word holds column 8w + AWQ_ORDER[i].
AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


def awq_unpack(packed: torch.Tensor) -> torch.Tensor:
    """int32 [..., R, C/8] AWQ words -> uint8 [..., R, C] values 0..15 in natural column order."""
    if packed.dtype != torch.int32:
        raise ValueError(f"AWQ tensors are int32, got {packed.dtype}")
    shifts = torch.tensor([4 * i for i in range(8)], dtype=torch.int32, device=packed.device)
    nib = (packed.unsqueeze(-1) >> shifts) & 0xF                      # [..., R, C/8, 8]: nibble i
    cols = torch.empty_like(nib)
    cols[..., list(AWQ_ORDER)] = nib                                   # column AWQ_ORDER[i] <- nibble i
    return cols.reshape(*packed.shape[:-1], packed.shape[-1] * 8).to(torch.uint8)


def pack_k_nibbles(q: torch.Tensor) -> torch.Tensor:
    """uint8 values [..., N, K] -> int32 [..., N, K/8] with nibble j of word w = k 8w + j
    (built as uint8 [..., N, K/2], low nibble = even k, viewed as little-endian words)."""
    if q.shape[-1] % 8:
        raise ValueError(f"K={q.shape[-1]} must be a multiple of 8")
    q = q.to(torch.uint8)
    return (q[..., 0::2] | (q[..., 1::2] << 4)).contiguous().view(torch.int32)


def pack_n_nibbles(z: torch.Tensor) -> torch.Tensor:
    """uint8 values [..., N, G] -> uint8 [..., N/2, G], even n in the low nibble."""
    if z.shape[-2] % 2:
        raise ValueError(f"N={z.shape[-2]} must be even")
    z = z.to(torch.uint8)
    return (z[..., 0::2, :] | (z[..., 1::2, :] << 4)).contiguous()


def awq_to_wna16(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
                 scale_dtype: torch.dtype = torch.bfloat16) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """AWQ (qweight [..., K, N/8], qzeros [..., K/G, N/8], scales [..., K/G, N])
    -> (b int32 [..., N, K/8], scales [..., N, K/G] in `scale_dtype`,
    zeros uint8 [..., N/2, K/G]) for moe_gemm_w4a16_zp. The group size is
    K / (K/G); it must divide K."""
    k, n8 = qweight.shape[-2:]
    kg, n = scales.shape[-2:]
    if n != 8 * n8 or tuple(qzeros.shape[-2:]) != (kg, n8) or qweight.shape[:-2] != scales.shape[:-2]:
        raise ValueError(f"AWQ shapes disagree: qweight {list(qweight.shape)}, qzeros {list(qzeros.shape)}, "
                         f"scales {list(scales.shape)}")
    if kg == 0 or k % kg:
        raise ValueError(f"{kg} scale groups do not divide K={k}")
    q = awq_unpack(qweight).transpose(-1, -2)          # [..., N, K]
    z = awq_unpack(qzeros).transpose(-1, -2)           # [..., N, K/G]
    b = pack_k_nibbles(q)
    s = scales.transpose(-1, -2).to(scale_dtype).contiguous()
    return b, s, pack_n_nibbles(z)
