# SPDX-License-Identifier: MIT
"""Host-side compositions of torch.ops.strix.* for whole layers.

These are the call chains the reference's plugin runs per forward
(python/strix_vllm/int8.py:22-29, python/strix_vllm/fp8.py:60-91,
python/strix_vllm/moe.py:905-1014), with the W8A8 activation quantizers and
the routing, alignment and combine steps as native kernels. Every step is a
HIP launch on the current stream; nothing syncs the host.
"""

from __future__ import annotations

import torch

S = torch.ops.strix


def w8a8_int8_linear(x: torch.Tensor, w: torch.Tensor, sw: torch.Tensor, bias: torch.Tensor | None = None):
    """INT8 W8A8 linear (config 1): per-token int8 activations x per-channel int8 weights."""
    q, s = S.int8_quant_per_token(x)
    out = S.w8a8_scaled_mm(q, s, w, sw)
    return out if bias is None else out + bias


def fp8_block_linear(x: torch.Tensor, w: torch.Tensor, sw: torch.Tensor, bias: torch.Tensor | None = None):
    """FP8-block W8A8 linear (config 2): 1x128 e4m3 activations x 128x128 e4m3 weights."""
    q, s = S.fp8_quant_group128(x)
    out = S.fp8_w8a8_block_gemm(q, s, w, sw)
    return out if bias is None else out + bias


def moe_block_m(tokens: int, top_k: int, num_experts: int) -> int:
    """Sorted-id block size by the average rows per expert: the 16/32 blocks
    stream the experts (decode), 64+ run the LDS-tiled MFMA kernels."""
    per_expert = tokens * top_k / max(num_experts, 1)
    if per_expert <= 16:
        return 16
    if per_expert <= 32:
        return 32
    if per_expert <= 96:
        return 64
    return 128


def route_and_align(logits: torch.Tensor, top_k: int, num_experts: int, block_m: int, renormalize: bool = True):
    ids, w = S.moe_route_topk(logits, top_k, renormalize)
    sorted_ids, expert_ids, num_post = S.moe_align(ids, num_experts, block_m)
    return ids, w, sorted_ids, expert_ids, num_post


def fused_moe_fp8_w8a8(x, logits, w13, w13_s, w2, w2_s, top_k: int, renormalize: bool = True,
                       activation: str = "silu", block_m: int | None = None):
    """FP8-block W8A8 fused MoE (config 3): route -> align -> e4m3 1x128 quant
    -> w13 (fused act*mul) -> e4m3 quant -> w2 (x top-k weight) -> sum."""
    t, h = x.shape
    e, n13, _ = w13.shape
    inter = n13 // 2
    bm = block_m or moe_block_m(t, top_k, e)
    ids, w, sorted_ids, expert_ids, num_post = route_and_align(logits, top_k, e, bm, renormalize)
    qx, sx = S.fp8_quant_group128(x)
    slots = t * top_k
    h13 = torch.empty((slots, inter), dtype=torch.bfloat16, device=x.device)
    S.moe_gemm_fp8_w8a8(h13, qx, sx, w13, w13_s, sorted_ids, expert_ids, num_post, None, top_k, bm, 128, True,
                        activation)
    qi, si = S.fp8_quant_group128(h13)
    y = torch.empty((slots, h), dtype=torch.bfloat16, device=x.device)
    S.moe_gemm_fp8_w8a8(y, qi, si, w2, w2_s, sorted_ids, expert_ids, num_post, w.reshape(-1), 1, bm, 128, False,
                        activation)
    out = torch.empty((t, h), dtype=torch.bfloat16, device=x.device)
    S.moe_sum(y.view(t, top_k, h), out)
    return out
