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
    stream the experts (decode), 64+ run the LDS-tiled MFMA kernels, 256 once
    an expert fills a 256-row tile (measured on MI355X: 555 vs 621 us for
    config 3 at T=4096, 885 vs 1017 us for config 4 at T=2048, 1501 vs
    1697 us for config 5 at T=8192, against 128)."""
    per_expert = tokens * top_k / max(num_experts, 1)
    if per_expert <= 16:
        return 16
    if per_expert <= 32:
        return 32
    if per_expert <= 48:
        return 64
    if per_expert < 192:
        return 128
    return 256


def route_and_align(logits: torch.Tensor, top_k: int, num_experts: int, block_m: int, renormalize: bool = True):
    """Router top-k and the expert alignment (one launch up to 1024 slots)."""
    return S.moe_route_align(logits, top_k, block_m, renormalize)


def fused_moe_fp8_w8a8(x, logits, w13, w13_s, w2, w2_s, top_k: int, renormalize: bool = True,
                       activation: str = "silu", block_m: int | None = None):
    """FP8-block W8A8 fused MoE (config 3): route -> align -> e4m3 1x128 quant
    -> w13 (fused act*mul) -> e4m3 quant -> w2 (x top-k weight) -> sum.
    Expert weights are row-major [E, N, K] or K-block-major [E, K/128, N, 128]
    (weight8_kmajor), with the same result."""
    t, h = x.shape
    e, n13 = w13.size(0), (w13.size(2) if w13.dim() == 4 else w13.size(1))
    inter = n13 // 2
    bm = block_m or moe_block_m(t, top_k, e)
    ids, w, sorted_ids, expert_ids, num_post, qx, sx = S.moe_route_align_quant(logits, x, top_k, bm, renormalize)
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


def _fused_moe_16(x, logits, top_k, inter, hidden, num_experts, renormalize, activation, block_m, w13_call, w2_call):
    """route -> align -> w13 (fused act*mul) -> w2 (x top-k weight) -> sum, bf16 activations throughout."""
    t = x.size(0)
    bm = block_m or moe_block_m(t, top_k, num_experts)
    _, w, sorted_ids, expert_ids, num_post = route_and_align(logits, top_k, num_experts, bm, renormalize)
    slots = t * top_k
    h13 = torch.empty((slots, inter), dtype=x.dtype, device=x.device)
    w13_call(h13, x, sorted_ids, expert_ids, num_post, None, top_k, bm, True, activation)
    y = torch.empty((slots, hidden), dtype=x.dtype, device=x.device)
    w2_call(y, h13, sorted_ids, expert_ids, num_post, w.reshape(-1), 1, bm, False, activation)
    out = torch.empty((t, hidden), dtype=x.dtype, device=x.device)
    S.moe_sum(y.view(t, top_k, hidden), out)
    return out


def fused_moe_mxfp4(x, logits, w13, w13_s, w2, w2_s, top_k: int, renormalize: bool = True,
                    activation: str = "silu", block_m: int | None = None):
    """MXFP4 W4A16 fused MoE (config 4): e2m1 + e8m0 experts decoded to bf16 in LDS, bf16 MFMA."""
    e, n13, _ = w13.shape
    hidden = w2.size(1)

    def g13(c, a, si, ei, npp, tw, k, bm, silu, act):
        S.moe_gemm_mxfp4(c, a, w13, w13_s, si, ei, npp, tw, k, bm, 64, silu, act)

    def g2(c, a, si, ei, npp, tw, k, bm, silu, act):
        S.moe_gemm_mxfp4(c, a, w2, w2_s, si, ei, npp, tw, k, bm, 64, silu, act)

    return _fused_moe_16(x, logits, top_k, n13 // 2, hidden, e, renormalize, activation, block_m, g13, g2)


def fused_moe_wna16(x, logits, w13, w13_s, w13_z, w2, w2_s, w2_z, top_k: int, group: int = 128,
                    renormalize: bool = True, activation: str = "silu", block_m: int | None = None):
    """WNA16 int4 fused MoE with zero points (config 5): (q - z) * s decoded to bf16 in LDS, bf16 MFMA."""
    e, n13, _ = w13.shape
    hidden = w2.size(1)

    def g13(c, a, si, ei, npp, tw, k, bm, silu, act):
        S.moe_gemm_w4a16_zp(c, a, w13, w13_s, w13_z, si, ei, npp, tw, k, bm, 64, silu, act, group)

    def g2(c, a, si, ei, npp, tw, k, bm, silu, act):
        S.moe_gemm_w4a16_zp(c, a, w2, w2_s, w2_z, si, ei, npp, tw, k, bm, 64, silu, act, group)

    return _fused_moe_16(x, logits, top_k, n13 // 2, hidden, e, renormalize, activation, block_m, g13, g2)
