# SPDX-License-Identifier: MIT
"""Fused-MoE experts on gfx950: tile tables, gates, the expert chains and the
vLLM hooks.

The reference (python/strix_vllm/moe.py:1-1108) swaps vLLM's Triton experts
for its grouped GEMMs: bf16 (`moe_gemm_bf16`), int4 WNA16 (`moe_gemm_w4a16`,
W4A8 prefill opt-in), int8 W8A16 (opt-in) and FP8 (`moe_gemm_fp8[_raw]`,
bf16/fp16 activations). Each chain is: align the routed slots by expert
(vLLM's `moe_align_block_size`), w13 with the gate activation-and-mul fused
into its epilogue, w2 with the top-k weight fused into its epilogue, then
vLLM's `moe_sum` over the top-k copies.

Here every step is a libstrix_amd op on the current stream: `moe_align`
(the same sorted-ids contract, stable within an expert), the grouped GEMMs,
and `moe_sum`. The FP8 chain keeps vLLM's W8A8 numerics on gfx950's FP8 MFMA
(e4m3 activations per (row, 128-element group), `moe_gemm_fp8_w8a8`) for
128x128 block-scaled experts; per-channel FP8 experts take the W8A16 kernel
(bf16 activations). int4 experts with zero points (`moe_gemm_w4a16_zp`) and
MXFP4 experts (`moe_gemm_mxfp4`) have chains too (the reference has neither).

The `*_experts` functions are vLLM-free (tested directly); the classes made
by `_make_*_cls` subclass vLLM's experts and call them.
"""

from __future__ import annotations

import os

import torch

from libstrix_amd.vllm_plugin import disabled, model_gate

# ---------------------------------------------------------------- tile tables
# The sorted-id block (block_m) picks the kernel family: 16 streams the
# experts' weights through a per-wave LDS ring (decode), 32 a register-pipelined
# stream, 64/128/256 the LDS-tiled MFMA kernels. It is chosen from the mean
# rows per expert, tokens * top_k / E (functional.moe_block_m), so one table
# serves every model shape (the reference keys per-model tables on the token
# count alone, python/strix_vllm/moe.py:40-138).
def _block_m(num_tokens: int, top_k: int, num_experts: int) -> int:
    from libstrix_amd.functional import moe_block_m

    return moe_block_m(num_tokens, top_k, num_experts)


def _block_n(*ns: int) -> int:
    return 128 if all(n % 128 == 0 for n in ns) else 64


def strix_blocks(num_tokens: int, top_k: int = 8, num_experts: int = 128, n: int = 0, k: int = 0) -> tuple[int, int]:
    """(block_m, block_n) for the bf16-activation expert GEMMs (bf16, int4,
    MXFP4, FP8 W8A16): both GEMMs share one alignment, so one block_m
    (python/strix_vllm/moe.py:40-47)."""
    return _block_m(num_tokens, top_k, num_experts), 64


def fp8_blocks(num_tokens: int, top_k: int = 8, num_experts: int = 128) -> tuple[int, int]:
    """(block_m, block_n) for the FP8 W8A8 expert GEMMs (python/strix_vllm/moe.py:82-91)."""
    return _block_m(num_tokens, top_k, num_experts), 128


def fp8_raw_blocks(num_tokens: int, n: int = 0, k: int = 0, top_k: int = 8, num_experts: int = 128) -> tuple[int, int]:
    """Tiles for the W8A16 FP8 expert kernels (`moe_gemm_fp8`, and
    `moe_gemm_fp8_raw` with fp16 activations), which share the bf16-MFMA
    kernel family on gfx950 (python/strix_vllm/moe.py:66-79)."""
    return strix_blocks(num_tokens, top_k, num_experts)


def wna16_blocks(num_tokens: int, n: int, k: int, top_k: int = 8, num_experts: int = 128) -> tuple[int, int]:
    """int4 expert tiles (python/strix_vllm/moe.py:134-138)."""
    return strix_blocks(num_tokens, top_k, num_experts)


# (n, k) -> the fewest rows at which the strix expert GEMM beat vLLM's own
# (python/strix_vllm/moe.py:141-159). No floor has been measured on gfx950: a
# missing key means the strix kernel is taken.
_MIN_ROWS: dict[tuple[int, int], int] = {}


def strix_moe_ok(rows: int, n: int, k: int) -> bool:
    return rows >= _MIN_ROWS.get((n, k), 0)


# int8 activations into the int4 expert GEMMs (moe_gemm_w4a8): opt-in
# (STRIX_ENABLE=moe_w4a8), prefill sizes only, 128-element groups
# (python/strix_vllm/moe.py:607-624).
_W4A8_MIN_TOKENS = int(os.environ.get("STRIX_MOE_W4A8_MIN_TOKENS", "1024"))


def _w4a8_ok(num_tokens: int, group: int, n: int, k: int) -> bool:
    return (not disabled("moe_w4a8") and num_tokens >= _W4A8_MIN_TOKENS and group == 128 and n % 128 == 0
            and k % 128 == 0)


def w4a8_blocks(num_tokens: int, top_k: int, num_experts: int) -> tuple[int, int]:
    """(block_m, block_n) of moe_gemm_w4a8 (its N are multiples of 128,
    _w4a8_ok): 128 x 128 once the experts
    average 128 routed rows, else 64 x 128. Measured on the C5 expert shapes
    (w13 + w2): 8192 tokens 510 + 404 us at 128 x 128 against 615 + 497 at
    64 x 128 and 565 + 429 at 256 x 256; 2048 tokens 172 + 117 against
    185 + 120; 64 tokens 68 + 42 at 64 x 128 against 99 + 60."""
    if num_tokens * top_k >= 128 * num_experts:
        return 128, 128
    return 64, 128


# ---------------------------------------------------------------- expert chains
S = torch.ops.strix


def _buf(workspace: torch.Tensor | None, shape: tuple[int, int], dtype, device) -> torch.Tensor:
    """A [rows, cols] view of a caller workspace (vLLM's _resize_cache), or a new tensor."""
    numel = shape[0] * shape[1]
    if workspace is not None and workspace.dtype == dtype and workspace.numel() >= numel and workspace.is_contiguous():
        return workspace.view(-1)[:numel].view(shape)
    return torch.empty(shape, dtype=dtype, device=device)


def _route(topk_ids: torch.Tensor, num_experts: int, bm: int):
    ids = topk_ids if topk_ids.dtype == torch.int32 and topk_ids.is_contiguous() else topk_ids.to(torch.int32).contiguous()
    return S.moe_align(ids, num_experts, bm)


def _weights(topk_weights: torch.Tensor, apply_router_weight_on_input: bool) -> torch.Tensor | None:
    return None if apply_router_weight_on_input else topk_weights.reshape(-1).to(torch.float32).contiguous()


def _act(activation) -> str:
    return getattr(activation, "value", activation)


def _chain(output, hidden_states, topk_weights, topk_ids, num_experts, n13, k_out, bm, apply_router_weight_on_input,
           workspace13, workspace2, w13_call, w2_call, inter_dtype=None, routed=None):
    """align -> w13 (act*mul fused) -> w2 (x top-k weight) -> sum over top-k.
    `routed` is an align already done by the caller (sorted_ids, expert_ids,
    num_post_padded)."""
    t = hidden_states.size(0)
    top_k = topk_ids.size(1)
    sorted_ids, expert_ids, num_post = routed if routed is not None else _route(topk_ids, num_experts, bm)
    slots = t * top_k
    cache2 = _buf(workspace13, (slots, n13 // 2), inter_dtype or hidden_states.dtype, hidden_states.device)
    w13_call(cache2, sorted_ids, expert_ids, num_post, top_k)
    cache3 = _buf(workspace2, (slots, k_out), hidden_states.dtype, hidden_states.device)
    w2_call(cache3, cache2, sorted_ids, expert_ids, num_post, _weights(topk_weights, apply_router_weight_on_input))
    if output is None:
        output = torch.empty((t, k_out), dtype=hidden_states.dtype, device=hidden_states.device)
    S.moe_sum(cache3.view(t, top_k, k_out), output)
    return output


def bf16_experts(output, hidden_states, w1, w2, topk_weights, topk_ids, activation="silu",
                 apply_router_weight_on_input=False, workspace13=None, workspace2=None):
    """Unquantized experts (python/strix_vllm/moe.py:228-332): w1 [E, 2I, H], w2 [E, H, I] bf16."""
    e, n13, _ = w1.shape
    k_out = w2.size(1)
    bm, bn = strix_blocks(hidden_states.size(0), topk_ids.size(1), e)
    act = _act(activation)

    def g13(c, si, ei, npp, top_k):
        S.moe_gemm_bf16(c, hidden_states, w1, si, ei, npp, None, top_k, bm, bn, True, act)

    def g2(c, a, si, ei, npp, wts):
        S.moe_gemm_bf16(c, a, w2, si, ei, npp, wts, 1, bm, bn, False, "silu")

    return _chain(output, hidden_states, topk_weights, topk_ids, e, n13, k_out, bm, apply_router_weight_on_input,
                  workspace13, workspace2, g13, g2)


def fp8_experts(output, hidden_states, w1, w2, s1, s2, topk_weights, topk_ids, activation="silu",
                apply_router_weight_on_input=False, workspace13=None, workspace2=None, w8a8=True):
    """FP8 experts (python/strix_vllm/moe.py:905-1014). s1/s2 fp32 block
    scales [E, N/128, K/128] run W8A8 (e4m3 activations) unless `w8a8` is
    False; per-channel scales [E, N] run W8A16 (bf16 activations)."""
    e, n13, _ = w1.shape
    k_out = w2.size(1)
    t, top_k = hidden_states.size(0), topk_ids.size(1)
    act = _act(activation)
    block = s1.dim() == 3 and s1.size(2) != 1
    routed = None
    if block and w8a8:
        bm, bn = fp8_blocks(t, top_k, e)[0], _block_n(n13, k_out)
        # The align and the activation quant in one call (one launch for decode).
        ids = topk_ids if topk_ids.dtype == torch.int32 and topk_ids.is_contiguous() else \
            topk_ids.to(torch.int32).contiguous()
        *routed, qx, sx = S.moe_align_quant(ids, hidden_states.contiguous(), e, bm)

        def g13(c, si, ei, npp, k):
            S.moe_gemm_fp8_w8a8(c, qx, sx, w1, s1, si, ei, npp, None, k, bm, bn, True, act)

        def g2(c, a, si, ei, npp, wts):
            qi, sq = S.fp8_quant_group128(a)
            S.moe_gemm_fp8_w8a8(c, qi, sq, w2, s2, si, ei, npp, wts, 1, bm, bn, False, "silu")
    else:
        bm, bn = fp8_raw_blocks(t, n13, w1.size(2), top_k, e)
        x = hidden_states if hidden_states.dtype == torch.bfloat16 else hidden_states.to(torch.bfloat16)

        def g13(c, si, ei, npp, k):
            S.moe_gemm_fp8(c, x, w1, s1, si, ei, npp, None, k, bm, bn, True, act)

        def g2(c, a, si, ei, npp, wts):
            S.moe_gemm_fp8(c, a, w2, s2, si, ei, npp, wts, 1, bm, bn, False, "silu")

    return _chain(output, hidden_states, topk_weights, topk_ids, e, n13, k_out, bm, apply_router_weight_on_input,
                  workspace13, workspace2, g13, g2, inter_dtype=torch.bfloat16, routed=routed)


def wna16_experts(output, hidden_states, w1, w2, s1, s2, topk_weights, topk_ids, group: int, activation="silu",
                  apply_router_weight_on_input=False, workspace13=None, workspace2=None, z1=None, z2=None,
                  w4a8=False):
    """int4 experts (python/strix_vllm/moe.py:335-604): uint8 [E, N, K/2]
    (low nibble first, symmetric (q - 8) * s) or, with zero points z1/z2,
    int32-packed [E, N, K/8] with (q - z) * s. `w4a8` (128-element groups)
    quantizes the activations to int8 per (row, 128) first."""
    e, n13 = w1.shape[0], w1.shape[1]
    k_out = w2.size(1)
    t, top_k = hidden_states.size(0), topk_ids.size(1)
    act = _act(activation)
    if w4a8 and z1 is None:
        bm, bn = w4a8_blocks(t, top_k, e)

        def q8(x):
            q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
            sa = torch.empty((x.size(0), x.size(1) // 128), dtype=torch.float32, device=x.device)
            S.moe_act_quant_i8(x, q, sa)
            return q, sa

        qx, sx = q8(hidden_states.contiguous())

        def g13(c, si, ei, npp, k):
            S.moe_gemm_w4a8(c, qx, sx, w1, s1, si, ei, npp, None, k, bm, bn, True, act)

        def g2(c, a, si, ei, npp, wts):
            qi, sq = q8(a)
            S.moe_gemm_w4a8(c, qi, sq, w2, s2, si, ei, npp, wts, 1, bm, bn, False, "silu")
    elif z1 is None:
        bm, bn = wna16_blocks(t, n13, 2 * w1.size(2), top_k, e)

        def g13(c, si, ei, npp, k):
            S.moe_gemm_w4a16(c, hidden_states, w1, s1, si, ei, npp, None, k, bm, bn, True, act, group)

        def g2(c, a, si, ei, npp, wts):
            S.moe_gemm_w4a16(c, a, w2, s2, si, ei, npp, wts, 1, bm, bn, False, "silu", group)
    else:
        bm, bn = wna16_blocks(t, n13, 0, top_k, e)

        def g13(c, si, ei, npp, k):
            S.moe_gemm_w4a16_zp(c, hidden_states, w1, s1, z1, si, ei, npp, None, k, bm, bn, True, act, group)

        def g2(c, a, si, ei, npp, wts):
            S.moe_gemm_w4a16_zp(c, a, w2, s2, z2, si, ei, npp, wts, 1, bm, bn, False, "silu", group)

    return _chain(output, hidden_states, topk_weights, topk_ids, e, n13, k_out, bm, apply_router_weight_on_input,
                  workspace13, workspace2, g13, g2)


def int8_experts(output, hidden_states, w1, w2, s1, s2, topk_weights, topk_ids, activation="silu",
                 apply_router_weight_on_input=False, workspace13=None, workspace2=None):
    """int8 per-channel experts, W8A16 (python/strix_vllm/moe.py:640-815)."""
    e, n13, _ = w1.shape
    k_out = w2.size(1)
    bm, bn = strix_blocks(hidden_states.size(0), topk_ids.size(1), e)
    act = _act(activation)

    def g13(c, si, ei, npp, k):
        S.moe_gemm_w8a16(c, hidden_states, w1, s1, si, ei, npp, None, k, bm, bn, True, act)

    def g2(c, a, si, ei, npp, wts):
        S.moe_gemm_w8a16(c, a, w2, s2, si, ei, npp, wts, 1, bm, bn, False, "silu")

    return _chain(output, hidden_states, topk_weights, topk_ids, e, n13, k_out, bm, apply_router_weight_on_input,
                  workspace13, workspace2, g13, g2)


def mxfp4_experts(output, hidden_states, w1, w2, s1, s2, topk_weights, topk_ids, activation="silu",
                  apply_router_weight_on_input=False, workspace13=None, workspace2=None):
    """MXFP4 experts: uint8 [E, N, K/2] e2m1 + e8m0 [E, N, K/32], bf16 activations."""
    e, n13 = w1.shape[0], w1.shape[1]
    k_out = w2.size(1)
    bm, bn = strix_blocks(hidden_states.size(0), topk_ids.size(1), e)
    act = _act(activation)

    def g13(c, si, ei, npp, k):
        S.moe_gemm_mxfp4(c, hidden_states, w1, s1, si, ei, npp, None, k, bm, bn, True, act)

    def g2(c, a, si, ei, npp, wts):
        S.moe_gemm_mxfp4(c, a, w2, s2, si, ei, npp, wts, 1, bm, bn, False, "silu")

    return _chain(output, hidden_states, topk_weights, topk_ids, e, n13, k_out, bm, apply_router_weight_on_input,
                  workspace13, workspace2, g13, g2)


# ---------------------------------------------------------------- eligibility
_FUSED = ("silu", "gelu_tanh")


def fp8_scales_ok(w: torch.Tensor, s: torch.Tensor | None, block_shape) -> bool:
    """fp32 block scales [E, N/128, K/128] (block_shape [128, 128]) or one
    scale per (expert, row) (python/strix_vllm/moe.py:856-867)."""
    if s is None:
        return False
    e, n, k = w.shape
    if block_shape is not None:
        return list(block_shape) == [128, 128] and n % 128 == 0 and k % 128 == 0 and tuple(s.shape) == (
            e, n // 128, k // 128)
    return s.numel() == e * n


def fp8_bad(hidden_states, w1, w2, s1, s2, block_shape, activation, expert_map, a1q_scale=None,
            has_bias=False, has_lora=False) -> list[str]:
    """Names of the failed FP8-chain checks ([] = eligible), python/strix_vllm/moe.py:869-903."""
    checks = {
        "2d": hidden_states.dim() == 2,
        "act": hidden_states.dtype in (torch.bfloat16, torch.float16) and a1q_scale is None,
        "w1_fp8": w1.dtype == torch.float8_e4m3fn,
        "w2_fp8": w2.dtype == torch.float8_e4m3fn,
        "scales": fp8_scales_ok(w1, s1, block_shape) and fp8_scales_ok(w2, s2, block_shape),
        "bias": not has_bias,
        "lora": not has_lora,
        "expert_map": expert_map is None,
        "activation": _act(activation) in _FUSED,
        "w13_row": w1.size(2) % (128 if block_shape else 64) == 0,
        "w2_row": w2.size(2) % (128 if block_shape else 64) == 0,
        "n64": w1.size(1) % 64 == 0 and w2.size(1) % 64 == 0,
        "aligned": w1.stride(1) % 16 == 0 and w2.stride(1) % 16 == 0,
    }
    return [name for name, ok in checks.items() if not ok]


def zp_layout_ok(w: torch.Tensor, z: torch.Tensor | None, group: int | None) -> bool:
    """vLLM's int4 MoE zero points: uint8 [E, N/2, K/group], two uint4 per
    byte along N (even n in the low nibble), for weights uint8 [E, N, K/2]
    (moe_gemm_w4a16_zp reads exactly this)."""
    if z is None or not group:
        return False
    e, n, k2 = w.shape
    return (z.dtype == torch.uint8 and z.dim() == 3 and n % 2 == 0 and (2 * k2) % group == 0
            and tuple(z.shape) == (e, n // 2, 2 * k2 // group) and (z.size(2) == 1 or z.stride(2) == 1))


def wna16_bad(hidden_states, w1, w2, s1, s2, group, activation, expert_map, a1q_scale=None, a2_scale=None,
              has_zp=False, has_bias=False, has_lora=False, z1=None, z2=None) -> list[str]:
    """Names of the failed int4-chain checks (python/strix_vllm/moe.py:360-409).
    Unlike the reference (which rejects zero points, python/strix_vllm/moe.py:
    376), asymmetric experts pass when both zero-point tensors have vLLM's
    packed layout (`zp_layout_ok`); they then run moe_gemm_w4a16_zp."""
    scale_dtypes = (torch.bfloat16, torch.float16, torch.float32)
    zp_scale_dtypes = (torch.bfloat16, torch.float16)
    checks = {
        "2d": hidden_states.dim() == 2,
        "act_dtype": hidden_states.dtype == torch.bfloat16,
        "w1_uint8": w1.dtype == torch.uint8,
        "w2_uint8": w2.dtype == torch.uint8,
        "act_scales": a1q_scale is None and a2_scale is None,
        "zero_point": not has_zp or (zp_layout_ok(w1, z1, group) and zp_layout_ok(w2, z2, group)
                                     and s1 is not None and s2 is not None
                                     and s1.dtype in zp_scale_dtypes and s2.dtype in zp_scale_dtypes),
        "group": group in (32, 64, 128),
        "scales": s1 is not None and s2 is not None and s1.dtype in scale_dtypes and s2.dtype in scale_dtypes,
        "bias": not has_bias,
        "lora": not has_lora,
        "expert_map": expert_map is None,
        "activation": _act(activation) in _FUSED,
        "w13_row": w1.size(2) % 8 == 0,
        "w2_row": w2.size(2) % 8 == 0,
    }
    return [name for name, ok in checks.items() if not ok]


def mxfp4_bad(hidden_states, w1, w2, s1, s2, activation, expert_map, a1q_scale=None, has_bias=False,
              has_lora=False) -> list[str]:
    """Names of the failed MXFP4-chain checks ([] = eligible): e2m1 experts
    uint8 [E, N, K/2] with e8m0 uint8 [E, N, K/32], bf16 activations, a
    fused gate activation, no biases (the reference has no MXFP4 MoE chain)."""
    def scales_ok(w, s):
        return (s is not None and s.dtype == torch.uint8 and s.dim() == 3
                and tuple(s.shape) == (w.size(0), w.size(1), 2 * w.size(2) // 32) and (s.size(2) == 1 or s.stride(2) == 1))

    checks = {
        "2d": hidden_states.dim() == 2,
        "act_dtype": hidden_states.dtype == torch.bfloat16 and a1q_scale is None,
        "w1_uint8": w1.dtype == torch.uint8 and w1.dim() == 3,
        "w2_uint8": w2.dtype == torch.uint8 and w2.dim() == 3,
        "scales": w1.dim() == 3 and w2.dim() == 3 and scales_ok(w1, s1) and scales_ok(w2, s2),
        "bias": not has_bias,
        "lora": not has_lora,
        "expert_map": expert_map is None,
        "activation": _act(activation) in _FUSED,
        "k32": w1.dim() == 3 and w2.dim() == 3 and (2 * w1.size(2)) % 64 == 0 and (2 * w2.size(2)) % 64 == 0,
        "n16": w1.dim() == 3 and w2.dim() == 3 and w1.size(1) % 32 == 0 and w2.size(1) % 16 == 0,
        "aligned": w1.dim() == 3 and w2.dim() == 3 and w1.stride(1) % 16 == 0 and w2.stride(1) % 16 == 0,
    }
    return [name for name, ok in checks.items() if not ok]


def bf16_ok(hidden_states, w1, w2, activation, expert_map, quantized=False, has_bias=False, has_lora=False) -> bool:
    """The unquantized chain's gate (python/strix_vllm/moe.py:196-227)."""
    return (hidden_states.dim() == 2 and hidden_states.dtype == torch.bfloat16 and w1.dtype == torch.bfloat16
            and w2.dtype == torch.bfloat16 and not quantized and not has_bias and not has_lora and expert_map is None
            and _act(activation) in _FUSED and w1.size(2) % 64 == 0 and w2.size(2) % 64 == 0
            and w1.size(1) % 128 == 0 and w2.size(1) % 64 == 0)


# ---------------------------------------------------------------- vLLM hooks
_APPLY_ARGS = ("output", "hidden_states", "w1", "w2", "topk_weights", "topk_ids", "activation", "global_num_experts",
               "expert_map", "a1q_scale", "a2_scale", "workspace13", "workspace2", "expert_tokens_meta",
               "apply_router_weight_on_input")


def _lora(experts) -> bool:
    return getattr(experts, "_lora_context", None) is not None


def _make_experts_cls():
    from vllm.model_executor.layers.fused_moe.experts.triton_moe import TritonExperts

    class StrixTritonExperts(TritonExperts):
        def apply(self, *args, **kwargs):
            a = dict(zip(_APPLY_ARGS, args), **kwargs)
            qc = self.quant_config
            quantized = bool(qc.use_fp8_w8a8 or qc.use_int8_w8a8 or qc.use_int8_w8a16 or qc.use_int4_w4a16)
            t = a["hidden_states"].size(0)
            if not (bf16_ok(a["hidden_states"], a["w1"], a["w2"], a["activation"], a["expert_map"], quantized,
                            self.w1_bias is not None or self.w2_bias is not None, _lora(self))
                    and not self.expects_unquantized_inputs
                    and strix_moe_ok(t, a["w1"].size(1), a["w1"].size(2))
                    and strix_moe_ok(t * a["topk_ids"].size(1), a["w2"].size(1), a["w2"].size(2))):
                return super().apply(**a)
            bf16_experts(a["output"], a["hidden_states"], a["w1"], a["w2"], a["topk_weights"], a["topk_ids"],
                         a["activation"], a["apply_router_weight_on_input"], a["workspace13"], a["workspace2"])

    return StrixTritonExperts


def _make_wna16_experts_cls():
    from vllm.model_executor.layers.fused_moe.experts.triton_moe import TritonWNA16Experts

    class StrixTritonWNA16Experts(TritonWNA16Experts):
        def __init__(self, *args, **kwargs):
            super().__init__(*args, **kwargs)
            self._strix_w4a8 = model_gate("moe_w4a8")

        def apply(self, *args, **kwargs):
            a = dict(zip(_APPLY_ARGS, args), **kwargs)
            bs = self.block_shape
            group = None if not bs or len(bs) < 2 else int(bs[1])
            z1, z2 = self.w1_zp, self.w2_zp
            has_zp = z1 is not None or z2 is not None
            bad = wna16_bad(a["hidden_states"], a["w1"], a["w2"], self.w1_scale, self.w2_scale, group,
                            a["activation"], a["expert_map"], a["a1q_scale"], a["a2_scale"], has_zp,
                            self.w1_bias is not None or self.w2_bias is not None, _lora(self), z1, z2)
            if bad:
                from vllm.logger import init_logger

                init_logger("vllm.strix").warning_once("moe_w4a16 falls back to Triton: " + ", ".join(bad))
                return super().apply(**a)
            w1, w2 = a["w1"], a["w2"]
            t = a["hidden_states"].size(0)
            w4a8 = not has_zp and self._strix_w4a8 and _w4a8_ok(t, group, w1.size(1), w2.size(1))
            wna16_experts(a["output"], a["hidden_states"], w1, w2, self.w1_scale, self.w2_scale, a["topk_weights"],
                          a["topk_ids"], group, a["activation"], a["apply_router_weight_on_input"],
                          a["workspace13"], a["workspace2"], z1=z1 if has_zp else None,
                          z2=z2 if has_zp else None, w4a8=w4a8)

    return StrixTritonWNA16Experts


def _make_fp8_experts_cls(w8a8: bool = True):
    from vllm.model_executor.layers.fused_moe.experts.triton_moe import TritonExperts

    class StrixFp8Experts(TritonExperts):
        @property
        def expects_unquantized_inputs(self) -> bool:
            # The chain quantizes the activations itself (e4m3, 1x128 groups).
            return True

        def _scales(self, w, s):
            if self.block_shape is not None:
                return s.to(torch.float32).contiguous()
            return s.reshape(w.size(0), w.size(1)).contiguous()

        def apply(self, *args, **kwargs):
            a = dict(zip(_APPLY_ARGS, args), **kwargs)
            bad = fp8_bad(a["hidden_states"], a["w1"], a["w2"], self.w1_scale, self.w2_scale, self.block_shape,
                          a["activation"], a["expert_map"], a["a1q_scale"],
                          self.w1_bias is not None or self.w2_bias is not None, _lora(self))
            if bad or not self.quant_config.use_fp8_w8a8:
                from vllm.logger import init_logger

                init_logger("vllm.strix").warning_once("moe_fp8 falls back to Triton: " + ", ".join(bad))
                return super().apply(**a)
            w1, w2 = a["w1"], a["w2"]
            fp8_experts(a["output"], a["hidden_states"], w1, w2, self._scales(w1, self.w1_scale),
                        self._scales(w2, self.w2_scale), a["topk_weights"], a["topk_ids"], a["activation"],
                        a["apply_router_weight_on_input"], a["workspace13"], a["workspace2"], w8a8=w8a8)

    return StrixFp8Experts


def _make_int8_experts_cls():
    from vllm.model_executor.layers.fused_moe.experts.triton_moe import TritonExperts

    class StrixInt8Experts(TritonExperts):
        @property
        def expects_unquantized_inputs(self) -> bool:
            return True

        def apply(self, *args, **kwargs):
            a = dict(zip(_APPLY_ARGS, args), **kwargs)
            w1, w2 = a["w1"], a["w2"]
            ok = (a["hidden_states"].dtype == torch.bfloat16 and w1.dtype == torch.int8 and w2.dtype == torch.int8
                  and a["expert_map"] is None and _act(a["activation"]) in _FUSED and self.w1_scale is not None
                  and self.w2_scale is not None and self.w1_bias is None and self.w2_bias is None)
            if not ok:
                return super().apply(**a)
            int8_experts(a["output"], a["hidden_states"], w1, w2, self.w1_scale.reshape(w1.size(0), -1),
                         self.w2_scale.reshape(w2.size(0), -1), a["topk_weights"], a["topk_ids"], a["activation"],
                         a["apply_router_weight_on_input"], a["workspace13"], a["workspace2"])

    return StrixInt8Experts


def _make_mxfp4_experts_cls():
    from vllm.model_executor.layers.fused_moe.experts.triton_moe import TritonExperts

    class StrixMxfp4Experts(TritonExperts):
        """MXFP4 experts (e2m1 + e8m0 per 32 K) on moe_gemm_mxfp4: weights
        decoded to bf16 in LDS or registers, bf16 MFMA, bf16 activations."""

        @property
        def expects_unquantized_inputs(self) -> bool:
            return True

        def apply(self, *args, **kwargs):
            a = dict(zip(_APPLY_ARGS, args), **kwargs)
            bad = mxfp4_bad(a["hidden_states"], a["w1"], a["w2"], self.w1_scale, self.w2_scale, a["activation"],
                            a["expert_map"], a["a1q_scale"],
                            self.w1_bias is not None or self.w2_bias is not None, _lora(self))
            if bad:
                from vllm.logger import init_logger

                init_logger("vllm.strix").warning_once("moe_mxfp4 falls back: " + ", ".join(bad))
                return super().apply(**a)
            mxfp4_experts(a["output"], a["hidden_states"], a["w1"], a["w2"], self.w1_scale, self.w2_scale,
                          a["topk_weights"], a["topk_ids"], a["activation"], a["apply_router_weight_on_input"],
                          a["workspace13"], a["workspace2"])

    return StrixMxfp4Experts


def _hook_backend(oracle_mod, enum_name: str, cls) -> bool:
    """Route an oracle module's Triton backend to `cls` (the FP8 / int8 /
    MXFP4 oracles of vLLM pick experts classes through
    `backend_to_kernel_cls(backend)`). False when the module has no such
    selector or enum member (another vLLM version): the hook is skipped."""
    enum = getattr(oracle_mod, enum_name, None)
    orig = getattr(oracle_mod, "backend_to_kernel_cls", None)
    triton = getattr(enum, "TRITON", None) if enum is not None else None
    if orig is None or triton is None:
        return False

    def _backend_to_kernel_cls(backend, _orig=orig, _cls=cls, _triton=triton):
        if backend == _triton:
            return [_cls]
        return _orig(backend)

    oracle_mod.backend_to_kernel_cls = _backend_to_kernel_cls
    return True


def register() -> None:
    """Hook vLLM's MoE selection (python/strix_vllm/moe.py:1019-1108): the
    unquantized method's experts class, the WNA16 oracle's module global and
    the FP8 / int8 oracles' backend selectors."""
    from vllm.model_executor.layers.fused_moe.experts.triton_moe import TritonExperts
    from vllm.model_executor.layers.fused_moe.unquantized_fused_moe_method import UnquantizedFusedMoEMethod

    if not disabled("moe_gemm"):
        experts_cls = _make_experts_cls()

        @UnquantizedFusedMoEMethod.register_oot
        class StrixUnquantizedFusedMoEMethod(UnquantizedFusedMoEMethod):
            def __init__(self, moe):
                super().__init__(moe)
                if self.experts_cls is TritonExperts:
                    self.experts_cls = experts_cls

    if not disabled("moe_w4a16"):
        from vllm.model_executor.layers.fused_moe.oracle import int_wna16

        cls = _make_wna16_experts_cls()
        int_wna16.TritonWNA16Experts = cls
        assert int_wna16.TritonWNA16Experts is cls

    if not disabled("moe_fp8"):
        from vllm.model_executor.layers.fused_moe.oracle import fp8 as fp8_oracle

        _hook_backend(fp8_oracle, "Fp8MoeBackend", _make_fp8_experts_cls(w8a8=not disabled("moe_fp8_w8a8")))

    if os.environ.get("STRIX_MOE_W8A16") and not disabled("moe_w8a16"):
        from vllm.model_executor.layers.fused_moe.oracle import int8 as int8_oracle

        _hook_backend(int8_oracle, "Int8MoeBackend", _make_int8_experts_cls())

    if not disabled("moe_mxfp4"):
        try:
            from vllm.model_executor.layers.fused_moe.oracle import mxfp4 as mxfp4_oracle
        except ImportError:
            mxfp4_oracle = None
        if mxfp4_oracle is None or not _hook_backend(mxfp4_oracle, "Mxfp4MoeBackend", _make_mxfp4_experts_cls()):
            from vllm.logger import init_logger

            init_logger("vllm.strix").info("moe_mxfp4: this vLLM has no MXFP4 MoE backend selector; not hooked")
