# SPDX-License-Identifier: MIT
"""W8A8 int8 linears (compressed-tensors int-quantized) on gfx950.

The reference's swap (python/strix_vllm/int8.py:1-102) puts its kernel first
among ROCm's int8 scaled-MM candidates and runs `strix::w8a8_wmma_gemm`, which
re-quantizes the activations per 128-element group inside the op and reads
the weights as excess-128 bytes (flipped in place at load).

Here the layer keeps vLLM's own numerics: dynamic symmetric per-token int8
activations (`int8_quant_per_token`) against the checkpoint's signed int8
weights [N, K] and per-channel fp32 scales (`w8a8_scaled_mm`, int8 MFMA with
an exact int32 accumulator). The weights are used as loaded: no flip, no copy.
A per-tensor weight scale is broadcast to one value per output channel at
load.
"""

from __future__ import annotations

import torch

from libstrix_amd.vllm_plugin import disabled

# The op namespace the dispatchers call through (a test may substitute a recorder).
S = torch.ops.strix

_registered = False


def _apply_impl(x_2d: torch.Tensor, w_q: torch.Tensor, w_s: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    """Per forward (python/strix_vllm/int8.py:22-29): quantize per token, int8 GEMM, bias."""
    q, s = S.int8_quant_per_token(x_2d.contiguous())
    out = S.w8a8_scaled_mm(q, s, w_q, w_s)
    if out.dtype != x_2d.dtype:
        out = out.to(x_2d.dtype)
    return out if bias is None else out + bias


def _apply_fake(x_2d, w_q, w_s, bias):
    return x_2d.new_empty((x_2d.size(0), w_q.size(0)))


def prepare_weights(w: torch.Tensor, s: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Load-time transform (python/strix_vllm/int8.py:54-67): int8 [N, K] rows
    as loaded (copied only when not contiguous in K), fp32 scales [N]."""
    if w.dtype == torch.uint8:
        raise RuntimeError("strix W8A8 takes signed int8 weights, got uint8")
    if w.dtype != torch.int8:
        raise RuntimeError(f"strix W8A8 takes int8 weights, got {w.dtype}")
    if w.stride(-1) != 1:
        w = w.contiguous()
    n = w.size(0)
    s = s.reshape(-1).float()
    if s.numel() == 1:
        s = s.expand(n)
    if s.numel() != n:
        raise RuntimeError(f"per-channel scale has {s.numel()} values for N={n}")
    return w, s.contiguous()


def can_implement(is_static_input_scheme: bool, input_symmetric: bool, act_dtype=torch.bfloat16):
    """(ok, reason), the reference's gate (python/strix_vllm/int8.py:44-52);
    per-tensor weight scales are taken too (broadcast at load)."""
    if is_static_input_scheme:
        return False, "strix W8A8 takes dynamic per-token activations"
    if not input_symmetric:
        return False, "strix W8A8 takes symmetric activations"
    if act_dtype not in (torch.bfloat16, torch.float16):
        return False, f"needs bf16/fp16 activations, got {act_dtype}"
    return True, None


def _kernel_class():
    from vllm.model_executor.kernels.linear.scaled_mm.triton import TritonInt8ScaledMMLinearKernel

    class StrixW8A8LinearKernel(TritonInt8ScaledMMLinearKernel):
        """vLLM's int8 scaled-MM contract on gfx950 int8 MFMA."""

        @classmethod
        def can_implement(cls, c) -> tuple[bool, str | None]:
            return can_implement(c.is_static_input_scheme, c.input_symmetric)

        def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
            w, s = prepare_weights(layer.weight.data, layer.weight_scale.data)
            layer.weight = torch.nn.Parameter(w, requires_grad=False)
            layer.weight_scale = torch.nn.Parameter(s, requires_grad=False)

        def apply_weights(self, layer: torch.nn.Module, x: torch.Tensor, bias: torch.Tensor | None = None):
            w_q, w_s = layer.weight, layer.weight_scale
            x_2d = x.reshape(-1, x.shape[-1])
            out = torch.ops.vllm.strix_w8a8_apply(x_2d, w_q, w_s, None if bias is None else bias.contiguous())
            return out.reshape(*x.shape[:-1], w_q.size(0))

    return StrixW8A8LinearKernel


def register() -> None:
    """Put the kernel at the front of ROCm's int8 candidates (idempotent)."""
    global _registered
    if _registered or disabled("w8a8"):
        return
    _registered = True
    from vllm.model_executor.kernels.linear import _POSSIBLE_INT8_KERNELS
    from vllm.platforms import PlatformEnum
    from vllm.utils.torch_utils import direct_register_custom_op

    direct_register_custom_op(op_name="strix_w8a8_apply", op_func=_apply_impl, mutates_args=[],
                              fake_impl=_apply_fake)
    _POSSIBLE_INT8_KERNELS.setdefault(PlatformEnum.ROCM, []).insert(0, _kernel_class())
