# SPDX-License-Identifier: MIT
"""MXFP4 (e2m1 + e8m0) W4A16 linears on gfx950.

Quark MXFP4 checkpoints carry `weight` u8 [N, K/2] (two e2m1 values per byte,
low nibble first) and `weight_scale` u8 [N, K/32] (e8m0). As in the reference
(python/strix_vllm/mxfp4.py:1-168) the packed bytes and scales are used as
loaded and the activations stay bf16 (the checkpoint's dynamic fp4 activation
QDQ is skipped: W4A16 is strictly more accurate).

Dispatch by M, measured on MI355X (N=5760/2880/17408, K=2880/5120):
- M <= GEMV_MAX_M: `mxfp4_gemv` (weights decoded in registers);
- M < DEQUANT_MIN_M: `mxfp4_wmma_gemm` (e2m1 decoded into LDS, bf16 MFMA),
  a weight stream up to 32-64 rows;
- from DEQUANT_MIN_M rows: `mxfp4_dequant` once per forward and hipBLASLt on
  the exact bf16 matrix (41.6 vs 68.3 us at M=128, 330 vs 436 us at M=8192 on
  N=5760 K=2880; the reference's rule, python/strix_vllm/mxfp4.py:43-45,
  with its crossover re-measured: 1024 rows there, 128 here).
"""

from __future__ import annotations

import torch

from libstrix_amd.vllm_plugin import disabled

# The op namespace the dispatchers call through (a test may substitute a recorder).
S = torch.ops.strix

GEMV_MAX_M = 8
DEQUANT_MIN_M = 128


def use_dequant(m: int, k: int) -> bool:
    """Decode the 4-bit weight once and run hipBLASLt, or keep the fused path."""
    return m >= DEQUANT_MIN_M


def _apply_impl(x_2d: torch.Tensor, w_q: torch.Tensor, w_s: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    """Per forward (python/strix_vllm/mxfp4.py:48-68)."""
    m, k = x_2d.shape
    x = x_2d if x_2d.dtype == torch.bfloat16 else x_2d.to(torch.bfloat16)
    if m <= GEMV_MAX_M and bias is None and x.is_contiguous() and x.stride(0) % 8 == 0 and w_q.stride(0) % 16 == 0:
        out = S.mxfp4_gemv(x, w_q, w_s)
    elif use_dequant(m, k):
        out = torch.nn.functional.linear(x, S.mxfp4_dequant(w_q, w_s))
        if bias is not None:
            out = out + bias
    else:
        out = S.mxfp4_wmma_gemm(w_q, x.contiguous(), w_s, bias)
    return out if out.dtype == x_2d.dtype else out.to(x_2d.dtype)


def _apply_fake(x_2d, w_q, w_s, bias):
    return x_2d.new_empty((x_2d.size(0), w_q.size(0)))


def can_implement(weight_only_or_mx_dynamic: bool, model_dtype) -> tuple[bool, str | None]:
    """The reference's gate (python/strix_vllm/mxfp4.py:124-139)."""
    if not weight_only_or_mx_dynamic:
        return False, "strix MXFP4 is weight-only (bf16 activations)"
    if model_dtype is not None and model_dtype != torch.bfloat16:
        return False, f"needs bf16 activations, model dtype is {model_dtype}"
    return True, None


def check_weights(w: torch.Tensor, s: torch.Tensor) -> None:
    """Load-time checks (python/strix_vllm/mxfp4.py:141-157)."""
    k = w.size(1) * 2
    if k % 128:
        raise ValueError(f"strix MXFP4: K={k} must be a multiple of 128 (N={w.size(0)})")
    if s.dtype != torch.uint8 or tuple(s.shape) != (w.size(0), k // 32):
        raise ValueError(f"strix MXFP4: weight_scale must be uint8 [N, K/32], got {s.dtype} {list(s.shape)}")


def _model_dtype():
    from vllm.config import get_current_vllm_config_or_none

    config = get_current_vllm_config_or_none()
    return None if config is None else config.model_config.dtype


def register() -> None:
    if disabled("mxfp4"):
        return
    import vllm.model_executor.kernels.linear as linear_kernels
    from torch.nn.parameter import Parameter
    from vllm.model_executor.kernels.linear.mxfp4.base import MxFp4LinearKernel, MxFp4LinearLayerConfig
    from vllm.model_executor.layers.quantization.utils.quant_utils import kMxfp4Dynamic
    from vllm.platforms import PlatformEnum
    from vllm.utils.torch_utils import direct_register_custom_op

    from libstrix_amd.vllm_plugin import on_gfx950

    direct_register_custom_op(op_name="strix_mxfp4_apply", op_func=_apply_impl, mutates_args=[],
                              fake_impl=_apply_fake)

    class StrixMxfp4LinearKernel(MxFp4LinearKernel):
        @classmethod
        def is_supported(cls, compute_capability: int | None = None) -> tuple[bool, str | None]:
            if not on_gfx950():
                return False, "strix MXFP4 W4A16 is built for gfx950"
            return True, None

        @classmethod
        def can_implement(cls, config: MxFp4LinearLayerConfig) -> tuple[bool, str | None]:
            return can_implement(config.activation_quant_key in (None, kMxfp4Dynamic), _model_dtype())

        def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
            for name in ("weight", "weight_scale"):
                param = getattr(layer, name)
                if not param.is_contiguous():
                    param = param.contiguous()
                if not isinstance(param, Parameter):
                    setattr(layer, name, Parameter(param, requires_grad=False))
            check_weights(layer.weight, layer.weight_scale)

        def apply_weights(self, layer: torch.nn.Module, x: torch.Tensor, bias: torch.Tensor | None = None):
            w_q, w_s = layer.weight, layer.weight_scale
            x_2d = x.reshape(-1, x.shape[-1])
            out = torch.ops.vllm.strix_mxfp4_apply(x_2d, w_q, w_s, bias)
            return out.reshape(*x.shape[:-1], w_q.size(0))

    linear_kernels._POSSIBLE_MXFP4_KERNELS[PlatformEnum.ROCM].insert(0, StrixMxfp4LinearKernel)
