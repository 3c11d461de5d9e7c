# SPDX-License-Identifier: MIT
"""W8A16 (compressed-tensors uint8b128) and W4A16 (uint4b8) linears on gfx950.

W8A16 follows the reference (python/strix_vllm/linear.py:74-93): weights
stored once as uint8 [N, K] (raw byte - 128 is the signed value); decode rows
run `w8a16_skinny_gemm` (bf16 activations, exact weights), larger M runs
`w8a8_wmma_gemm` (activations quantized per 128-element group inside the op,
int8 MFMA) with the scales as fp32 [N] or [G, N], transposed once per weight
and cached.

W4A16 takes the RDNAHybridW4A16 packed int4 words (python/strix_vllm/linear.py:
100-137). The reference keeps decode on vLLM's own skinny int4 kernel and
runs prefill as W4A8 (int8 activations) or, for 32-element groups, a bf16
dequant tile. Here every M stays W4A16 (bf16 activations, exact weights):
`w4a16_wmma_gemm` below DEQUANT_MIN_M rows, `w4a16_dequant` + hipBLASLt from
there (51 vs 126 us at M=128, 463 vs 658 us at M=8192, N=K=5120, MI355X);
W4A8 has no speed to offer on gfx950, where the bf16 path is the faster one.
"""

from __future__ import annotations

import weakref

import torch

from libstrix_amd.vllm_plugin import disabled
from libstrix_amd.vllm_plugin.mxfp4 import DEQUANT_MIN_M

# The op namespace the dispatchers call through (a test may substitute a recorder).
S = torch.ops.strix

MAX_SKINNY_BATCH_SIZE = 8
_W8A8_GROUP_SIZE = 128
# fp32 W8A8 scale copies keyed by weight identity (python/strix_vllm/linear.py:
# 27, 42-71); covers every quantized linear of a large model.
_W8A8_PREP_MAX_ENTRIES = 1024
_W8A8_PREP: dict[int, tuple[weakref.ref, torch.Tensor]] = {}


def pack_w8_rows(unpacked: torch.Tensor) -> torch.Tensor:
    """[N, K] integers holding 0..255 -> uint8 [N, K] (python/strix_vllm/linear.py:30-39)."""
    return (unpacked & 0xFF).to(torch.uint8).contiguous()


def w8a8_scales(w_q: torch.Tensor, w_s: torch.Tensor, group_size: int) -> torch.Tensor | None:
    """fp32 scales for the W8A8 op: [N] per channel, [G, N] for 128-element
    groups; None when the layout is one the op does not take. Cached per
    weight tensor (the weakref guards against a reused id)."""
    n, k = w_q.shape
    if group_size == 0:
        if w_s.numel() != n:
            return None
    elif group_size != _W8A8_GROUP_SIZE or tuple(w_s.shape) != (n, k // group_size):
        return None
    if k % _W8A8_GROUP_SIZE:
        return None
    entry = _W8A8_PREP.get(id(w_q))
    if entry is not None and entry[0]() is w_q:
        return entry[1]
    s = w_s.reshape(-1).float().contiguous() if group_size == 0 else w_s.float().t().contiguous()
    if len(_W8A8_PREP) >= _W8A8_PREP_MAX_ENTRIES:
        _W8A8_PREP.pop(next(iter(_W8A8_PREP)))
    _W8A8_PREP[id(w_q)] = (weakref.ref(w_q), s)
    return s


def _apply_impl(x_2d: torch.Tensor, w_q: torch.Tensor, w_s: torch.Tensor, bias: torch.Tensor | None,
                group_size: int) -> torch.Tensor:
    """W8A16 per forward. group_size 0 = per channel, else 32 or 128."""
    m = x_2d.size(0)
    x = x_2d.contiguous()
    if m <= MAX_SKINNY_BATCH_SIZE:
        s = w_s if w_s.dtype == x.dtype else w_s.to(x.dtype)
        out = S.w8a16_skinny_gemm(w_q, x, s, bias, 0, group_size)
    else:
        s = w8a8_scales(w_q, w_s, group_size)
        if s is None:
            raise RuntimeError(f"strix W8A16: W8A8 path cannot run N={w_q.size(0)} K={w_q.size(1)} "
                               f"group_size={group_size}")
        out = S.w8a8_wmma_gemm(w_q, x, s)
        out = out if bias is None else out + bias
    return out


def _apply_fake(x_2d, w_q, w_s, bias, group_size):
    return x_2d.new_empty((x_2d.size(0), w_q.size(0)))


def _w4_apply_impl(x_2d: torch.Tensor, w_q: torch.Tensor, w_s: torch.Tensor, bias: torch.Tensor | None,
                   group_size: int) -> torch.Tensor:
    """W4A16 per forward: int8 [N, K/2] RDNAHybridW4A16 words, bf16 scales
    [N, K/group] (group_size -1 = one group of K)."""
    m, k = x_2d.shape
    g = k if group_size in (-1, 0) else group_size
    x = x_2d if x_2d.dtype == torch.bfloat16 else x_2d.to(torch.bfloat16)
    s = w_s if w_s.dtype == torch.bfloat16 else w_s.to(torch.bfloat16)
    if s.dim() == 1:
        s = s.reshape(-1, 1)
    if m >= DEQUANT_MIN_M:
        out = torch.nn.functional.linear(x, S.w4a16_dequant(w_q, s, g))
        out = out if bias is None else out + bias
    else:
        out = S.w4a16_wmma_gemm(x.contiguous(), w_q, s, bias, g)
    return out if out.dtype == x_2d.dtype else out.to(x_2d.dtype)


def can_implement_w8(weight_type: str, zero_points: bool, act_type, group_size: int, k: int):
    """The W8A16 gate (python/strix_vllm/linear.py:165-180)."""
    if weight_type != "uint8b128":
        return False, "strix W8A16 takes symmetric uint8b128 weights"
    if zero_points:
        return False, "zero points not supported"
    if act_type not in (torch.float16, torch.bfloat16):
        return False, "needs fp16/bf16 activations"
    if group_size not in (-1, 32, 128):
        return False, f"group_size {group_size} not in (-1, 32, 128)"
    if k % 128:
        return False, f"K={k} must be a multiple of 128"
    return True, None


def can_implement_w4(weight_type: str, zero_points: bool, group_size: int, k: int):
    """The W4A16 gate (python/strix_vllm/linear.py:227-239)."""
    if weight_type != "uint4b8" or zero_points:
        return False, "strix W4A16 takes symmetric uint4b8 weights"
    if group_size not in (-1, 32, 64, 128):
        return False, f"group_size {group_size} not in (-1, 32, 64, 128)"
    if k % 128:
        return False, "K must be a multiple of 128"
    return True, None


def register() -> None:
    use_w8, use_w4 = not disabled("w8a16"), not disabled("w4a16")
    if not (use_w8 or use_w4):
        return
    import vllm.model_executor.kernels.linear as linear_kernels
    from vllm.model_executor.kernels.linear.mixed_precision.MPLinearKernel import MPLinearKernel, MPLinearLayerConfig
    from vllm.model_executor.layers.quantization.utils.quant_utils import unpack_quantized_values_into_int32
    from vllm.model_executor.parameter import permute_param_layout_
    from vllm.platforms import PlatformEnum
    from vllm.utils.torch_utils import direct_register_custom_op

    direct_register_custom_op(op_name="strix_w8a16_apply", op_func=_apply_impl, mutates_args=[],
                              fake_impl=_apply_fake)

    class StrixW8A16LinearKernel(MPLinearKernel):
        @classmethod
        def get_min_capability(cls) -> int:
            return 0

        @classmethod
        def can_implement(cls, c: MPLinearLayerConfig) -> tuple[bool, str | None]:
            return can_implement_w8(str(c.weight_type), bool(c.zero_points), c.act_type, c.group_size,
                                    c.partition_weight_shape[0])

        def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
            c = self.config
            w_q_raw = getattr(layer, self.w_q_name)
            w_s_raw = getattr(layer, self.w_s_name)
            unpacked = unpack_quantized_values_into_int32(w_q_raw.data, c.weight_type, packed_dim=w_q_raw.packed_dim)
            if getattr(w_q_raw, "output_dim", 0) != 0:
                unpacked = unpacked.t().contiguous()
            w_q = pack_w8_rows(unpacked)
            if w_s_raw.dim() == 2:
                permute_param_layout_(w_s_raw, input_dim=1, output_dim=0)
            w_s = w_s_raw.data.contiguous()
            self._transform_param(layer, self.w_q_name, lambda _: w_q)
            self._transform_param(layer, self.w_s_name, lambda _: w_s)

        def apply_weights(self, layer: torch.nn.Module, x: torch.Tensor, bias: torch.Tensor | None = None):
            w_q, w_s, _ = self._get_weight_params(layer)
            x_2d = x.reshape(-1, x.shape[-1])
            group_size = 0 if self.config.group_size == -1 else self.config.group_size
            out = torch.ops.vllm.strix_w8a16_apply(x_2d, w_q, w_s, bias, group_size)
            return out.reshape(*x.shape[:-1], w_q.size(0))

    direct_register_custom_op(op_name="strix_w4a16_apply", op_func=_w4_apply_impl, mutates_args=[],
                              fake_impl=_apply_fake)
    from vllm.model_executor.kernels.linear.mixed_precision.rdna_hybrid_w4a16 import RDNAHybridW4A16LinearKernel

    class StrixW4A16LinearKernel(RDNAHybridW4A16LinearKernel):
        """The RDNAHybridW4A16 packed weights, every M on gfx950 bf16 MFMA."""

        @classmethod
        def can_implement(cls, c: MPLinearLayerConfig) -> tuple[bool, str | None]:
            ok, why = super().can_implement(c)
            if not ok:
                return ok, why
            return can_implement_w4(str(c.weight_type), bool(c.zero_points), c.group_size,
                                    c.partition_weight_shape[0])

        def apply_weights(self, layer: torch.nn.Module, x: torch.Tensor, bias: torch.Tensor | None = None):
            w_q, w_s, _ = self._get_weight_params(layer)
            x_2d = x.reshape(-1, x.shape[-1])
            out = torch.ops.vllm.strix_w4a16_apply(x_2d, w_q, w_s, bias, self.config.group_size)
            return out.reshape(*x.shape[:-1], w_q.size(0))

    ours = [StrixW4A16LinearKernel] * use_w4 + [StrixW8A16LinearKernel] * use_w8
    for cls in ours:
        linear_kernels.register_linear_kernel(cls, PlatformEnum.ROCM, "mp")
    # Selection takes the first kernel that can implement a layer: ours go first.
    rocm = linear_kernels._POSSIBLE_KERNELS[PlatformEnum.ROCM]
    for cls in ours:
        rocm.insert(0, rocm.pop(rocm.index(cls)))
