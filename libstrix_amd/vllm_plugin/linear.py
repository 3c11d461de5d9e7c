# SPDX-License-Identifier: MIT
"""W8A16 (compressed-tensors uint8b128) and W4A16 (uint4b8) linears on gfx950.

W8A16 keeps the checkpoint's numerics (bf16/fp16 activations against exact
weights) for decode and, like the reference (python/strix_vllm/linear.py:
74-93), quantizes prefill activations per 128-element group onto the int8
MFMA path. Weights are stored once as uint8 [N, K] (byte - 128 is the signed
value). Everything the forward needs is prepared once at load by
`prepare_w8`:

- the raw scales in the checkpoint's [N] / [N, G] layout, read by the decode
  and group-32/64 paths;
- for per-channel and 128-group layers, an fp32 copy in the layout the W8A8
  op reads ([N], or [G, N]), kept on the layer beside the weight. Other
  group sizes have none and run W8A16 at every M on `w8a16_gemm`.

Per forward: up to MAX_SKINNY_BATCH_SIZE rows `w8a16_skinny_gemm`; above,
`w8a8_wmma_gemm` with the load-time fp32 scales, or `w8a16_gemm` when the
layer has none.

W4A16 takes the RDNAHybridW4A16 packed int4 words (python/strix_vllm/linear.py:
100-137). The reference keeps decode on vLLM's own skinny int4 kernel and
runs prefill as W4A8 (int8 activations) or, for 32-element groups, a bf16
dequant tile. Here every M stays W4A16 (bf16 activations, exact weights):
`w4a16_wmma_gemm` below DEQUANT_MIN_M rows, `w4a16_dequant` + hipBLASLt from
there (51 vs 126 us at M=128, 463 vs 658 us at M=8192, N=K=5120, MI355X).
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from libstrix_amd.vllm_plugin import disabled
from libstrix_amd.vllm_plugin.mxfp4 import DEQUANT_MIN_M

# The op namespace the dispatchers call through (a test may substitute a recorder).
S = torch.ops.strix

MAX_SKINNY_BATCH_SIZE = 8
W8A8_GROUP = 128  # the activation group of the W8A8 op; weight groups must match it (or be per channel)
# Attribute holding the load-time W8A8 scales on a vLLM layer.
W8A8_SCALE_ATTR = "strix_w8a8_scale"


class W8Weights(NamedTuple):
    """A W8A16 layer's tensors after loading."""

    w_q: torch.Tensor            # uint8 [N, K], byte - 128 = signed value
    w_s: torch.Tensor            # checkpoint scales: [N] per channel or [N, K/group]
    w8a8_s: torch.Tensor | None  # fp32 [N] or [K/128, N] for w8a8_wmma_gemm; None = W8A16 at every M
    group_size: int              # 0 = per channel


def pack_w8_rows(unpacked: torch.Tensor) -> torch.Tensor:
    """[N, K] integers holding 0..255 -> uint8 [N, K] (python/strix_vllm/linear.py:30-39)."""
    return (unpacked & 0xFF).to(torch.uint8).contiguous()


def w8a8_scale_layout(w_s: torch.Tensor, n: int, k: int, group_size: int) -> torch.Tensor | None:
    """The fp32 weight scales in the W8A8 op's layout: [N] per channel,
    [K/128, N] for 128-element groups; None for any other grouping (or a K
    the op cannot take)."""
    if k % W8A8_GROUP:
        return None
    if group_size == 0:
        return w_s.reshape(-1).float().contiguous() if w_s.numel() == n else None
    if group_size == W8A8_GROUP and tuple(w_s.shape) == (n, k // W8A8_GROUP):
        return w_s.float().t().contiguous()
    return None


def prepare_w8(w_q: torch.Tensor, w_s: torch.Tensor, group_size: int) -> W8Weights:
    """Load-time preparation of one W8A16 layer: uint8 rows [N, K] and its
    scales (group_size -1 or 0 = per channel)."""
    g = 0 if group_size in (-1, 0) else group_size
    n, k = w_q.shape
    if g:
        if tuple(w_s.shape) != (n, k // g):
            raise RuntimeError(f"strix W8A16: group scales must be [{n}, {k // g}], got {list(w_s.shape)}")
        w_s = w_s.contiguous()
    else:
        if w_s.numel() != n:
            raise RuntimeError(f"strix W8A16: per-channel scales must hold {n} values, got {w_s.numel()}")
        w_s = w_s.reshape(n).contiguous()
    return W8Weights(w_q, w_s, w8a8_scale_layout(w_s, n, k, g), g)


def _apply_impl(x_2d: torch.Tensor, w_q: torch.Tensor, w_s: torch.Tensor, w8a8_s: torch.Tensor | None,
                bias: torch.Tensor | None, group_size: int) -> torch.Tensor:
    """W8A16 per forward. group_size 0 = per channel, else 32, 64 or 128."""
    m = x_2d.size(0)
    x = x_2d.contiguous()
    s = w_s if w_s.dtype == x.dtype else w_s.to(x.dtype)
    if m <= MAX_SKINNY_BATCH_SIZE:
        return S.w8a16_skinny_gemm(w_q, x, s, bias, 0, group_size)
    if w8a8_s is None:
        return S.w8a16_gemm(w_q, x, s, bias, group_size)
    out = S.w8a8_wmma_gemm(w_q, x, w8a8_s)
    return out if bias is None else out + bias


def _apply_fake(x_2d, w_q, w_s, w8a8_s, bias, group_size):
    return x_2d.new_empty((x_2d.size(0), w_q.size(0)))


def _w4_apply_fake(x_2d, w_q, w_s, bias, group_size):
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
    if group_size not in (-1, 32, 64, 128):
        return False, f"group_size {group_size} not in (-1, 32, 64, 128)"
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
            ints = unpack_quantized_values_into_int32(w_q_raw.data, c.weight_type, packed_dim=w_q_raw.packed_dim)
            rows = pack_w8_rows(ints if getattr(w_q_raw, "output_dim", 0) == 0 else ints.t())
            if w_s_raw.dim() == 2:
                permute_param_layout_(w_s_raw, input_dim=1, output_dim=0)
            prep = prepare_w8(rows, w_s_raw.data, c.group_size)
            self._transform_param(layer, self.w_q_name, lambda _: prep.w_q)
            self._transform_param(layer, self.w_s_name, lambda _: prep.w_s)
            setattr(layer, W8A8_SCALE_ATTR, prep.w8a8_s)

        def apply_weights(self, layer: torch.nn.Module, x: torch.Tensor, bias: torch.Tensor | None = None):
            w_q, w_s, _ = self._get_weight_params(layer)
            x_2d = x.reshape(-1, x.shape[-1])
            group_size = 0 if self.config.group_size == -1 else self.config.group_size
            out = torch.ops.vllm.strix_w8a16_apply(x_2d, w_q, w_s, getattr(layer, W8A8_SCALE_ATTR), bias,
                                                   group_size)
            return out.reshape(*x.shape[:-1], w_q.size(0))

    direct_register_custom_op(op_name="strix_w4a16_apply", op_func=_w4_apply_impl, mutates_args=[],
                              fake_impl=_w4_apply_fake)
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
