# SPDX-License-Identifier: MIT
"""FP8 (float8_e4m3fn) linears on gfx950: 128x128 block-scaled and
per-output-channel checkpoints.

The reference (python/strix_vllm/fp8.py:1-262) targets a GPU without FP8
matrix instructions, so it keeps the activations in bf16 (W8A16: skinny
kernel for M <= 5, a decode-in-LDS tile below 768 rows, dequant + hipBLASLt
above) and turns vLLM's activation quantization off.

gfx950 has FP8 MFMA, so the block-scaled layer keeps vLLM's own W8A8
numerics: activations quantized per (row, 128-element group) to e4m3
(`fp8_quant_group128`, s = absmax / 448) and `fp8_w8a8_block_gemm_kmajor` (e4m3
MFMA, per-128-K block-scale fold in fp32) at every M; the GEMM's own dispatch
picks the streaming decode kernels for small M and the LDS-tiled ones above.
At load the weights are re-laid K-block-major (`weight8_kmajor`: each 128-K
block of all rows contiguous), which gives the same bits 9-12 % faster from
M=1 to M=1024 on N=17408 K=5120 (20.4 -> 18.2 us at M=1) and the same time at
M=4096. With STRIX_DISABLE=fp8_w8a8 the layer runs W8A16 instead (bf16
activations, row-major weights decoded exactly), as the reference does.

Per-channel checkpoints run W8A16: the e4m3 weights with one fp32 scale per
output channel against bf16 activations (`fp8_wmma_gemm`), or, from
W8A16_DEQUANT_MIN_M rows, `fp8_dequant` + hipBLASLt. Thresholds were measured
on MI355X (N=17408 K=5120 and N=5120 K=17408, bf16 out).
"""

from __future__ import annotations

import torch

from libstrix_amd.vllm_plugin import disabled

# The op namespace the dispatchers call through (a test may substitute a recorder).
S = torch.ops.strix

BLOCK = 128
# W8A16 (bf16 activations): the fused tile is a weight stream up to ~32 rows
# (23-38 us on 89 MB of e4m3 at M 1-8); from 64 rows decode-once + hipBLASLt
# wins (83 vs 102 us at M=64, 562 vs 1164 us at M=4096, N=17408 K=5120).
W8A16_DEQUANT_MIN_M = 64
# K granularity of the per-channel path (the scale is not blocked along K).
CHANNEL_K = 64
_W8A8 = [True]


def w8a16_uses_dequant(m: int) -> bool:
    return m >= W8A16_DEQUANT_MIN_M


def _apply_impl(x_2d: torch.Tensor, w: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None,
                w8a8: bool) -> torch.Tensor:
    """Per forward (python/strix_vllm/fp8.py:60-91). `scale` is fp32 block
    scales [ceil(N/128), K/128] or per-channel [N]."""
    m = x_2d.size(0)
    block = scale.dim() == 2
    if block and w8a8:
        q, s = S.fp8_quant_group128(x_2d.contiguous())
        if w.dim() == 3:  # K-block-major [K/128, N, 128]
            out = S.fp8_w8a8_block_gemm_kmajor(q, s, w, scale)
        else:
            out = S.fp8_w8a8_block_gemm(q, s, w, scale)
        if out.dtype != x_2d.dtype:
            out = out.to(x_2d.dtype)
    elif w8a16_uses_dequant(m):
        out = torch.nn.functional.linear(x_2d, S.fp8_dequant(w, scale).to(x_2d.dtype))
    else:
        out = S.fp8_wmma_gemm(w, x_2d.to(torch.bfloat16).contiguous(), scale)
        if out.dtype != x_2d.dtype:
            out = out.to(x_2d.dtype)
    return out if bias is None else out + bias


def out_features(w: torch.Tensor) -> int:
    """N of a row-major [N, K] or K-block-major [K/128, N, 128] weight."""
    return w.size(1) if w.dim() == 3 else w.size(0)


def _apply_fake(x_2d, w, scale, bias, w8a8):
    return x_2d.new_empty((x_2d.size(0), out_features(w)))


def can_implement_block(group_shape, out_dtype, k: int) -> tuple[bool, str | None]:
    """The block-scaled gate (python/strix_vllm/fp8.py:153-164)."""
    if tuple(group_shape) != (BLOCK, BLOCK):
        return False, "needs 128x128 weight blocks"
    if out_dtype not in (torch.bfloat16, torch.float16):
        return False, f"needs bf16/fp16 activations, got {out_dtype}"
    if k % BLOCK:
        return False, f"K={k} must be a multiple of 128"
    return True, None


def can_implement_channel(weight_dtype, per_channel: bool, out_dtype, k: int) -> tuple[bool, str | None]:
    """The per-channel gate (python/strix_vllm/fp8.py:210-220)."""
    if weight_dtype != torch.float8_e4m3fn:
        return False, f"needs float8_e4m3fn weights, got {weight_dtype}"
    if not per_channel:
        return False, "needs per-channel weight scales"
    if out_dtype not in (None, torch.bfloat16, torch.float16):
        return False, f"needs bf16/fp16 activations, got {out_dtype}"
    if k % CHANNEL_K:
        return False, f"K={k} must be a multiple of {CHANNEL_K}"
    return True, None


def prepare_block(w: torch.Tensor, block_scale: torch.Tensor, kmajor: bool = False
                  ) -> tuple[torch.Tensor, torch.Tensor]:
    """Load-time transform (python/strix_vllm/fp8.py:147-160): e4m3 [N, K] rows
    made contiguous in K, fp32 block scales; with `kmajor` (the W8A8 path) the
    weights are re-laid [K/128, N, 128] for fp8_w8a8_block_gemm_kmajor."""
    if w.dtype != torch.float8_e4m3fn:
        raise RuntimeError(f"strix FP8 takes float8_e4m3fn, got {w.dtype}")
    if w.stride(-1) != 1:
        w = w.contiguous()
    n, k = w.shape
    bs = block_scale.float().contiguous()
    if tuple(bs.shape) != ((n + BLOCK - 1) // BLOCK, k // BLOCK):
        raise RuntimeError(f"block scales must be [{(n + BLOCK - 1) // BLOCK}, {k // BLOCK}], got {list(bs.shape)}")
    if kmajor:
        w = S.weight8_kmajor(w)
    return w, bs


def prepare_channel(w: torch.Tensor, s: torch.Tensor, n: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-channel load transform (python/strix_vllm/fp8.py:222-241): the
    weight may arrive as a [K, N] view; rows are made [N, K], scales fp32 [N].

    The orientation is read from the strides, not the sizes, so square
    weights (N == K) are handled: a column-major view (stride(0) == 1) is the
    transpose of [N, K] rows. A row-major tensor is [N, K] when its first
    size is N, else a stored [K, N] matrix."""
    if w.dtype != torch.float8_e4m3fn:
        raise RuntimeError(f"strix FP8 takes float8_e4m3fn, got {w.dtype}")
    if w.dim() != 2:
        raise RuntimeError(f"strix FP8 per-channel weight must be 2-D, got {w.dim()}-D")
    col_major = w.stride(0) == 1 and w.stride(1) != 1 and w.size(0) > 1
    if col_major or w.size(0) != n:
        w = w.t()
    if w.size(0) != n:
        raise RuntimeError(f"per-channel weight {list(w.shape)} has no dimension of N={n} rows")
    w = w.contiguous()
    s = s.float().reshape(-1).contiguous()
    if s.numel() == 1:
        s = s.expand(n).contiguous()
    if s.numel() != n:
        raise RuntimeError(f"per-channel scale has {s.numel()} values for N={n}")
    return w, s


def register() -> None:
    if disabled("fp8"):
        return
    _W8A8[0] = not disabled("fp8_w8a8")
    import vllm.model_executor.kernels.linear as linear_kernels
    from vllm.model_executor.kernels.linear.scaled_mm.BlockScaledMMLinearKernel import Fp8BlockScaledMMLinearKernel
    from vllm.model_executor.kernels.linear.scaled_mm.ScaledMMLinearKernel import FP8ScaledMMLinearLayerConfig
    from vllm.model_executor.utils import replace_parameter
    from vllm.platforms import PlatformEnum
    from vllm.utils.torch_utils import direct_register_custom_op

    from libstrix_amd.vllm_plugin import on_gfx950

    direct_register_custom_op(op_name="strix_fp8_apply", op_func=_apply_impl, mutates_args=[],
                              fake_impl=_apply_fake)

    class StrixFp8BlockScaledMMKernel(Fp8BlockScaledMMLinearKernel):
        # The op quantizes the activations itself (e4m3, 1x128 groups).
        apply_input_quant = False

        @classmethod
        def is_supported(cls, compute_capability=None):
            if not on_gfx950():
                return False, "strix FP8 is built for gfx950"
            return True, None

        @classmethod
        def can_implement(cls, config: FP8ScaledMMLinearLayerConfig):
            ok, why = super().can_implement(config)
            if not ok:
                return ok, why
            return can_implement_block(config.weight_quant_key.scale.group_shape, config.out_dtype,
                                       config.weight_shape[-1])

        def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
            super().process_weights_after_loading(layer)
            params = self._get_layer_params(layer)
            self._w8a8 = _W8A8[0]
            w, bs = prepare_block(params.weight, params.block_scale, kmajor=self._w8a8)
            replace_parameter(layer, params.WEIGHT, w)
            replace_parameter(layer, params.block_scale_attr, bs)

        def apply_weights(self, layer, x, bias=None, **kwargs):
            params = self._get_layer_params(layer)
            w = params.weight
            x_2d = x.reshape(-1, x.shape[-1])
            out = torch.ops.vllm.strix_fp8_apply(x_2d, w, params.block_scale, bias, self._w8a8)
            return out.reshape(*x.shape[:-1], out_features(w))

        def apply_block_scaled_mm(self, A, B, As, Bs):
            raise NotImplementedError("strix FP8 overrides apply_weights")

    kernels = linear_kernels._POSSIBLE_FP8_BLOCK_KERNELS[PlatformEnum.ROCM]
    if StrixFp8BlockScaledMMKernel not in kernels:
        kernels.insert(0, StrixFp8BlockScaledMMKernel)

    if disabled("fp8_channel"):
        return
    from vllm.model_executor.kernels.linear.scaled_mm.ScaledMMLinearKernel import FP8ScaledMMLinearKernel
    from vllm.model_executor.layers.quantization.utils.quant_utils import GroupShape

    class StrixFp8ChannelMMKernel(FP8ScaledMMLinearKernel):
        """W8A16 for per-channel FP8 weights (bf16 activations in)."""

        @classmethod
        def is_supported(cls, compute_capability=None):
            if not on_gfx950():
                return False, "strix FP8 is built for gfx950"
            return True, None

        @classmethod
        def can_implement(cls, config: FP8ScaledMMLinearLayerConfig):
            wkey = config.weight_quant_key
            return can_implement_channel(wkey.dtype, tuple(wkey.scale.group_shape) == tuple(GroupShape.PER_CHANNEL),
                                         config.out_dtype, config.weight_shape[-1])

        def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
            w_name, s_name, _, _ = self.layer_param_names
            w, s = prepare_channel(getattr(layer, w_name), getattr(layer, s_name), self.config.weight_shape[0])
            replace_parameter(layer, w_name, w)
            replace_parameter(layer, s_name, s)

        def apply_weights(self, layer, x, bias=None, **kwargs):
            w_name, s_name, _, _ = self.layer_param_names
            w, s = getattr(layer, w_name), getattr(layer, s_name)
            x_2d = x.reshape(-1, x.shape[-1])
            out = torch.ops.vllm.strix_fp8_apply(x_2d, w, s, bias, False)
            return out.reshape(*x.shape[:-1], w.size(0))

        def apply_scaled_mm(self, **kwargs):
            raise NotImplementedError("strix FP8 overrides apply_weights")

    kernels = linear_kernels._POSSIBLE_FP8_KERNELS[PlatformEnum.ROCM]
    if StrixFp8ChannelMMKernel not in kernels:
        kernels.insert(0, StrixFp8ChannelMMKernel)
