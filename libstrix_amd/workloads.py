# SPDX-License-Identifier: MIT
"""Seeded synthetic inputs of the five configurations, in the kernels' layouts.

Everything is generated on the CPU with torch.Generator (so results never
depend on the device RNG) and moved to `device`. The weight quantizers here
are load-time transforms (what a checkpoint loader does once), not part of
the per-call hot path.

  C1  INT8 W8A8 dense:   x [M, K] ~N(0,1) bf16, W [N, K] ~N(0,0.02) -> per-channel int8
  C2  FP8-block dense:   W [N, K] ~N(0,0.02) -> e4m3 + 128x128 fp32 scales, x bf16 [M, K]
  C3  FP8-block MoE:     E=128 top-8 H=2048 I=768, w13 [E, 2I, H], w2 [E, H, I]
  C4  MXFP4 MoE:         E=32 top-4 H=I=2880, e2m1 codes uniform, e8m0 in 2^-8..2^-4
  C5  WNA16 int4+zp MoE: E=128 top-8 H=2048 I=768, g128, uint4 zero points
"""

from __future__ import annotations

import torch


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def quantize_int8_per_channel(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric per-output-channel int8: s = max|w_n|/127, q = round(w/s)."""
    amax = w.abs().amax(dim=1)
    s = torch.where(amax > 0, amax / 127.0, torch.ones_like(amax))
    q = torch.clamp(torch.round(w / s[:, None]), -127, 127).to(torch.int8)
    return q, s.float()


def quantize_fp8_block(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """e4m3fn with one fp32 scale per 128x128 block (amax/448) over the last
    two dims; N may be ragged (the last block row is partial)."""
    *lead, n, k = w.shape
    nb = (n + 127) // 128
    pad = nb * 128 - n
    wp = torch.nn.functional.pad(w, (0, 0, 0, pad)) if pad else w
    blocks = wp.reshape(*lead, nb, 128, k // 128, 128)
    amax = blocks.abs().amax(dim=(-3, -1))
    s = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = (blocks / s[..., :, None, :, None]).to(torch.float8_e4m3fn)
    q = q.reshape(*lead, nb * 128, k)[..., :n, :]
    return q.contiguous(), s.float().contiguous()


def _route_logits(g: torch.Generator, t: int, e: int) -> torch.Tensor:
    return torch.randn(t, e, generator=g)


def c1_int8(seed: int = 1, m: int = 32, k: int = 5120, n: int = 5120, device="cpu") -> dict:
    g = _gen(seed)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = torch.randn(n, k, generator=g) * 0.02
    wq, ws = quantize_int8_per_channel(w)
    return {"x": x.to(device), "w": wq.to(device), "sw": ws.to(device)}


def c2_fp8(seed: int = 2, m: int = 4096, n: int = 17408, k: int = 5120, device="cpu", weights=None) -> dict:
    g = _gen(seed)
    if weights is None:
        w = torch.randn(n, k, generator=g) * 0.02
        wq, ws = quantize_fp8_block(w)
        del w
    else:
        wq, ws = weights
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    return {"x": x.to(device), "w": wq.to(device), "sw": ws.to(device)}


def c3_fp8_moe(seed: int = 3, t: int = 64, e: int = 128, top_k: int = 8, h: int = 2048, inter: int = 768,
               device="cpu") -> dict:
    g = _gen(seed)
    w13q, w13s = quantize_fp8_block(torch.randn(e, 2 * inter, h, generator=g) * 0.02)
    w2q, w2s = quantize_fp8_block(torch.randn(e, h, inter, generator=g) * 0.02)
    logits = _route_logits(g, t, e)
    x = torch.randn(t, h, generator=g).to(torch.bfloat16)
    d = {"x": x, "logits": logits, "w13": w13q, "w13_s": w13s, "w2": w2q, "w2_s": w2s, "top_k": top_k}
    return {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in d.items()}


def _mxfp4_weights(g: torch.Generator, e: int, n: int, k: int):
    w = torch.randint(0, 256, (e, n, k // 2), generator=g, dtype=torch.uint8)
    s = torch.randint(119, 124, (e, n, k // 32), generator=g, dtype=torch.uint8)
    return w, s


def c4_mxfp4_moe(seed: int = 4, t: int = 2048, e: int = 32, top_k: int = 4, h: int = 2880, inter: int = 2880,
                 device="cpu") -> dict:
    g = _gen(seed)
    w13, w13_s = _mxfp4_weights(g, e, 2 * inter, h)
    w2, w2_s = _mxfp4_weights(g, e, h, inter)
    logits = _route_logits(g, t, e)
    x = torch.randn(t, h, generator=g).to(torch.bfloat16)
    d = {"x": x, "logits": logits, "w13": w13, "w13_s": w13_s, "w2": w2, "w2_s": w2_s, "top_k": top_k}
    return {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in d.items()}


def pack_int4_k(q: torch.Tensor) -> torch.Tensor:
    """uint4 values [.., N, K] -> int32 [.., N, K/8], nibble j of word w = k 8w+j."""
    *lead, n, k = q.shape
    q = q.to(torch.int64).reshape(*lead, n, k // 8, 8)
    word = torch.zeros(*lead, n, k // 8, dtype=torch.int64)
    for j in range(8):
        word |= q[..., j] << (4 * j)
    word = torch.where(word >= 2**31, word - 2**32, word)
    return word.to(torch.int32)


def pack_zeros_n(z: torch.Tensor) -> torch.Tensor:
    """uint4 zero points [.., N, G] -> uint8 [.., N/2, G], even n in the low nibble."""
    return (z[..., 0::2, :] | (z[..., 1::2, :] << 4)).to(torch.uint8)


def _wna16_weights(g: torch.Generator, e: int, n: int, k: int, group: int):
    q = torch.randint(0, 16, (e, n, k), generator=g, dtype=torch.uint8)
    s = (torch.rand(e, n, k // group, generator=g) * 0.015 + 0.005).to(torch.bfloat16)
    z = torch.randint(0, 16, (e, n, k // group), generator=g, dtype=torch.uint8)
    return pack_int4_k(q), s, pack_zeros_n(z)


def c5_wna16_moe(seed: int = 5, t: int = 8192, e: int = 128, top_k: int = 8, h: int = 2048, inter: int = 768,
                 group: int = 128, device="cpu") -> dict:
    g = _gen(seed)
    w13, w13_s, w13_z = _wna16_weights(g, e, 2 * inter, h, group)
    w2, w2_s, w2_z = _wna16_weights(g, e, h, inter, group)
    logits = _route_logits(g, t, e)
    x = torch.randn(t, h, generator=g).to(torch.bfloat16)
    d = {"x": x, "logits": logits, "w13": w13, "w13_s": w13_s, "w13_z": w13_z, "w2": w2, "w2_s": w2_s,
         "w2_z": w2_z, "top_k": top_k, "group": group}
    return {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in d.items()}
