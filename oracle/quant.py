# SPDX-License-Identifier: MIT
"""Quantizers and weight decoders of the oracle (CPU). Test infrastructure only."""

from __future__ import annotations

import torch

# e2m1 magnitudes by 3-bit code (tests/test_mxfp4.py:15).
MX_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


def _f32(x: torch.Tensor) -> torch.Tensor:
    return x.detach().to("cpu", torch.float32)


def int8_quant_per_token(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-token symmetric int8: s = max|x|/127 (1 for a
    zero row), q = clamp(round_half_even(x / s), -127, 127). The per-group
    convention it restates: csrc/gemm/w8a8_wmma_gemm.hip:15-21 and
    tests/test_moe_w4a8.py:30-33, with the group widened to the whole row.
    Pinned by: tests/test_oracle_quant.py (error bound |x - q s| <= s/2,
    max |q| == 127 on each nonzero row, brute-force rounding on tiny rows)."""
    xf = _f32(x)
    amax = xf.abs().amax(dim=1)
    s = torch.where(amax > 0, amax / 127.0, torch.ones_like(amax))
    q = torch.clamp(torch.round(xf / s[:, None]), -127, 127).to(torch.int8)
    return q, s


def _group_scale(xf: torch.Tensor, qmax: float) -> torch.Tensor:
    m, k = xf.shape
    g = xf.reshape(m, k // 128, 128).abs().amax(dim=2)
    return torch.where(g > 0, g / qmax, torch.ones_like(g))


def int8_quant_group128(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """int8 per (row, 128-group): tests/test_moe_w4a8.py:29-33 (s = amax/127,
    1 for an all-zero group, q = clamp(round(x/s), -127, 127)).
    Pinned by: tests/test_oracle_quant.py (group independence, error bound)."""
    xf = _f32(x)
    m, k = xf.shape
    s = _group_scale(xf, 127.0)
    q = torch.clamp(torch.round(xf.reshape(m, k // 128, 128) / s[..., None]), -127, 127)
    return q.reshape(m, k).to(torch.int8), s


def fp8_quant_group128(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """e4m3fn per (row, 1x128 group) (BASELINE config 2/3): s = amax/448 (1
    for an all-zero group), q = e4m3_rne(x / s), via torch's own
    float8_e4m3fn cast. vLLM's per-token-group FP8 quant, which the
    reference's FP8 path disables (python/strix_vllm/fp8.py:122-124).
    Pinned by: tests/test_oracle_quant.py (torch's cast against an
    independent nearest-even encoder over all 256 codes)."""
    xf = _f32(x)
    m, k = xf.shape
    s = _group_scale(xf, 448.0)
    q = (xf.reshape(m, k // 128, 128) / s[..., None]).to(torch.float8_e4m3fn)
    return q.reshape(m, k), s


def e4m3_decode(w: torch.Tensor) -> torch.Tensor:
    """e4m3fn bytes -> fp32 exactly (tests/test_fp8.py:43-54 pins every
    finite code against the float reference). Pinned by:
    tests/test_oracle_quant.py (all 256 codes against the sign/exponent/
    mantissa formula and tests/golden/kat.json)."""
    if w.dtype != torch.float8_e4m3fn:
        w = w.view(torch.float8_e4m3fn)
    return w.detach().to("cpu").float()


def mxfp4_decode(w_u8: torch.Tensor, s_u8: torch.Tensor) -> torch.Tensor:
    """MXFP4 [N, K/2] packed e2m1 (low nibble = even k) + e8m0 [N, K/32]
    -> fp32 [N, K] (tests/test_mxfp4.py:28-45, zero block for an e8m0 byte of
    0: tests/test_mxfp4.py:75-95, 114-127). Leading dims are batched.
    Pinned by: tests/test_oracle_quant.py (known answers, nibble order,
    zero block) and tests/golden/kat.json."""
    w = w_u8.detach().to("cpu").to(torch.int32)
    lut = torch.tensor(MX_VALUES, dtype=torch.float32)

    def value(nib):
        v = lut[(nib & 7).long()]
        return torch.where((nib & 8) != 0, -v, v)

    even = value(w & 15)
    odd = value((w >> 4) & 15)
    out = torch.stack([even, odd], dim=-1).reshape(*w.shape[:-1], w.shape[-1] * 2)
    e = s_u8.detach().to("cpu").to(torch.float32)
    scale = torch.where(e > 0, torch.pow(2.0, e - 127.0), torch.zeros_like(e))
    return out * scale.repeat_interleave(32, dim=-1)


def wna16_sym_decode(w_u8: torch.Tensor, scales: torch.Tensor, group: int) -> torch.Tensor:
    """vLLM Triton WNA16 uint8 [.., N, K/2] (low nibble = even k), symmetric
    (q - 8) * s per group (tests/test_moe_wna16.py:46-61). Pinned by:
    tests/test_oracle_quant.py (nibble order and brute-force decode)."""
    w = w_u8.detach().to("cpu").to(torch.int32)
    q = torch.stack([(w & 15), (w >> 4) & 15], dim=-1).reshape(*w.shape[:-1], w.shape[-1] * 2).float()
    return (q - 8.0) * scales.detach().to("cpu").float().repeat_interleave(group, dim=-1)


def wna16_zp_decode(qweight: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, group: int) -> torch.Tensor:
    """WNA16 with zero points (AWQ-style): qweight int32
    [.., N, K/8] with k = 8w + j in nibble j (little-endian, byte-identical to
    the reference's uint8 [.., N, K/2] low-nibble-first layout,
    csrc/moe/moe_gemm_w4a16.hip:7-10), scales [.., N, K/G], zeros uint8
    [.., N/2, K/G] with n even in the low nibble (vLLM's fused_moe zp layout);
    w = (q - z) * s. Pinned by: tests/test_oracle_quant.py (brute-force
    per-element decode on tiny shapes)."""
    qw = qweight.detach().to("cpu").to(torch.int64) & 0xFFFFFFFF
    nib = torch.stack([(qw >> (4 * j)) & 15 for j in range(8)], dim=-1)
    q = nib.reshape(*qw.shape[:-1], qw.shape[-1] * 8).float()
    z = zeros.detach().to("cpu").to(torch.int32)
    zn = torch.stack([z & 15, (z >> 4) & 15], dim=-2)  # [.., N/2, 2, G]
    zn = zn.reshape(*z.shape[:-2], z.shape[-2] * 2, z.shape[-1]).float()
    s = scales.detach().to("cpu").float()
    return (q - zn.repeat_interleave(group, dim=-1)) * s.repeat_interleave(group, dim=-1)


# nibble j of each 32-bit word holds k = EX_ORDER[j] of its 8 consecutive k
EX_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


def wna16_ex_pack(q: torch.Tensor) -> torch.Tensor:
    """uint4 values [.., N, K] -> the RDNAHybridW4A16 int8 [.., N, K/2] view of
    ExLlama-shuffled int32 words: little-endian words of 8 consecutive k,
    nibble j = k EX_ORDER[j] (csrc/gemm/w4a16_wmma_gemm.hip:1-8, 82-89; the
    reference tests build it with vLLM's pack_skinny_int4, tests/test_w8a16.py:74-95).
    Pinned by: tests/test_oracle_quant.py (hand-packed known word, inverse of
    wna16_ex_decode)."""
    q = q.detach().to("cpu").to(torch.int64)
    *lead, k = q.shape
    g = q.reshape(*lead, k // 8, 8)
    word = torch.zeros(*lead, k // 8, dtype=torch.int64)
    for j, kk in enumerate(EX_ORDER):
        word |= (g[..., kk] & 15) << (4 * j)
    b = torch.stack([(word >> (8 * i)) & 0xFF for i in range(4)], dim=-1).reshape(*lead, k // 2)
    return b.to(torch.uint8).view(torch.int8)


def wna16_ex_unpack(w: torch.Tensor) -> torch.Tensor:
    """Inverse of wna16_ex_pack: int8/uint8 [.., N, K/2] -> uint4 [.., N, K]."""
    b = w.detach().to("cpu").view(torch.uint8).to(torch.int64)
    *lead, k2 = b.shape
    word = b.reshape(*lead, k2 // 4, 4)
    word = word[..., 0] | (word[..., 1] << 8) | (word[..., 2] << 16) | (word[..., 3] << 24)
    q = torch.zeros(*lead, k2 // 4, 8, dtype=torch.int64)
    for j, kk in enumerate(EX_ORDER):
        q[..., kk] = (word >> (4 * j)) & 15
    return q.reshape(*lead, k2 * 2)


def wna16_ex_decode(w: torch.Tensor, scales: torch.Tensor, group: int) -> torch.Tensor:
    """(u4 - 8) * scale in fp32 for the RDNAHybridW4A16 layout, scales
    [.., N, K/group] (tests/test_w8a16.py:102-119). Pinned by:
    tests/test_oracle_quant.py."""
    q = wna16_ex_unpack(w).float()
    return (q - 8.0) * scales.detach().to("cpu").float().repeat_interleave(group, dim=-1)


def u8b128_decode(w_u8: torch.Tensor, scales: torch.Tensor, group: int) -> torch.Tensor:
    """uint8b128 weights [N, K]: (b - 128) * scale, scales [N] (group 0) or
    [N, K/group] (tests/test_w8a16.py:9-17). Pinned by: tests/test_oracle_quant.py."""
    w = w_u8.detach().to("cpu").to(torch.float32) - 128.0
    s = scales.detach().to("cpu").float()
    if group:
        return w * s.repeat_interleave(group, dim=-1)[..., : w.shape[-1]]
    return w * s.reshape(-1, 1)
