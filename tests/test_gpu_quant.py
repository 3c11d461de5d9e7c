# SPDX-License-Identifier: MIT
"""Activation quantizers against the oracle: q and s bit for bit."""

import pytest
import torch

import libstrix_amd  # noqa: F401
import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _x(m, k, seed, dtype=torch.bfloat16, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g) * scale
    return x.to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,k", [(1, 5120), (32, 5120), (7, 1024), (3, 8), (300, 2048)])
def test_int8_per_token_bit_exact(m, k, dtype):
    x = _x(m, k, 0, dtype, 3.0)
    if m > 2:
        x[1] = 0  # a zero row takes scale 1
    q, s = torch.ops.strix.int8_quant_per_token(x.to(DEV))
    qr, sr = oracle.int8_quant_per_token(x)
    assert torch.equal(s.cpu(), sr)
    assert torch.equal(q.cpu(), qr)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,k", [(1, 5120), (16, 5120), (37, 768), (4096, 2048)])
def test_fp8_group128_bit_exact(m, k, dtype):
    x = _x(m, k, 1, dtype)
    x[0, 128:256] = 0
    if m > 5:
        x[5, :128] *= 1e-3  # small groups: subnormal-heavy codes
    q, s = torch.ops.strix.fp8_quant_group128(x.to(DEV))
    qr, sr = oracle.fp8_quant_group128(x)
    assert torch.equal(s.cpu(), sr)
    assert torch.equal(q.cpu().view(torch.uint8), qr.view(torch.uint8))


def _all16(dtype):
    v = torch.arange(0, 1 << 15, dtype=torch.int32).to(torch.int16).view(dtype).float()
    return v[torch.isfinite(v)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fp8_group128_every_input_value(dtype):
    # Each 128-group holds one maximum and 127 values at or below it; every
    # 16-bit value (both signs) meets 48 sampled maxima, including the
    # smallest ones (subnormal scales) and the largest: the kernel's
    # reciprocal-product quotient must round like the oracle's division.
    xs = _all16(dtype)
    xs = torch.cat([xs, -xs])
    pos = _all16(dtype)
    pos = pos[pos > 0]
    mxs = torch.cat([pos[:4], pos[::(pos.numel() // 40)], pos[-4:]])
    groups = []
    for mx in mxs.tolist():
        v = xs[xs.abs() <= mx]
        v = torch.cat([v, v.new_zeros((-v.numel()) % 127)]).view(-1, 127)
        groups.append(torch.cat([v.new_full((v.shape[0], 1), mx), v], dim=1))
    g = torch.cat(groups)
    g = torch.cat([g, g.new_zeros((-g.shape[0]) % 8, 128)]).view(-1, 1024).to(dtype)
    q, s = torch.ops.strix.fp8_quant_group128(g.to(DEV))
    qr, sr = oracle.fp8_quant_group128(g)
    assert torch.equal(s.cpu(), sr)
    assert torch.equal(q.cpu().view(torch.uint8), qr.view(torch.uint8))


def test_moe_act_quant_i8_bit_exact():
    # tests/test_moe_w4a8.py:24-36 shape; division, so no off-by-one ties
    x = _x(37, 640, 2, scale=3.0)
    x[5, 128:256] = 0
    q = torch.empty(37, 640, dtype=torch.int8, device=DEV)
    sa = torch.empty(37, 5, dtype=torch.float32, device=DEV)
    torch.ops.strix.moe_act_quant_i8(x.to(DEV), q, sa)
    qr, sr = oracle.int8_quant_group128(x)
    assert torch.equal(sa.cpu(), sr)
    assert torch.equal(q.cpu(), qr)
