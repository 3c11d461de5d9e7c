# SPDX-License-Identifier: MIT
"""The FP8 group quantizer (libstrix_amd/csrc/quant.hip, div_for_e4m3) forms
x / sc as x * RN(1/sc) and takes the IEEE division only near e4m3 rounding
midpoints, in e4m3's subnormal range and for subnormal scales. This CPU test
checks that argument on every 16-bit input x against a sample of group maxima
(every 13th bf16 and fp16 bit pattern, plus edge cases): the e4m3 byte of the
guarded product equals the e4m3 byte of the IEEE quotient. The same formula
without the guard must disagree somewhere, so the check has teeth. The GPU
tests compare the kernel itself with the oracle's IEEE division."""

import pytest
import torch


def _all16(dtype):
    bits = torch.arange(0, 1 << 15, dtype=torch.int32).to(torch.int16)
    v = bits.view(dtype).float()
    return v[torch.isfinite(v)]


def _guarded(x, sc, guard=True):
    r = 1.0 / sc
    q = x * r
    b = q.view(torch.int32) & 0x7FFFFFFF
    d = (b & 0xFFFFF) - 0x80000
    slow = (sc < 2.0 ** -126) | ((b >= 1) & (b < (121 << 23)))
    if guard:
        slow = slow | ((d >= -4) & (d <= 4))
    return torch.where(slow, x / sc, q)


def _mismatches(dtype, guard=True):
    xs = _all16(dtype)
    xs = torch.cat([xs, -xs])
    pos = _all16(dtype)
    pos = pos[pos > 0]
    mxs = torch.cat([pos[::13], pos[-3:], pos[:3]])
    bad = 0
    for i in range(0, mxs.numel(), 64):
        mx = mxs[i:i + 64, None]
        sc = mx / 448.0
        x = xs[None, :].expand(mx.shape[0], -1)
        keep = x.abs() <= mx
        x, scb = x[keep], sc.expand_as(keep)[keep]
        a = (x / scb).to(torch.float8_e4m3fn).view(torch.uint8)
        b = _guarded(x, scb, guard).to(torch.float8_e4m3fn).view(torch.uint8)
        bad += int((a != b).sum())
    return bad


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_guarded_product_rounds_like_ieee_division(dtype):
    assert _mismatches(dtype) == 0


def test_unguarded_product_differs():
    assert _mismatches(torch.bfloat16, guard=False) > 0
