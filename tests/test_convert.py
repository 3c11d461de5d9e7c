# SPDX-License-Identifier: MIT
"""Load-time AWQ -> WNA16 zero-point converter (CPU).

Pinned independently of the converter's own code: an AWQ packer written
from the format's definition with Python integers (nibble i of a word holds
column 8w + order[i]) and AutoAWQ's known word for columns 0..7; then the
converted tensors decode, through the oracle, to (q - z) * s transposed."""

import pytest
import torch

import oracle
from libstrix_amd import convert, workloads

ORDER = [0, 2, 4, 6, 1, 3, 5, 7]


def awq_pack_reference(vals: torch.Tensor) -> torch.Tensor:
    """[R, C] values 0..15 -> int32 [R, C/8] AWQ words, Python integer loops."""
    r, c = vals.shape
    out = torch.zeros(r, c // 8, dtype=torch.int32)
    v = vals.tolist()
    for i in range(r):
        for w in range(c // 8):
            word = 0
            for nib in range(8):
                word |= int(v[i][8 * w + ORDER[nib]]) << (4 * nib)
            out[i, w] = word - (1 << 32) if word >= (1 << 31) else word
    return out


def test_awq_known_word():
    # Columns 0..7 holding their own index pack to 0x75316420 (AutoAWQ order).
    w = awq_pack_reference(torch.arange(8).reshape(1, 8))
    assert int(w[0, 0]) & 0xFFFFFFFF == 0x75316420
    assert convert.awq_unpack(w).tolist() == [list(range(8))]


@pytest.mark.parametrize("experts", [None, 3])
def test_awq_to_wna16_decodes_to_q_minus_z_times_s(experts):
    k, n, group = 256, 48, 64
    g = torch.Generator().manual_seed(11)
    lead = () if experts is None else (experts,)
    q = torch.randint(0, 16, (*lead, k, n), generator=g)
    z = torch.randint(0, 16, (*lead, k // group, n), generator=g)
    s = (torch.rand(*lead, k // group, n, generator=g) * 0.02 + 0.001).to(torch.float16)
    flat = lambda t: t.reshape(-1, t.shape[-1])
    qw = awq_pack_reference(flat(q)).reshape(*lead, k, n // 8)
    qz = awq_pack_reference(flat(z)).reshape(*lead, k // group, n // 8)
    b, sc, zz = convert.awq_to_wna16(qw, qz, s)
    assert b.dtype == torch.int32 and tuple(b.shape) == (*lead, n, k // 8)
    assert sc.dtype == torch.bfloat16 and tuple(sc.shape) == (*lead, n, k // group)
    assert zz.dtype == torch.uint8 and tuple(zz.shape) == (*lead, n // 2, k // group)
    # The kernel layouts, as the workloads' own packers build them.
    qt, zt = q.transpose(-1, -2), z.transpose(-1, -2)
    assert torch.equal(b, workloads.pack_int4_k(qt))
    assert torch.equal(zz, workloads.pack_zeros_n(zt.to(torch.uint8)))
    want = (qt.float() - zt.float().repeat_interleave(group, -1)) * s.transpose(-1, -2).to(
        torch.bfloat16).float().repeat_interleave(group, -1)
    assert torch.equal(oracle.wna16_zp_decode(b, sc, zz, group), want)


def test_awq_shape_errors():
    with pytest.raises(ValueError, match="disagree"):
        convert.awq_to_wna16(torch.zeros(128, 4, dtype=torch.int32), torch.zeros(2, 4, dtype=torch.int32),
                             torch.zeros(2, 16))
    with pytest.raises(ValueError, match="int32"):
        convert.awq_unpack(torch.zeros(4, 4, dtype=torch.int64))
