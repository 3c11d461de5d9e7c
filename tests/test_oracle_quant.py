# SPDX-License-Identifier: MIT
"""Pins the oracle's quantizers and decoders (CPU only).

Each check is independent of the oracle's own formula: the format
definitions in tests/golden/kat.json, brute-force nearest-value search,
error bounds and hand-computed cases.
"""

import json
import math
from pathlib import Path

import torch

import oracle
from libstrix_amd import workloads

KAT = json.loads((Path(__file__).parent / "golden" / "kat.json").read_text())


def test_e4m3_decode_matches_format_definition_for_all_codes():
    codes = torch.arange(256, dtype=torch.uint8)
    got = oracle.e4m3_decode(codes.view(torch.float8_e4m3fn))
    for c in range(256):
        want = KAT["e4m3fn"][c]
        if want == "nan":
            assert math.isnan(got[c].item()), c
        else:
            assert got[c].item() == want, (c, got[c].item(), want)
    # landmarks: largest finite, smallest subnormal, smallest normal
    assert KAT["e4m3fn"][0x7E] == 448.0 and KAT["e4m3fn"][0x01] == 2.0**-9 and KAT["e4m3fn"][0x08] == 2.0**-6


def _nearest_even_e4m3(v: torch.Tensor) -> torch.Tensor:
    """Independent encoder: the finite e4m3 code nearest to v, ties to the
    code with an even mantissa (bit 0 clear). Brute force over all codes."""
    vals = torch.tensor([x if x != "nan" else float("inf") for x in KAT["e4m3fn"]], dtype=torch.float64)
    codes = torch.arange(256)
    finite = torch.isfinite(vals)
    vals, codes = vals[finite], codes[finite]
    d = (v.double()[:, None] - vals[None, :]).abs()
    best = d.min(dim=1, keepdim=True).values
    cand = d == best
    # prefer even mantissa among ties, and +0 over -0
    score = cand.double() * (2.0 + ((codes & 1) == 0).double() + (codes == 0).double() * 0.5)[None, :]
    return codes[score.argmax(dim=1)].to(torch.uint8)


def test_fp8_quant_matches_independent_nearest_even_encoder():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(6, 512, generator=g) * torch.logspace(-3, 2, 512)[None, :]
    x[1, 128:256] = 0.0  # an all-zero group
    x[2, :128] *= 1e-4   # tiny values land on e4m3 subnormals after scaling
    x = x.to(torch.bfloat16)
    q, s = oracle.fp8_quant_group128(x)
    xf = x.float()
    amax = xf.reshape(6, 4, 128).abs().amax(-1)
    assert torch.equal(s, torch.where(amax > 0, amax / 448.0, torch.ones_like(amax)))
    assert s[1, 1].item() == 1.0
    scaled = xf.reshape(6, 4, 128) / s[..., None]
    want = _nearest_even_e4m3(scaled.flatten()).reshape(6, 512)
    assert torch.equal(q.view(torch.uint8), want)
    # the group maximum maps to the largest finite code
    assert (q.float().abs().reshape(6, 4, 128).amax(-1)[amax > 0] == 448.0).all()


def test_int8_per_token_bounds_and_extremes():
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(9, 640, generator=g) * 3).to(torch.bfloat16)
    x[4] = 0
    q, s = oracle.int8_quant_per_token(x)
    xf = x.float()
    assert s[4].item() == 1.0 and q[4].abs().max().item() == 0
    live = [i for i in range(9) if i != 4]
    assert (q[live].abs().amax(dim=1) == 127).all()
    err = (xf - q.float() * s[:, None]).abs()
    # half a step, plus the fp32 rounding of q * s itself (|q s| <= 127 s)
    assert (err <= s[:, None] / 2 + 127 * s[:, None] * 2.0**-23).all()
    assert torch.allclose(s[live], xf[live].abs().amax(1) / 127.0, rtol=0, atol=0)


def test_int8_rounding_ties_go_to_even():
    # amax 127 makes s exactly 1, so x/s = x and the tie cases are exact.
    x = torch.tensor([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.0]], dtype=torch.bfloat16)
    q, s = oracle.int8_quant_per_token(torch.nn.functional.pad(x, (0, 120)))
    assert s.item() == 1.0
    assert q[0, :8].tolist() == [127, 0, 2, 2, 0, -2, -2, 3]


def test_int8_group_quant_groups_are_independent():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(3, 384, generator=g).to(torch.bfloat16)
    x[0, 128:256] *= 100
    q, s = oracle.int8_quant_group128(x)
    for gi in range(3):
        qs, ss = oracle.int8_quant_per_token(x[:, 128 * gi:128 * (gi + 1)])
        assert torch.equal(q[:, 128 * gi:128 * (gi + 1)], qs)
        assert torch.equal(s[:, gi], ss)


def test_mxfp4_decode_known_answers_and_nibble_order():
    lut = KAT["e2m1"]
    # byte 0x21: low nibble 1 (0.5) is k=0, high nibble 2 (1.0) is k=1
    w = torch.zeros(1, 16, dtype=torch.uint8)
    w[0, 0] = 0x21
    w[0, 1] = 0xF7  # k=2: 6.0, k=3: -6.0
    s = torch.tensor([[127]], dtype=torch.uint8)
    d = oracle.mxfp4_decode(w, s)
    assert d[0, :4].tolist() == [lut[1], lut[2], lut[7], lut[15]] == [0.5, 1.0, 6.0, -6.0]
    # exponent folding and the zero block
    s2 = torch.tensor([[120]], dtype=torch.uint8)
    assert oracle.mxfp4_decode(w, s2)[0, 2].item() == 6.0 * KAT["e8m0"]["120"]
    assert oracle.mxfp4_decode(w, torch.zeros(1, 1, dtype=torch.uint8)).abs().max().item() == 0.0


def test_mxfp4_decode_brute_force():
    g = torch.Generator().manual_seed(3)
    w = torch.randint(0, 256, (3, 32), generator=g, dtype=torch.uint8)
    s = torch.randint(110, 140, (3, 2), generator=g, dtype=torch.uint8)
    d = oracle.mxfp4_decode(w, s)
    for n in range(3):
        for k in range(64):
            byte = int(w[n, k // 2])
            nib = byte & 15 if k % 2 == 0 else byte >> 4
            want = KAT["e2m1"][nib] * 2.0 ** (int(s[n, k // 32]) - 127)
            assert d[n, k].item() == want


def test_wna16_zp_decode_brute_force():
    g = torch.Generator().manual_seed(4)
    e, n, k, grp = 2, 4, 256, 128
    q = torch.randint(0, 16, (e, n, k), generator=g, dtype=torch.uint8)
    z = torch.randint(0, 16, (e, n, k // grp), generator=g, dtype=torch.uint8)
    s = (torch.rand(e, n, k // grp, generator=g) * 0.02).to(torch.bfloat16)
    qw = workloads.pack_int4_k(q)
    zp = workloads.pack_zeros_n(z)
    assert qw.dtype == torch.int32 and tuple(qw.shape) == (e, n, k // 8)
    d = oracle.wna16_zp_decode(qw, s, zp, grp)
    for ei in range(e):
        for ni in range(n):
            for ki in (0, 1, 7, 8, 127, 128, 255):
                word = int(qw[ei, ni, ki // 8]) & 0xFFFFFFFF
                qq = (word >> (4 * (ki % 8))) & 15
                zb = int(zp[ei, ni // 2, ki // grp])
                zz = zb & 15 if ni % 2 == 0 else zb >> 4
                assert qq == int(q[ei, ni, ki]) and zz == int(z[ei, ni, ki // grp])
                assert d[ei, ni, ki].item() == (qq - zz) * float(s[ei, ni, ki // grp])


def test_wna16_sym_decode_nibble_order():
    w = torch.tensor([[[0x9A]]], dtype=torch.uint8)  # k=0: 10, k=1: 9
    s = torch.tensor([[[2.0]]], dtype=torch.bfloat16)
    assert oracle.wna16_sym_decode(w, s, 2).tolist() == [[[4.0, 2.0]]]


def test_wna16_ex_pack_known_word_and_inverse():
    # k = 0..7 with value k: nibble j must hold k (0 2 4 6 1 3 5 7)[j], so the
    # little-endian word is 0x75316420 -> bytes 20 64 31 75.
    q = torch.arange(8).reshape(1, 8)
    b = oracle.wna16_ex_pack(q).view(torch.uint8)
    assert b.tolist() == [[0x20, 0x64, 0x31, 0x75]]
    g = torch.Generator().manual_seed(3)
    q = torch.randint(0, 16, (5, 64), generator=g)
    assert torch.equal(oracle.wna16_ex_unpack(oracle.wna16_ex_pack(q)), q)
    s = torch.rand(5, 2, generator=g)
    d = oracle.wna16_ex_decode(oracle.wna16_ex_pack(q), s, 32)
    assert torch.equal(d, (q.float() - 8) * s.repeat_interleave(32, 1))


def test_u8b128_decode_channel_and_group():
    w = torch.tensor([[0, 128, 255, 129]], dtype=torch.uint8)
    assert oracle.u8b128_decode(w, torch.tensor([2.0]), 0).tolist() == [[-256.0, 0.0, 254.0, 2.0]]
    s = torch.tensor([[1.0, 0.5]])
    assert oracle.u8b128_decode(w, s, 2).tolist() == [[-128.0, 0.0, 63.5, 0.5]]
