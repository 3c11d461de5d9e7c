# SPDX-License-Identifier: MIT
"""The MFMA fragment conventions every kernel relies on (strix_common.h), the
gfx950 counterpart of the reference's tests/test_wmma_layout.py."""

import numpy as np
import pytest
import torch

import libstrix_amd  # noqa: F401

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rand(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    if dtype == torch.int8:
        return torch.randint(-128, 128, shape, generator=g, dtype=torch.int8)
    x = torch.randn(shape, generator=g)
    if dtype == torch.float8_e4m3fn:
        return (x * 8).clamp(-448, 448).to(dtype)
    return x.to(dtype)


@pytest.mark.parametrize("k", [32, 64, 512])
def test_bf16_tile_matches_matmul(k):
    a, b = _rand((16, k), 0, torch.bfloat16), _rand((16, k), 1, torch.bfloat16)
    d = torch.ops.strix._mfma_tile(a.to(DEV), b.to(DEV)).cpu()
    torch.testing.assert_close(d, a.float() @ b.float().t(), rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("k", [128, 512])
def test_fp8_tile_matches_matmul(k):
    a, b = _rand((16, k), 2, torch.float8_e4m3fn), _rand((16, k), 3, torch.float8_e4m3fn)
    d = torch.ops.strix._mfma_tile(a.to(DEV), b.to(DEV)).cpu()
    ref = (a.double() @ b.double().t()).float()
    # The e4m3 MFMA sums its 128 exact products with fp32-level rounding
    # inside the instruction (observed ~1e-4 of the tile's peak); a K mapping
    # that differed between A and B would be wrong by O(1) instead.
    peak = ref.abs().max()
    torch.testing.assert_close(d / peak, ref / peak, rtol=0, atol=2e-4)


@pytest.mark.parametrize("k", [64, 512])
def test_int8_tile_is_exact(k):
    a, b = _rand((16, k), 4, torch.int8), _rand((16, k), 5, torch.int8)
    d = torch.ops.strix._mfma_tile(a.to(DEV), b.to(DEV)).cpu().numpy()
    assert np.array_equal(d, a.numpy().astype(np.int64) @ b.numpy().astype(np.int64).T)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn, torch.int8])
def test_layout_is_not_transposed(dtype):
    k = {torch.bfloat16: 32, torch.float8_e4m3fn: 128, torch.int8: 64}[dtype]
    a = torch.zeros(16, k)
    b = torch.zeros(16, k)
    a[3, 5] = 1
    b[11, 5] = 2
    a[7, k - 1] = 1  # the last K position of a lane group lands too
    b[2, k - 1] = 1
    d = torch.ops.strix._mfma_tile(a.to(dtype).to(DEV), b.to(dtype).to(DEV)).cpu()
    assert d[3, 11] == 2 and d[7, 2] == 1 and d.count_nonzero() == 2


def test_global_to_lds_lane_placement():
    src = torch.arange(1024, dtype=torch.int64).to(torch.uint8)
    dst = torch.ops.strix._g2l_probe(src.to(DEV)).cpu()
    want = src.reshape(64, 16).flip(0).reshape(-1)
    assert torch.equal(dst, want)


def test_hardware_converters():
    """gfx950's fp4->bf16 (scaled), fp8->f32 and f32->bf16 converters against
    the format definitions (tests/golden/kat.json) and torch's RNE cast."""
    import json
    from pathlib import Path

    kat = json.loads((Path(__file__).parent / "golden" / "kat.json").read_text())
    exps = [1, 2, 100, 120, 127, 128, 200, 252, 254]
    scales = torch.tensor([2.0 ** (e - 127) for e in exps], dtype=torch.float32)
    x = torch.randn(4096, generator=torch.Generator().manual_seed(0)) * torch.logspace(-38, 38, 4096)
    x[:4] = torch.tensor([float("inf"), float("-inf"), 1.0 + 2.0**-8, 1.0 + 3 * 2.0**-8])
    fp4, fp8, b16 = torch.ops.strix._cvt_probe(scales.to(DEV), x.to(DEV))
    fp4 = fp4.cpu().view(torch.bfloat16).float()
    lut = torch.tensor(kat["e2m1"], dtype=torch.float32)
    codes = torch.arange(256)
    want8 = torch.tensor([float("nan") if v == "nan" else v for v in kat["e4m3fn"]])
    got8 = fp8.cpu()
    fin = ~torch.isnan(want8)
    print("fp8 converter mismatches:", (got8[fin] != want8[fin]).nonzero().flatten().tolist()[:8])
    assert torch.equal(got8[fin], want8[fin]) and torch.isnan(got8[~fin]).all()
    assert torch.equal(b16.cpu().view(torch.bfloat16), x.to(torch.bfloat16))
    # The scaled fp4 converter (which the MXFP4 decoders use for e8m0
    # exponents 2..252) follows the (low nibble, high nibble) -> (element 0,
    # element 1) reading of every byte in every byte lane, exactly, wherever
    # the scaled values are normal bf16 numbers (exponents 1 and 254 are
    # outside that range and not checked).
    for si, (e, sc) in enumerate(zip(exps, scales.tolist())):
        if not 2 <= e <= 252:
            continue
        want = (torch.stack([lut[codes & 15], lut[codes >> 4]], dim=-1) * sc).to(torch.bfloat16).float()
        bad = int((fp4[si] != want[None]).any(dim=-1).sum())
        assert bad == 0, f"fp4 converter: {bad} (byte lane, byte) mismatches at exponent {e}"
