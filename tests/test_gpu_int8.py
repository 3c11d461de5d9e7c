# SPDX-License-Identifier: MIT
"""INT8 W8A8 and the reference's w8a8_wmma_gemm.

int32 accumulators must match the oracle bit for bit; the bf16 output must
stay within max relative error 1e-2 of the dequantize-then-fp32 reference
(peak-normalized, as the reference's tests do: tests/test_w8a8_int8.py:96-100).
"""

import numpy as np
import pytest
import torch

import libstrix_amd  # noqa: F401
import oracle
from conftest import peak_rel_err
from libstrix_amd import functional, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-2


def _case(m, n, k, seed=0):
    d = workloads.c1_int8(seed=seed, m=m, k=k, n=n)
    q, s = oracle.int8_quant_per_token(d["x"])
    return d, q, s


def test_config1_int32_accumulator_bit_exact():
    d, q, s = _case(32, 5120, 5120, seed=1)
    acc = torch.ops.strix._w8a8_i32_acc(q.to(DEV), d["w"].to(DEV)).cpu().numpy()
    assert np.array_equal(acc, oracle.w8a8_int8_acc(q, d["w"]))


def test_config1_bf16_output():
    d, q, s = _case(32, 5120, 5120, seed=1)
    out = functional.w8a8_int8_linear(d["x"].to(DEV), d["w"].to(DEV), d["sw"].to(DEV))
    ref = oracle.w8a8_int8_gemm(q, s, d["w"], d["sw"])
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (32, 5120)
    assert peak_rel_err(out, ref) <= TOL
    # Same fp32 epilogue order as the oracle: the bf16 values agree exactly.
    assert torch.equal(out.cpu(), ref.to(torch.bfloat16))


@pytest.mark.parametrize("m", [1, 5, 16, 17, 33, 64, 100, 300])
@pytest.mark.parametrize("n,k", [(384, 1024), (200, 2048), (520, 4096)])
def test_accumulator_shapes(m, n, k):
    """K 2048 and 4096 at M <= 32 run the decode ring split over 2 and 4
    waves of K: the int32 partial sums must still add up exactly."""
    d, q, s = _case(m, n, k, seed=m)
    acc = torch.ops.strix._w8a8_i32_acc(q.to(DEV), d["w"].to(DEV)).cpu().numpy()
    assert np.array_equal(acc, oracle.w8a8_int8_acc(q, d["w"]))
    out = torch.ops.strix.w8a8_scaled_mm(q.to(DEV), s.to(DEV), d["w"].to(DEV), d["sw"].to(DEV))
    assert peak_rel_err(out, oracle.w8a8_int8_gemm(q, s, d["w"], d["sw"])) <= TOL


@pytest.mark.parametrize("cfg", range(13))
def test_every_cfg_bit_exact(cfg):
    d, q, s = _case(70, 512, 1024, seed=cfg)
    g = torch.ops.strix.w8a8_scaled_mm_cfg(q.to(DEV), s.to(DEV), d["w"].to(DEV), d["sw"].to(DEV), cfg)
    assert torch.equal(g.cpu(), oracle.w8a8_int8_gemm(q, s, d["w"], d["sw"]).to(torch.bfloat16))


def test_tail_split_columns_bit_exact():
    """cfg 5 past one round of 256x256 tiles: the 128x128 tail strip (ragged
    240 columns) must give the same bits as the oracle too."""
    m, n, k = 768, 22000, 256
    d, q, s = _case(m, n, k, seed=12)
    g = torch.ops.strix.w8a8_scaled_mm_cfg(q.to(DEV), s.to(DEV), d["w"].to(DEV), d["sw"].to(DEV), 5).cpu()
    rows = torch.cat([torch.arange(4), torch.arange(254, 258), torch.arange(m - 4, m)])
    ref = oracle.w8a8_int8_gemm(q[rows], s[rows], d["w"], d["sw"]).to(torch.bfloat16)
    assert torch.equal(g[rows], ref)


def test_extreme_accumulator():
    q = torch.full((16, 5120), 127, dtype=torch.int8)
    w = torch.full((32, 5120), -127, dtype=torch.int8)
    acc = torch.ops.strix._w8a8_i32_acc(q.to(DEV), w.to(DEV)).cpu()
    assert (acc == -5120 * 127 * 127).all()


# ---- reference API: uint8b128 weights, per-128-group activations in the op
def _ref_w8a8_wmma(x, w_u8, s_ng):
    qa, sa = oracle.int8_quant_group128(x)
    return oracle.w8a8_int8_group_gemm(qa, sa, (w_u8.to(torch.int16) - 128).to(torch.int8), s_ng)


@pytest.mark.parametrize("m", [1, 6, 64, 300])
@pytest.mark.parametrize("layout", ["gn", "ng", "n"])
def test_w8a8_wmma_gemm_matches_reference(m, layout):
    g = torch.Generator().manual_seed(m)
    n, k = 512, 1024
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = torch.randint(0, 256, (n, k), generator=g, dtype=torch.uint8)
    s_ng = torch.rand(n, k // 128, generator=g) * 0.01
    if layout == "n":
        s_ng = s_ng[:, :1].contiguous()
        scale = s_ng.reshape(n)
    elif layout == "gn":
        scale = s_ng.t().contiguous()
    else:
        scale = s_ng
    out = torch.ops.strix.w8a8_wmma_gemm(w.to(DEV), x.to(DEV), scale.to(DEV))
    assert peak_rel_err(out, _ref_w8a8_wmma(x, w, s_ng)) <= TOL


def test_w8a8_wmma_gemm_padded_rows_and_errors():
    g = torch.Generator().manual_seed(9)
    n, k = 256, 512
    buf = torch.randint(0, 256, (n, k + 128), generator=g, dtype=torch.uint8)
    x = torch.randn(40, k, generator=g).to(torch.bfloat16)
    s = torch.rand(n, generator=g) * 0.01
    out = torch.ops.strix.w8a8_wmma_gemm(buf.to(DEV)[:, :k], x.to(DEV), s.to(DEV))
    assert peak_rel_err(out, _ref_w8a8_wmma(x, buf[:, :k], s[:, None])) <= TOL
    with pytest.raises(RuntimeError, match="K must be divisible by the weight group 128"):
        torch.ops.strix.w8a8_wmma_gemm(buf.to(DEV)[:, :100], x.to(DEV)[:, :100], s.to(DEV))
