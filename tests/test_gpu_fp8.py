# SPDX-License-Identifier: MIT
"""FP8-block W8A8 dense linear against the oracle.

The oracle applies the same 1x128 activation QDQ, dequantizes the weights
with their 128x128 block scales and runs an fp32 matmul (tests/test_fp8.py's
pattern). Bar: max relative error 1e-2 of the peak (bf16 output).
"""

import pytest
import torch

import libstrix_amd  # noqa: F401
import oracle
from conftest import peak_rel_err
from libstrix_amd import workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-2


@pytest.fixture(scope="module")
def c2_weights():
    d = workloads.c2_fp8(seed=2, m=1)
    return d["w"], d["sw"]


@pytest.mark.parametrize("m", [1, 16, 256, 4096])
def test_config2_sweep(m, c2_weights):
    w, sw = c2_weights
    d = workloads.c2_fp8(seed=20 + m, m=m, weights=(w, sw))
    x = d["x"].to(DEV)
    qa, sa = torch.ops.strix.fp8_quant_group128(x)
    out = torch.ops.strix.fp8_w8a8_block_gemm(qa, sa, w.to(DEV), sw.to(DEV))
    rows = torch.arange(m) if m <= 64 else torch.randperm(m, generator=torch.Generator().manual_seed(m))[:48]
    ref = oracle.fp8_block_gemm(qa.cpu()[rows], sa.cpu()[rows], w, sw)
    assert peak_rel_err(out.cpu()[rows], ref) <= TOL


@pytest.mark.parametrize("m", [1, 6, 16, 17, 33, 64, 65, 129, 300])
@pytest.mark.parametrize("n,k", [(300, 1024), (1024, 2048), (520, 4096)])
def test_shapes_and_ragged_n(m, n, k):
    d = workloads.c2_fp8(seed=m, m=m, n=n, k=k)
    qa, sa = oracle.fp8_quant_group128(d["x"])
    out = torch.ops.strix.fp8_w8a8_block_gemm(qa.to(DEV), sa.to(DEV), d["w"].to(DEV), d["sw"].to(DEV))
    assert peak_rel_err(out, oracle.fp8_block_gemm(qa, sa, d["w"], d["sw"])) <= TOL


@pytest.mark.parametrize("cfg", range(13))
def test_every_cfg(cfg):
    d = workloads.c2_fp8(seed=cfg, m=70, n=640, k=1536)
    qa, sa = oracle.fp8_quant_group128(d["x"])
    out = torch.ops.strix.fp8_w8a8_block_gemm_cfg(qa.to(DEV), sa.to(DEV), d["w"].to(DEV), d["sw"].to(DEV), cfg)
    assert peak_rel_err(out, oracle.fp8_block_gemm(qa, sa, d["w"], d["sw"])) <= TOL


def test_tail_split_columns():
    """cfg 5 with more 256x256 tiles than one round: whole rounds take the
    first columns, 128x128 tiles the rest (here a ragged 412-column strip)."""
    m, n, k = 512, 33180, 256
    d = workloads.c2_fp8(seed=11, m=m, n=n, k=k)
    qa, sa = oracle.fp8_quant_group128(d["x"])
    out = torch.ops.strix.fp8_w8a8_block_gemm_cfg(qa.to(DEV), sa.to(DEV), d["w"].to(DEV), d["sw"].to(DEV), 5).cpu()
    rows = torch.cat([torch.arange(8), torch.arange(248, 264), torch.arange(m - 8, m)])
    ref = oracle.fp8_block_gemm(qa[rows], sa[rows], d["w"], d["sw"])
    assert peak_rel_err(out[rows], ref) <= TOL
    assert peak_rel_err(out[rows, 32768:], ref[:, 32768:]) <= TOL


def test_padded_weight_rows():
    d = workloads.c2_fp8(seed=5, m=40, n=512, k=1024)
    buf = torch.zeros(512, 1024 + 128, dtype=torch.uint8)
    buf[:, :1024] = d["w"].view(torch.uint8)
    wv = buf.view(torch.float8_e4m3fn).to(DEV)[:, :1024]
    qa, sa = oracle.fp8_quant_group128(d["x"])
    out = torch.ops.strix.fp8_w8a8_block_gemm(qa.to(DEV), sa.to(DEV), wv, d["sw"].to(DEV))
    assert peak_rel_err(out, oracle.fp8_block_gemm(qa, sa, d["w"], d["sw"])) <= TOL


def test_one_hot_activations_read_back_the_weights():
    d = workloads.c2_fp8(seed=6, m=1, n=256, k=256)
    qa = torch.zeros(256, 256).to(torch.float8_e4m3fn)
    qa[range(256), range(256)] = 1.0
    sa = torch.ones(256, 2)
    out = torch.ops.strix.fp8_w8a8_block_gemm(qa.to(DEV), sa.to(DEV), d["w"].to(DEV), d["sw"].to(DEV))
    want = oracle.fp8_block_dequant(d["w"], d["sw"]).t().to(torch.bfloat16)
    assert torch.equal(out.cpu(), want)


def test_rejects_bad_k():
    x = torch.zeros(4, 96, dtype=torch.float8_e4m3fn, device=DEV)
    with pytest.raises(RuntimeError, match="K must be a multiple of 128"):
        torch.ops.strix.fp8_w8a8_block_gemm(x, torch.ones(4, 1, device=DEV), x, torch.ones(1, 1, device=DEV))


def test_weight8_kmajor_layout():
    # [E, N, K] -> [E, K/128, N, 128] is a pure permutation of bytes.
    g = torch.Generator().manual_seed(7)
    w = torch.randint(-128, 128, (3, 200, 384), generator=g, dtype=torch.int8)
    got = torch.ops.strix.weight8_kmajor(w.to(DEV)).cpu()
    want = w.view(3, 200, 3, 128).permute(0, 2, 1, 3).contiguous()
    assert torch.equal(got, want)
    got2 = torch.ops.strix.weight8_kmajor(w[1].to(DEV)).cpu()
    assert torch.equal(got2, want[1])


@pytest.mark.parametrize("m", [1, 4, 16, 17, 32, 33, 100, 256, 520, 4096])
@pytest.mark.parametrize("n,k", [(17408, 5120), (300, 1024), (520, 4096)])
def test_kmajor_gemm_matches_rowmajor(m, n, k):
    # Same kernels, other weight addressing: the outputs agree bit for bit.
    if m == 4096 and n != 17408:
        pytest.skip("one full-size prefill shape is enough")
    d = workloads.c2_fp8(seed=40 + m, m=m, n=n, k=k, device=DEV)
    qa, sa = torch.ops.strix.fp8_quant_group128(d["x"])
    want = torch.ops.strix.fp8_w8a8_block_gemm(qa, sa, d["w"], d["sw"])
    wk = torch.ops.strix.weight8_kmajor(d["w"])
    got = torch.ops.strix.fp8_w8a8_block_gemm_kmajor(qa, sa, wk, d["sw"])
    assert torch.equal(got, want)


@pytest.mark.parametrize("cfg", range(13))
def test_kmajor_every_cfg(cfg):
    d = workloads.c2_fp8(seed=60 + cfg, m=70, n=520, k=1024, device=DEV)
    qa, sa = torch.ops.strix.fp8_quant_group128(d["x"])
    want = torch.ops.strix.fp8_w8a8_block_gemm_cfg(qa, sa, d["w"], d["sw"], cfg)
    got = torch.ops.strix.fp8_w8a8_block_gemm_kmajor(qa, sa, torch.ops.strix.weight8_kmajor(d["w"]), d["sw"], cfg)
    assert torch.equal(got, want)
