# SPDX-License-Identifier: MIT
"""The reference's weight-only decode ops and its int4 x int8 ops, against the
oracle (dequantize, then fp32 matmul), following the reference tests:
w8a16_skinny_gemm / w4a16_wmma_gemm / w4a16_dequant / w4a8_wmma_gemm
(tests/test_w8a16.py), fp8_skinny_gemm (tests/test_fp8.py:57-67, 158-166),
mxfp4_gemv (tests/test_mxfp4.py:130-141), moe_gemm_w4a8
(tests/test_moe_w4a8.py) and the _wmma_bf16_tile probe
(tests/test_wmma_layout.py). Bar: max error 1e-2 of the output's peak; the
dequant op is exact."""

import pytest
import torch

import libstrix_amd  # noqa: F401
import oracle
from conftest import peak_rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-2
S = torch.ops.strix


def _g(seed):
    return torch.Generator().manual_seed(seed)


# ------------------------------------------------------------------ w8a16 skinny
@pytest.mark.parametrize("n,k", [(256, 1024), (2048, 5120)])
@pytest.mark.parametrize("m", [1, 3, 5, 8])
@pytest.mark.parametrize("group_size", [0, 32, 128])
def test_w8a16_skinny(n, k, m, group_size):
    g = _g(m * 7 + group_size)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = torch.randint(0, 256, (n, k), generator=g, dtype=torch.uint8)
    s = (torch.rand(n, k // group_size if group_size else 1, generator=g) * 0.01).to(torch.bfloat16)
    if group_size == 0:
        s = s.reshape(n)
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    out = S.w8a16_skinny_gemm(w.to(DEV), x.to(DEV), s.to(DEV), bias.to(DEV), 40, group_size).cpu()
    ref = x.float() @ oracle.u8b128_decode(w, s, group_size).t() + bias.float()
    assert out.shape == (m, n) and peak_rel_err(out, ref) <= TOL


def test_w8a16_skinny_rejects_more_than_8_rows():
    x = torch.randn(9, 256, device=DEV, dtype=torch.bfloat16)
    w = torch.randint(0, 256, (128, 256), device=DEV, dtype=torch.uint8)
    s = torch.full((128,), 0.01, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="1-8 rows"):
        S.w8a16_skinny_gemm(w, x, s, None, 40, 0)


# ------------------------------------------------------------------ fp8 skinny
def _fp8_make(n, k, seed):
    g = _g(seed)
    w_q = (torch.randn(n, k, generator=g) * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
    bs = torch.rand((n + 127) // 128, k // 128, generator=g) * 0.02 + 0.005
    return w_q, bs


@pytest.mark.parametrize("n,k", [(256, 1024), (6144, 5120)])
@pytest.mark.parametrize("m", [1, 2, 5, 8])
def test_fp8_skinny_block_scales(n, k, m):
    w_q, bs = _fp8_make(n, k, m)
    x = torch.randn(m, k, generator=_g(m)).to(torch.bfloat16)
    s = bs.repeat_interleave(128, 0)[:n].contiguous()  # [N, K/128], as the reference's tests expand them
    bias = torch.randn(n, generator=_g(m + 1)).to(torch.bfloat16)
    out = S.fp8_skinny_gemm(w_q.to(DEV), x.to(DEV), s.to(DEV), bias.to(DEV), 40).cpu()
    ref = x.float() @ oracle.fp8_block_dequant(w_q, bs).t() + bias.float()
    assert peak_rel_err(out, ref) <= TOL


@pytest.mark.parametrize("m", [1, 5])
def test_fp8_skinny_channel_scales(m):
    n, k = 512, 2048
    g = _g(40 + m)
    w_q = (torch.randn(n, k, generator=g) * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
    s = torch.rand(n, generator=g) * 0.02 + 0.005
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    out = S.fp8_skinny_gemm(w_q.to(DEV), x.to(DEV), s.to(DEV), None, 40).cpu()
    ref = x.float() @ (oracle.e4m3_decode(w_q.view(torch.uint8)) * s[:, None]).t()
    assert peak_rel_err(out, ref) <= TOL


# ------------------------------------------------------------------ mxfp4 gemv
@pytest.mark.parametrize("n,k", [(256, 1024), (1024, 2688), (512, 5376)])
@pytest.mark.parametrize("m", [1, 2, 3, 5, 8])
def test_mxfp4_gemv(n, k, m):
    g = _g(n + m)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = torch.randint(0, 256, (n, k // 2), generator=g, dtype=torch.uint8)
    s = torch.randint(118, 134, (n, k // 32), generator=g, dtype=torch.uint8)
    out = S.mxfp4_gemv(x.to(DEV), w.to(DEV), s.to(DEV)).cpu()
    assert peak_rel_err(out, x.float() @ oracle.mxfp4_decode(w, s).t()) <= TOL


def test_mxfp4_gemv_rejects_more_than_8_rows():
    with pytest.raises(RuntimeError, match="M <= 8"):
        S.mxfp4_gemv(torch.zeros(9, 64, dtype=torch.bfloat16, device=DEV), torch.zeros(8, 32, dtype=torch.uint8,
                     device=DEV), torch.zeros(8, 2, dtype=torch.uint8, device=DEV))


# ------------------------------------------------------------------ W4A16 RDNAHybrid layout
def _w4(n, k, group, seed):
    g = _g(seed)
    q = torch.randint(0, 16, (n, k), generator=g)
    s = (torch.rand(n, k // group, generator=g) * 0.05 + 0.01).to(torch.bfloat16)
    return q, oracle.wna16_ex_pack(q), s


@pytest.mark.parametrize("n,k", [(256, 1024), (2048, 2560)])
@pytest.mark.parametrize("m", [1, 6, 64, 300])
@pytest.mark.parametrize("group_size", [32, 128])
def test_w4a16_wmma_gemm(n, k, m, group_size):
    q, w, s = _w4(n, k, group_size, m + group_size)
    x = torch.randn(m, k, generator=_g(m)).to(torch.bfloat16)
    bias = torch.randn(n, generator=_g(m + 3)).to(torch.bfloat16)
    out = S.w4a16_wmma_gemm(x.to(DEV), w.to(DEV), s.to(DEV), bias.to(DEV), group_size).cpu()
    ref = x.float() @ oracle.wna16_ex_decode(w, s, group_size).t() + bias.float()
    assert out.shape == (m, n) and peak_rel_err(out, ref) <= TOL


@pytest.mark.parametrize("n,k", [(256, 1024), (5376, 2048)])
@pytest.mark.parametrize("group_size", [32, 128])
def test_w4a16_dequant_exact(n, k, group_size):
    q, w, s = _w4(n, k, group_size, 5)
    out = S.w4a16_dequant(w.to(DEV), s.to(DEV), group_size).cpu()
    assert torch.equal(out, oracle.wna16_ex_decode(w, s, group_size).to(torch.bfloat16))


# ------------------------------------------------------------------ W4A8
@pytest.mark.parametrize("n,k", [(256, 1024), (2048, 2560)])
@pytest.mark.parametrize("m", [6, 64, 300])
@pytest.mark.parametrize("group_size", [0, 32, 128])
def test_w4a8_wmma_gemm(n, k, m, group_size):
    g = _g(m + n + group_size)
    q = torch.randint(0, 16, (n, k), generator=g)
    s = torch.rand(n, k // group_size if group_size else 1, generator=g) * 0.05 + 0.01
    w = oracle.wna16_ex_pack(q)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    sf = s.reshape(n) if group_size == 0 else s.t().contiguous()  # [N] or [G, N], as the reference's tests pass them
    out = S.w4a8_wmma_gemm(w.to(DEV), x.to(DEV), sf.to(DEV)).cpu()
    qa, sa = oracle.int8_quant_group128(x)  # the op's own activation quantization
    a_deq = qa.float() * sa.repeat_interleave(128, dim=1)
    wq = (q.float() - 8.0) * (s.repeat_interleave(group_size, 1) if group_size else s)
    assert peak_rel_err(out, a_deq @ wq.t()) <= TOL


def test_moe_gemm_w4a8_matches_dequantized_reference():
    e, top_k, t, n, k = 8, 4, 37, 256, 640
    g = _g(11)
    q4 = torch.randint(0, 16, (e, n, k), generator=g, dtype=torch.uint8)
    w_u8 = (q4[..., 0::2] | (q4[..., 1::2] << 4)).contiguous()
    scales = (torch.rand(e, n, k // 128, generator=g) * 0.02 + 0.001).to(torch.bfloat16)
    a = torch.randn(t * top_k, k, generator=g).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(e, generator=g)[:top_k] for _ in range(t)]).to(torch.int32)
    weights = torch.rand(t, top_k, generator=g)
    qa = torch.empty(a.shape, dtype=torch.int8, device=DEV)
    sa = torch.empty(a.size(0), k // 128, dtype=torch.float32, device=DEV)
    S.moe_act_quant_i8(a.to(DEV), qa, sa)
    sorted_ids, expert_ids, num_post = S.moe_align(ids.to(DEV), e, 64)
    c = torch.full((t * top_k, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    S.moe_gemm_w4a8(c, qa, sa, w_u8.to(DEV), scales.to(DEV), sorted_ids, expert_ids, num_post,
                    weights.reshape(-1).to(DEV), 1, 64, 128, False, "silu")
    a_deq = qa.cpu().float() * sa.cpu().repeat_interleave(128, dim=1)
    b = oracle.wna16_sym_decode(w_u8, scales, 128)
    ref = oracle.moe_expert_gemm(a_deq, b, ids, 1, weights)
    assert not torch.isnan(c).any()
    assert peak_rel_err(c.cpu(), ref) <= TOL


# ------------------------------------------------------------------ layout probe
@pytest.mark.parametrize("k", [16, 64, 512])
def test_wmma_bf16_tile_matches_matmul(k):
    a = torch.randn(16, k, generator=_g(k)).to(torch.bfloat16)
    b = torch.randn(16, k, generator=_g(k + 1)).to(torch.bfloat16)
    d = S._wmma_bf16_tile(a.to(DEV), b.to(DEV)).cpu()
    torch.testing.assert_close(d, a.float() @ b.float().t(), rtol=1e-5, atol=1e-4)


def test_wmma_bf16_tile_not_transposed():
    a = torch.zeros(16, 16, dtype=torch.bfloat16)
    b = torch.zeros_like(a)
    a[3, 5] = 1
    b[11, 5] = 2
    d = S._wmma_bf16_tile(a.to(DEV), b.to(DEV)).cpu()
    assert d[3, 11] == 2 and d.count_nonzero() == 1
