# SPDX-License-Identifier: MIT
"""MXFP4 (e2m1 + e8m0): the dense W4A16 ops of the reference and the MXFP4
fused MoE of BASELINE config 4, against the oracle's LUT decode
(tests/test_mxfp4.py:28-45 pattern). Dequant is byte-exact; GEMMs within max
relative error 1e-2 of the peak."""

import pytest
import torch

import libstrix_amd  # noqa: F401
import oracle
from conftest import peak_rel_err
from libstrix_amd import functional, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-2


def _w(n, k, seed, lo=118, hi=134):
    g = torch.Generator().manual_seed(seed)
    w = torch.randint(0, 256, (n, k // 2), generator=g, dtype=torch.uint8)
    s = torch.randint(lo, hi, (n, k // 32), generator=g, dtype=torch.uint8)
    return w, s


@pytest.mark.parametrize("n,k", [(256, 1024), (2048, 2688), (96, 5376), (64, 2880)])
def test_dequant_byte_exact(n, k):
    w, s = _w(n, k, 0)
    s[0, :3] = 0  # zero blocks
    out = torch.ops.strix.mxfp4_dequant(w.to(DEV), s.to(DEV)).cpu()
    assert out.dtype == torch.bfloat16 and out.shape == (n, k)
    assert torch.equal(out.float(), oracle.mxfp4_decode(w, s))


def test_dequant_extreme_exponents():
    w, _ = _w(32, 256, 1)
    s = torch.randint(1, 255, (32, 8), generator=torch.Generator().manual_seed(2), dtype=torch.uint8)
    out = torch.ops.strix.mxfp4_dequant(w.to(DEV), s.to(DEV)).cpu()
    assert torch.equal(out.float(), oracle.mxfp4_decode(w, s).to(torch.bfloat16).float())


@pytest.mark.parametrize("m", [1, 5, 32, 64, 100, 513])
@pytest.mark.parametrize("n,k", [(256, 1024), (2048, 2688), (400, 2880)])
def test_gemm_matches_oracle(m, n, k):
    w, s = _w(n, k, m)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16)
    out = torch.ops.strix.mxfp4_wmma_gemm(w.to(DEV), x.to(DEV), s.to(DEV), None)
    ref = x.float() @ oracle.mxfp4_decode(w, s).t()
    assert peak_rel_err(out, ref) <= TOL


@pytest.mark.parametrize("cfg", range(8))
def test_every_cfg(cfg):
    w, s = _w(384, 1536, cfg)
    x = torch.randn(70, 1536, generator=torch.Generator().manual_seed(cfg)).to(torch.bfloat16)
    out = torch.ops.strix.mxfp4_wmma_gemm_cfg(w.to(DEV), x.to(DEV), s.to(DEV), None, cfg)
    assert peak_rel_err(out, x.float() @ oracle.mxfp4_decode(w, s).t()) <= TOL


def test_one_hot_activations_are_the_dequantizer():
    n, k = 256, 128
    w, s = _w(n, k, 3, 120, 135)
    x = torch.eye(k, dtype=torch.bfloat16)
    out = torch.ops.strix.mxfp4_wmma_gemm(w.to(DEV), x.to(DEV), s.to(DEV), None).cpu()
    assert torch.equal(out.t().float(), oracle.mxfp4_decode(w, s))


@pytest.mark.parametrize("m", [8, 128])
def test_one_hot_every_normal_exponent(m):
    """Exponents 2..252 (every scaled value a normal bf16) and zero blocks,
    through the GEMM's own weight decoder: exact."""
    n, k = 256, 256
    w, _ = _w(n, k, 7)
    s = torch.randint(2, 253, (n, k // 32), generator=torch.Generator().manual_seed(8), dtype=torch.uint8)
    s[:4, 0] = 0
    x = torch.zeros(m, k, dtype=torch.bfloat16)
    cols = torch.arange(m) % k
    x[torch.arange(m), cols] = 1.0
    out = torch.ops.strix.mxfp4_wmma_gemm(w.to(DEV), x.to(DEV), s.to(DEV), None).cpu()
    assert torch.equal(out.float(), oracle.mxfp4_decode(w, s)[:, cols].t())


def test_zero_block_scale_is_zero():
    n, k = 64, 128
    w, _ = _w(n, k, 4)
    s = torch.zeros(n, k // 32, dtype=torch.uint8)
    s[:, 1] = 127
    x0 = torch.zeros(8, k, dtype=torch.bfloat16)
    x0[:, :32] = 1.0
    x1 = torch.zeros(8, k, dtype=torch.bfloat16)
    x1[:, 32:] = 1.0
    assert torch.count_nonzero(torch.ops.strix.mxfp4_wmma_gemm(w.to(DEV), x0.to(DEV), s.to(DEV), None)) == 0
    assert torch.count_nonzero(torch.ops.strix.mxfp4_wmma_gemm(w.to(DEV), x1.to(DEV), s.to(DEV), None)) > 0


@pytest.mark.parametrize("bias_dim", [1, 2])
@pytest.mark.parametrize("m", [8, 200])
def test_bias(bias_dim, m):
    n, k = 512, 1024
    w, s = _w(n, k, 5)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    bias = torch.randn(n if bias_dim == 1 else m * n, generator=g).to(torch.bfloat16)
    if bias_dim == 2:
        bias = bias.reshape(m, n)
    out = torch.ops.strix.mxfp4_wmma_gemm(w.to(DEV), x.to(DEV), s.to(DEV), bias.to(DEV))
    ref = x.float() @ oracle.mxfp4_decode(w, s).t() + bias.float()
    assert peak_rel_err(out, ref) <= TOL


def test_rejects_unbuilt_shapes():
    x = torch.zeros(4, 96, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(8, 48, dtype=torch.uint8, device=DEV)
    s = torch.zeros(8, 3, dtype=torch.uint8, device=DEV)
    with pytest.raises(RuntimeError, match="K must be a multiple of 64"):
        torch.ops.strix.mxfp4_wmma_gemm(w, x, s, None)
    x = torch.zeros(4, 128, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(8, 64, dtype=torch.uint8, device=DEV)
    with pytest.raises(RuntimeError, match="scale must be uint8"):
        torch.ops.strix.mxfp4_wmma_gemm(w, x, w.float(), None)


# ---------------------------------------------------------------- MoE, config 4
E_SMALL, TOPK = 8, 4


@pytest.fixture(scope="module")
def small_experts():
    return workloads.c4_mxfp4_moe(seed=41, t=1, e=E_SMALL)


@pytest.mark.parametrize("tokens", [1, 5, 40, 300])
@pytest.mark.parametrize("block_m", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("gemm,activation", [("w13", "silu"), ("w13", "gelu_tanh"), ("w2", "silu")])
def test_expert_gemm(tokens, block_m, gemm, activation, small_experts):
    d = small_experts
    g = torch.Generator().manual_seed(tokens * 13 + block_m)
    ids = torch.stack([torch.randperm(E_SMALL, generator=g)[:TOPK] for _ in range(tokens)]).to(torch.int32)
    w, ws = (d["w13"], d["w13_s"]) if gemm == "w13" else (d["w2"], d["w2_s"])
    n, k = w.size(1), w.size(2) * 2
    if gemm == "w13":
        a = torch.randn(tokens, k, generator=g).to(torch.bfloat16)
        a_topk, weights, cols = TOPK, None, n // 2
    else:
        a = torch.randn(tokens * TOPK, k, generator=g).to(torch.bfloat16)
        a_topk, weights, cols = 1, torch.rand(tokens, TOPK, generator=g), n
    sorted_ids, expert_ids, num_post = torch.ops.strix.moe_align(ids.to(DEV), E_SMALL, block_m)
    c = torch.full((tokens * TOPK, cols), float("nan"), dtype=torch.bfloat16, device=DEV)
    torch.ops.strix.moe_gemm_mxfp4(c, a.to(DEV), w.to(DEV), ws.to(DEV), sorted_ids, expert_ids, num_post,
                                   None if weights is None else weights.reshape(-1).to(DEV), a_topk, block_m, 64,
                                   gemm == "w13", activation)
    deq = oracle.mxfp4_decode(w, ws)
    ref = oracle.moe_expert_gemm(a, deq, ids, a_topk, weights)
    if gemm == "w13":
        g_, u_ = ref[:, :cols], ref[:, cols:]
        act = torch.nn.functional.silu(g_) if activation == "silu" else torch.nn.functional.gelu(g_, approximate="tanh")
        ref = act * u_
    assert not torch.isnan(c).any()
    assert peak_rel_err(c, ref) <= TOL


@pytest.mark.parametrize("block_m", [64, 128, 256])
def test_identity_routing_single_expert(block_m):
    """One expert, slot i = token i, the sorted ids alone in a fresh
    allocation (no padding ids): the tiled kernels form no address outside
    the sorted-id range while setting up their copies."""
    t, n, k = 512, 5760, 2880
    w, s = _w(n, k, 7)
    x = torch.randn(t, k, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16)
    sorted_ids = torch.arange(t, dtype=torch.int32, device=DEV)
    expert_ids = torch.zeros(t // block_m, dtype=torch.int32, device=DEV)
    num_post = torch.tensor([t], dtype=torch.int32, device=DEV)
    c = torch.full((t, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    torch.ops.strix.moe_gemm_mxfp4(c, x.to(DEV), w[None].to(DEV), s[None].to(DEV), sorted_ids, expert_ids, num_post,
                                   None, 1, block_m, 64, False, "silu")
    rows = torch.cat([torch.arange(4), torch.arange(t - 4, t)])
    ref = x[rows].float() @ oracle.mxfp4_decode(w, s).t()
    assert not torch.isnan(c).any()
    assert peak_rel_err(c.cpu()[rows], ref) <= TOL


@pytest.fixture(scope="module")
def c4_weights():
    d = workloads.c4_mxfp4_moe(seed=4, t=1)
    dev = {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in d.items()}
    return d, dev


@pytest.mark.parametrize("t", [1, 2048])
def test_config4_fused_moe(t, c4_weights):
    d, dev = c4_weights
    g = torch.Generator().manual_seed(400 + t)
    x = torch.randn(t, 2880, generator=g).to(torch.bfloat16)
    logits = torch.randn(t, 32, generator=g)
    out = functional.fused_moe_mxfp4(x.to(DEV), logits.to(DEV), dev["w13"], dev["w13_s"], dev["w2"], dev["w2_s"], 4)
    ids, w = oracle.route_topk(logits, 4)
    # Every token row is checked.
    ref = oracle.fused_moe(x, ids, w, lambda e: oracle.mxfp4_decode(d["w13"][e], d["w13_s"][e]),
                           lambda e: oracle.mxfp4_decode(d["w2"][e], d["w2_s"][e]))
    assert ref.shape == out.shape
    assert peak_rel_err(out, ref) <= TOL
