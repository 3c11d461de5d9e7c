# SPDX-License-Identifier: MIT
"""MoE plumbing and the FP8-block W8A8 fused MoE.

Routing ids, sorted ids, expert ids and num_post_padded are compared bit for
bit; floating outputs within max relative error 1e-2 of the peak. Outputs
start as NaN so an unwritten slot fails (tests/test_moe_gemm.py:68-70).
"""

import pytest
import torch

import libstrix_amd  # noqa: F401
import oracle
from conftest import peak_rel_err
from libstrix_amd import functional, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-2


@pytest.mark.parametrize("t,e,k", [(4096, 128, 8), (2048, 32, 4), (1, 128, 8), (7, 1000, 5)])
@pytest.mark.parametrize("renorm", [True, False])
def test_route_ids_bit_exact(t, e, k, renorm):
    logits = torch.randn(t, e, generator=torch.Generator().manual_seed(t + e))
    ids, w = torch.ops.strix.moe_route_topk(logits.to(DEV), k, renorm)
    rid, rw = oracle.route_topk(logits, k, renorm)
    assert torch.equal(ids.cpu(), rid)
    torch.testing.assert_close(w.cpu(), rw, rtol=1e-5, atol=1e-7)


def test_route_ties_and_bf16_logits():
    logits = torch.zeros(3, 64)
    logits[0, [5, 9, 40]] = 1.0       # a three-way tie: lower ids first
    logits[1, :] = 0.5                # all equal: ids 0..k-1
    logits[2, [63, 0]] = 2.0
    lb = logits.to(torch.bfloat16)
    ids, _ = torch.ops.strix.moe_route_topk(lb.to(DEV), 4, True)
    rid, _ = oracle.route_topk(lb.float(), 4, True)
    assert torch.equal(ids.cpu(), rid)
    assert ids.cpu()[0].tolist()[:3] == [5, 9, 40] and ids.cpu()[1].tolist() == [0, 1, 2, 3]


@pytest.mark.parametrize("t,k,e,bm", [(1, 8, 128, 16), (64, 8, 128, 16), (5, 4, 16, 32), (2048, 4, 32, 64),
                                      (4096, 8, 128, 128), (8192, 8, 128, 256), (300, 8, 256, 64)])
def test_align_bit_exact(t, k, e, bm):
    g = torch.Generator().manual_seed(t * 7 + e)
    ids = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(t)]).to(torch.int32)
    sorted_ids, expert_ids, num_post = torch.ops.strix.moe_align(ids.to(DEV), e, bm)
    rs, re, total = oracle.align(ids, bm, e)
    assert int(num_post.item()) == total
    s = sorted_ids.cpu()
    assert s[:total].tolist() == rs
    assert (s[total:] == t * k).all()
    x = expert_ids.cpu()
    assert x[:total // bm].tolist() == re
    assert (x[total // bm:] == -1).all()


@pytest.mark.parametrize("s,e,bm", [(1024, 128, 16), (1025, 128, 16), (1000, 1024, 64), (1024, 96, 32),
                                    (3000, 1000, 128), (2049, 7, 16), (0, 8, 16)])
def test_align_single_block_threshold_bit_exact(s, e, bm):
    """Up to 1024 slots the align runs as one block, above as three passes:
    both against the contract, with uneven E, empty experts and no slots."""
    g = torch.Generator().manual_seed(s + e)
    ids = torch.randint(0, e, (s,), generator=g, dtype=torch.int32)
    if s:
        ids[ids == 1] = 2          # expert 1 never routed
    sorted_ids, expert_ids, num_post = torch.ops.strix.moe_align(ids.to(DEV), e, bm)
    rs, re, total = oracle.align(ids, bm, e)
    assert int(num_post.item()) == total
    assert sorted_ids.cpu()[:total].tolist() == rs and (sorted_ids.cpu()[total:] == s).all()
    assert expert_ids.cpu()[:total // bm].tolist() == re and (expert_ids.cpu()[total // bm:] == -1).all()


@pytest.mark.parametrize("t,e,k,bm", [(1, 128, 8, 16), (64, 128, 8, 16), (128, 128, 8, 64), (129, 128, 8, 64),
                                      (3, 32, 4, 32), (300, 1000, 3, 16)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_route_align_matches_route_then_align(t, e, k, bm, dtype):
    logits = torch.randn(t, e, generator=torch.Generator().manual_seed(t * e + k)).to(dtype)
    ids, w, sorted_ids, expert_ids, num_post = torch.ops.strix.moe_route_align(logits.to(DEV), k, bm, True)
    rid, rw = oracle.route_topk(logits.float(), k, True)
    assert torch.equal(ids.cpu(), rid)
    torch.testing.assert_close(w.cpu(), rw, rtol=1e-5, atol=1e-7)
    rs, re, total = oracle.align(rid, bm, e)
    assert int(num_post.item()) == total and sorted_ids.cpu()[:total].tolist() == rs
    assert (sorted_ids.cpu()[total:] == t * k).all()
    assert expert_ids.cpu()[:total // bm].tolist() == re and (expert_ids.cpu()[total // bm:] == -1).all()


def test_moe_sum_bit_exact():
    y = torch.randn(37, 8, 2048, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    out = torch.empty(37, 2048, dtype=torch.bfloat16, device=DEV)
    torch.ops.strix.moe_sum(y.to(DEV), out)
    assert torch.equal(out.cpu(), oracle.moe_sum(y.reshape(-1, 2048), 8).to(torch.bfloat16))


# ---------------------------------------------------------------- expert GEMM
E_SMALL, TOPK = 16, 8


@pytest.fixture(scope="module")
def small_experts():
    d = workloads.c3_fp8_moe(seed=11, t=1, e=E_SMALL)
    deq13 = torch.stack([oracle.fp8_block_dequant(d["w13"][i], d["w13_s"][i]) for i in range(E_SMALL)])
    deq2 = torch.stack([oracle.fp8_block_dequant(d["w2"][i], d["w2_s"][i]) for i in range(E_SMALL)])
    return d, deq13, deq2


@pytest.mark.parametrize("tokens", [1, 5, 40, 300])
@pytest.mark.parametrize("block_m", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("gemm,activation", [("w13", "silu"), ("w13", "gelu_tanh"), ("w2", "silu")])
def test_expert_gemm(tokens, block_m, gemm, activation, small_experts):
    d, deq13, deq2 = small_experts
    g = torch.Generator().manual_seed(tokens * 31 + block_m)
    ids = torch.stack([torch.randperm(E_SMALL, generator=g)[:TOPK] for _ in range(tokens)]).to(torch.int32)
    if gemm == "w13":
        w, ws, deq, k_in = d["w13"], d["w13_s"], deq13, 2048
        a = torch.randn(tokens, k_in, generator=g).to(torch.bfloat16)
        a_topk, weights, cols = TOPK, None, deq.size(1) // 2
    else:
        w, ws, deq, k_in = d["w2"], d["w2_s"], deq2, 768
        a = torch.randn(tokens * TOPK, k_in, generator=g).to(torch.bfloat16)
        a_topk, weights, cols = 1, torch.rand(tokens, TOPK, generator=g), deq.size(1)
    qa, sa = oracle.fp8_quant_group128(a)
    sorted_ids, expert_ids, num_post = torch.ops.strix.moe_align(ids.to(DEV), E_SMALL, block_m)
    c = torch.full((tokens * TOPK, cols), float("nan"), dtype=torch.bfloat16, device=DEV)
    torch.ops.strix.moe_gemm_fp8_w8a8(c, qa.to(DEV), sa.to(DEV), w.to(DEV), ws.to(DEV), sorted_ids, expert_ids,
                                      num_post, None if weights is None else weights.reshape(-1).to(DEV), a_topk,
                                      block_m, 128, gemm == "w13", activation)
    a_deq = qa.float() * sa.repeat_interleave(128, dim=1)
    ref = oracle.moe_expert_gemm(a_deq, deq, ids, a_topk, weights)
    if gemm == "w13":
        n2 = cols
        g_, u_ = ref[:, :n2], ref[:, n2:]
        act = torch.nn.functional.silu(g_) if activation == "silu" else torch.nn.functional.gelu(g_, approximate="tanh")
        ref = act * u_
    assert not torch.isnan(c).any()
    assert peak_rel_err(c, ref) <= TOL


@pytest.mark.parametrize("block_m", [128, 256])
@pytest.mark.parametrize("gemm", ["w13", "w2"])
def test_expert_gemm_ragged_columns(block_m, gemm):
    """Column counts that are not a multiple of the 256-column tile (gated
    halves of 384, three 128-column halves; a w2 of 384 rows), experts
    holding more than one block. (Gated FP8-block halves must be whole
    128-row scale blocks.)"""
    e, k_top, t, inter, h = 4, 2, 700, 384, 384
    g = torch.Generator().manual_seed(block_m + len(gemm))
    ids = torch.stack([torch.randperm(e, generator=g)[:k_top] for _ in range(t)]).to(torch.int32)
    if gemm == "w13":
        n, k_in, a_rows, a_topk = 2 * inter, h, t, k_top
    else:
        n, k_in, a_rows, a_topk = h, inter, t * k_top, 1
    w = (torch.randn(e, n, k_in, generator=g) * 0.02)
    wq, ws = workloads.quantize_fp8_block(w)
    deq = torch.stack([oracle.fp8_block_dequant(wq[i], ws[i]) for i in range(e)])
    a = torch.randn(a_rows, k_in, generator=g).to(torch.bfloat16)
    weights = None if gemm == "w13" else torch.rand(t, k_top, generator=g)
    qa, sa = oracle.fp8_quant_group128(a)
    sorted_ids, expert_ids, num_post = torch.ops.strix.moe_align(ids.to(DEV), e, block_m)
    cols = inter if gemm == "w13" else n
    c = torch.full((t * k_top, cols), float("nan"), dtype=torch.bfloat16, device=DEV)
    torch.ops.strix.moe_gemm_fp8_w8a8(c, qa.to(DEV), sa.to(DEV), wq.to(DEV), ws.to(DEV), sorted_ids, expert_ids,
                                      num_post, None if weights is None else weights.reshape(-1).to(DEV), a_topk,
                                      block_m, 64, gemm == "w13", "silu")
    ref = oracle.moe_expert_gemm(qa.float() * sa.repeat_interleave(128, dim=1), deq, ids, a_topk, weights)
    if gemm == "w13":
        ref = torch.nn.functional.silu(ref[:, :inter]) * ref[:, inter:]
    assert not torch.isnan(c).any()
    assert peak_rel_err(c, ref) <= TOL


# ---------------------------------------------------------------- fused, config 3
@pytest.fixture(scope="module")
def c3_weights():
    d = workloads.c3_fp8_moe(seed=3, t=1)
    dev = {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in d.items()}
    return d, dev


@pytest.mark.parametrize("t", [1, 64, 4096])
def test_config3_fused_moe(t, c3_weights):
    d, dev = c3_weights
    g = torch.Generator().manual_seed(100 + t)
    x = torch.randn(t, 2048, generator=g).to(torch.bfloat16)
    logits = torch.randn(t, 128, generator=g)
    out = functional.fused_moe_fp8_w8a8(x.to(DEV), logits.to(DEV), dev["w13"], dev["w13_s"], dev["w2"],
                                        dev["w2_s"], 8)
    ids, w = oracle.route_topk(logits, 8)
    # Every token row is checked (the output starts uninitialized, so a row
    # the chain never writes fails).
    ref = oracle.fused_moe(x, ids, w,
                           lambda e: oracle.fp8_block_dequant(d["w13"][e], d["w13_s"][e]),
                           lambda e: oracle.fp8_block_dequant(d["w2"][e], d["w2_s"][e]), act_quant="fp8")
    assert ref.shape == out.shape
    assert peak_rel_err(out, ref) <= TOL


@pytest.mark.parametrize("t", [1, 64, 700])
def test_fused_moe_kmajor_weights_bit_identical(t):
    # K-block-major expert weights (weight8_kmajor) through the whole chain:
    # the same bits as row-major, for the decode and the tiled kernels.
    c3 = workloads.c3_fp8_moe(seed=5, t=1, device=DEV)
    logits = torch.randn(t, 128, generator=torch.Generator().manual_seed(t)).to(DEV)
    x = torch.randn(t, 2048, generator=torch.Generator().manual_seed(t + 1)).to(torch.bfloat16).to(DEV)
    want = functional.fused_moe_fp8_w8a8(x, logits, c3["w13"], c3["w13_s"], c3["w2"], c3["w2_s"], 8)
    w13k, w2k = torch.ops.strix.weight8_kmajor(c3["w13"]), torch.ops.strix.weight8_kmajor(c3["w2"])
    assert w13k.shape == (128, 16, 1536, 128) and w2k.shape == (128, 6, 2048, 128)
    got = functional.fused_moe_fp8_w8a8(x, logits, w13k, c3["w13_s"], w2k, c3["w2_s"], 8)
    assert torch.equal(got, want)


@pytest.mark.parametrize("t", [1, 3, 15, 16, 17, 64, 300])
@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float16])
def test_route_align_quant_matches_separate_ops(t, xdtype):
    # Up to 16 tokens one kernel routes, aligns and quantizes (idle waves
    # quantize while the router runs; all waves after the align at 16); above,
    # the separate kernels run. Either way: the same bits as the two ops.
    g = torch.Generator().manual_seed(100 + t)
    logits = torch.randn(t, 128, generator=g).to(DEV)
    x = (torch.randn(t, 2048, generator=g) * 3).to(xdtype).to(DEV)
    if t > 2:
        x[1, 256:384] = 0  # an all-zero group takes scale 1
    got = torch.ops.strix.moe_route_align_quant(logits, x, 8, 16)
    want = torch.ops.strix.moe_route_align(logits, 8, 16) + torch.ops.strix.fp8_quant_group128(x)
    for a, b in zip(got, want):
        if a.dtype == torch.float8_e4m3fn:
            a, b = a.view(torch.uint8), b.view(torch.uint8)
        assert torch.equal(a, b)


@pytest.mark.parametrize("t", [1, 37, 64, 65, 128, 200])
def test_align_quant_matches_separate_ops(t):
    # Up to 1024 slots and 64 tokens the single-block align also quantizes the
    # tokens; above, the separate kernels run. The same bits either way.
    g = torch.Generator().manual_seed(200 + t)
    ids = torch.stack([torch.randperm(128, generator=g)[:8] for _ in range(t)]).to(torch.int32).to(DEV)
    x = (torch.randn(t, 2048, generator=g) * 2).to(torch.bfloat16).to(DEV)
    got = torch.ops.strix.moe_align_quant(ids, x, 128, 16)
    want = torch.ops.strix.moe_align(ids, 128, 16) + torch.ops.strix.fp8_quant_group128(x)
    for a, b in zip(got, want):
        if a.dtype == torch.float8_e4m3fn:
            a, b = a.view(torch.uint8), b.view(torch.uint8)
        assert torch.equal(a, b)
