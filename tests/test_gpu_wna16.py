# SPDX-License-Identifier: MIT
"""WNA16 int4 experts: the reference's symmetric moe_gemm_w4a16
(tests/test_moe_wna16.py pattern) and the zero-point variant of BASELINE
config 5 (AWQ-style uint4 + bf16 scales + uint4 zero points, group 128)."""

import pytest
import torch

import libstrix_amd  # noqa: F401
import oracle
from conftest import peak_rel_err
from libstrix_amd import functional, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-2


def _ref(a, deq, ids, a_topk, weights, gemm, activation, cols):
    ref = oracle.moe_expert_gemm(a, deq, ids, a_topk, weights)
    if gemm == "w13":
        g_, u_ = ref[:, :cols], ref[:, cols:]
        act = torch.nn.functional.silu(g_) if activation == "silu" else torch.nn.functional.gelu(g_, approximate="tanh")
        ref = act * u_
    return ref


E, TOPK = 16, 8


@pytest.fixture(scope="module")
def zp_experts():
    return workloads.c5_wna16_moe(seed=51, t=1, e=E)


@pytest.mark.parametrize("tokens", [1, 5, 40, 300])
@pytest.mark.parametrize("block_m", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("gemm,activation", [("w13", "silu"), ("w13", "gelu_tanh"), ("w2", "silu")])
def test_zp_expert_gemm(tokens, block_m, gemm, activation, zp_experts):
    d = zp_experts
    g = torch.Generator().manual_seed(tokens * 7 + block_m)
    ids = torch.stack([torch.randperm(E, generator=g)[:TOPK] for _ in range(tokens)]).to(torch.int32)
    key = "w13" if gemm == "w13" else "w2"
    w, s, z = d[key], d[key + "_s"], d[key + "_z"]
    n, k = w.size(1), w.size(2) * 8
    if gemm == "w13":
        a = torch.randn(tokens, k, generator=g).to(torch.bfloat16)
        a_topk, weights, cols = TOPK, None, n // 2
    else:
        a = torch.randn(tokens * TOPK, k, generator=g).to(torch.bfloat16)
        a_topk, weights, cols = 1, torch.rand(tokens, TOPK, generator=g), n
    sorted_ids, expert_ids, num_post = torch.ops.strix.moe_align(ids.to(DEV), E, block_m)
    c = torch.full((tokens * TOPK, cols), float("nan"), dtype=torch.bfloat16, device=DEV)
    torch.ops.strix.moe_gemm_w4a16_zp(c, a.to(DEV), w.to(DEV), s.to(DEV), z.to(DEV), sorted_ids, expert_ids, num_post,
                                      None if weights is None else weights.reshape(-1).to(DEV), a_topk, block_m, 64,
                                      gemm == "w13", activation, 128)
    deq = oracle.wna16_zp_decode(w, s, z, 128)
    assert not torch.isnan(c).any()
    assert peak_rel_err(c, _ref(a, deq, ids, a_topk, weights, gemm, activation, cols)) <= TOL


@pytest.mark.parametrize("tokens", [1, 5, 40])
@pytest.mark.parametrize("gemm", ["w13", "w2"])
def test_zp_expert_gemm_fp16_activations(tokens, gemm, zp_experts):
    """fp16 tokens and output through the decode paths (block_m 16), whose
    folded int4 decode feeds the codes to the fp16 MFMA as 1024 + q."""
    d = zp_experts
    g = torch.Generator().manual_seed(tokens + 991)
    ids = torch.stack([torch.randperm(E, generator=g)[:TOPK] for _ in range(tokens)]).to(torch.int32)
    w, s, z = d[gemm], d[gemm + "_s"], d[gemm + "_z"]
    n, k = w.size(1), w.size(2) * 8
    if gemm == "w13":
        a = torch.randn(tokens, k, generator=g).to(torch.float16)
        a_topk, weights, cols = TOPK, None, n // 2
    else:
        a = torch.randn(tokens * TOPK, k, generator=g).to(torch.float16)
        a_topk, weights, cols = 1, torch.rand(tokens, TOPK, generator=g), n
    sorted_ids, expert_ids, num_post = torch.ops.strix.moe_align(ids.to(DEV), E, 16)
    c = torch.full((tokens * TOPK, cols), float("nan"), dtype=torch.float16, device=DEV)
    torch.ops.strix.moe_gemm_w4a16_zp(c, a.to(DEV), w.to(DEV), s.to(DEV), z.to(DEV), sorted_ids, expert_ids, num_post,
                                      None if weights is None else weights.reshape(-1).to(DEV), a_topk, 16, 64,
                                      gemm == "w13", "silu", 128)
    deq = oracle.wna16_zp_decode(w, s, z, 128)
    assert not torch.isnan(c).any()
    assert peak_rel_err(c, _ref(a, deq, ids, a_topk, weights, gemm, "silu", cols)) <= TOL


# Reference shapes: tests/test_moe_wna16.py:14-20 (gemma group 32, qfn group 128).
@pytest.mark.parametrize("model", [(32, 8, 32, (1408, 2816), (2816, 704)), (16, 10, 128, (1280, 2560), (2560, 640))])
@pytest.mark.parametrize("tokens", [1, 5, 70])
@pytest.mark.parametrize("block_m", [16, 64, 128])
@pytest.mark.parametrize("gemm,activation", [("w13", "silu"), ("w13", "gelu_tanh"), ("w2", "silu")])
@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float16])
def test_sym_matches_reference(model, tokens, block_m, gemm, activation, scale_dtype):
    e, top_k, group, w13, w2 = model
    n, k = w13 if gemm == "w13" else w2
    g = torch.Generator().manual_seed(tokens + block_m)
    q = torch.randint(0, 16, (e, n, k), generator=g, dtype=torch.uint8)
    w_u8 = (q[..., 0::2] | (q[..., 1::2] << 4)).contiguous()
    scales = (torch.rand(e, n, k // group, generator=g) * 0.02 + 0.001).to(scale_dtype)
    ids = torch.stack([torch.randperm(e, generator=g)[:top_k] for _ in range(tokens)]).to(torch.int32)
    if gemm == "w13":
        a = torch.randn(tokens, k, generator=g).to(torch.bfloat16)
        a_topk, weights, cols = top_k, None, n // 2
    else:
        a = torch.randn(tokens * top_k, k, generator=g).to(torch.bfloat16)
        a_topk, weights, cols = 1, torch.rand(tokens, top_k, generator=g), n
    sorted_ids, expert_ids, num_post = torch.ops.strix.moe_align(ids.to(DEV), e, block_m)
    c = torch.full((tokens * top_k, cols), float("nan"), dtype=torch.bfloat16, device=DEV)
    torch.ops.strix.moe_gemm_w4a16(c, a.to(DEV), w_u8.to(DEV), scales.to(DEV), sorted_ids, expert_ids, num_post,
                                   None if weights is None else weights.reshape(-1).to(DEV), a_topk, block_m, 64,
                                   gemm == "w13", activation, group)
    deq = oracle.wna16_sym_decode(w_u8, scales, group)
    assert not torch.isnan(c).any()
    assert peak_rel_err(c, _ref(a, deq, ids, a_topk, weights, gemm, activation, cols)) <= TOL


@pytest.fixture(scope="module")
def c5_weights():
    d = workloads.c5_wna16_moe(seed=5, t=1)
    dev = {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in d.items()}
    return d, dev


@pytest.mark.parametrize("t", [1, 64, 8192])
def test_config5_fused_moe(t, c5_weights):
    d, dev = c5_weights
    g = torch.Generator().manual_seed(500 + t)
    x = torch.randn(t, 2048, generator=g).to(torch.bfloat16)
    logits = torch.randn(t, 128, generator=g)
    out = functional.fused_moe_wna16(x.to(DEV), logits.to(DEV), dev["w13"], dev["w13_s"], dev["w13_z"], dev["w2"],
                                     dev["w2_s"], dev["w2_z"], 8, 128)
    ids, w = oracle.route_topk(logits, 8)
    # Every token row is checked.
    ref = oracle.fused_moe(x, ids, w,
                           lambda e: oracle.wna16_zp_decode(d["w13"][e], d["w13_s"][e], d["w13_z"][e], 128),
                           lambda e: oracle.wna16_zp_decode(d["w2"][e], d["w2_s"][e], d["w2_z"][e], 128))
    assert ref.shape == out.shape
    assert peak_rel_err(out, ref) <= TOL


def test_empty_sorted_ids_writes_nothing(zp_experts):
    """No routed positions at all (sorted_ids empty, one expert block): the
    call returns without touching the output (the kernels' row lookups
    assume a non-empty sorted_ids, so the launcher stops first)."""
    d = zp_experts
    w, s, z = d["w13"], d["w13_s"], d["w13_z"]
    n, k = w.size(1), w.size(2) * 8
    a = torch.randn(3, k).to(torch.bfloat16).to(DEV)
    c = torch.full((3 * TOPK, n // 2), 7.0, dtype=torch.bfloat16, device=DEV)
    sorted_ids = torch.empty(0, dtype=torch.int32, device=DEV)
    expert_ids = torch.zeros(1, dtype=torch.int32, device=DEV)
    num_post = torch.zeros(1, dtype=torch.int32, device=DEV)
    for block_m in (16, 256):
        torch.ops.strix.moe_gemm_w4a16_zp(c, a, w.to(DEV), s.to(DEV), z.to(DEV), sorted_ids, expert_ids, num_post,
                                          None, TOPK, block_m, 64, True, "silu", 128)
    torch.cuda.synchronize()
    assert bool((c == 7.0).all())
