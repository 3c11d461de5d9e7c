# SPDX-License-Identifier: MIT
"""Pins the oracle's MoE references (CPU only)."""

import torch

import oracle


def test_route_matches_torch_topk_without_ties():
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(50, 128, generator=g)
    ids, w = oracle.route_topk(logits, 8, renormalize=True)
    p = torch.softmax(logits, -1)
    tv, ti = torch.topk(p, 8, dim=-1)
    assert torch.equal(ids.long(), ti)
    assert torch.allclose(w, tv / tv.sum(-1, keepdim=True), rtol=1e-6, atol=0)
    assert torch.allclose(w.sum(-1), torch.ones(50), atol=1e-6)


def test_route_ties_prefer_lower_expert_id():
    logits = torch.tensor([[0.0, 2.0, 1.0, 2.0, 1.0, -1.0]])
    ids, w = oracle.route_topk(logits, 4, renormalize=False)
    assert ids.tolist() == [[1, 3, 2, 4]]
    p = torch.softmax(logits, -1)[0]
    assert torch.allclose(w[0], p[[1, 3, 2, 4]])


def test_align_invariants_brute_force():
    g = torch.Generator().manual_seed(1)
    t, k, e, bm = 37, 4, 16, 8
    ids = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(t)]).to(torch.int32)
    sorted_ids, expert_ids, total = oracle.align(ids, bm, e)
    pad = t * k
    assert total % bm == 0 and len(expert_ids) * bm == total
    real = [s for s in sorted_ids if s != pad]
    assert sorted(real) == list(range(t * k))  # every slot exactly once
    flat = ids.flatten().tolist()
    for b, ex in enumerate(expert_ids):
        blk = sorted_ids[b * bm:(b + 1) * bm]
        assert all(s == pad or flat[s] == ex for s in blk)
    assert expert_ids == sorted(expert_ids)
    # within an expert: ascending slot order, padding only at the end of a run
    for ex in set(expert_ids):
        run = [s for b, x in enumerate(expert_ids) if x == ex for s in sorted_ids[b * bm:(b + 1) * bm]]
        live = [s for s in run if s != pad]
        assert live == sorted(live) and run[:len(live)] == live
        assert len(run) - len(live) == (-len(live)) % bm


def test_fused_moe_matches_hand_composition():
    g = torch.Generator().manual_seed(2)
    t, e, k, h, i = 5, 6, 2, 32, 16
    x = torch.randn(t, h, generator=g).to(torch.bfloat16)
    w13 = torch.randn(e, 2 * i, h, generator=g) * 0.1
    w2 = torch.randn(e, h, i, generator=g) * 0.1
    ids, w = oracle.route_topk(torch.randn(t, e, generator=g), k)
    out = oracle.fused_moe(x, ids, w, w13, w2)
    hcat = oracle.moe_expert_gemm(x, w13, ids, k)
    inter = (torch.nn.functional.silu(hcat[:, :i]) * hcat[:, i:]).to(torch.bfloat16)
    y = oracle.moe_expert_gemm(inter, w2, ids, 1, w).to(torch.bfloat16)
    ref = oracle.moe_sum(y, k)
    assert torch.allclose(out, ref, rtol=1e-5, atol=1e-5)
    sub = oracle.fused_moe(x, ids, w, w13, w2, tokens=[1, 3])
    assert torch.allclose(sub, ref[[1, 3]], rtol=1e-5, atol=1e-5)


def test_moe_sum_slot_order():
    y = torch.arange(12, dtype=torch.float32).reshape(6, 2)
    assert oracle.moe_sum(y, 3).tolist() == [[0 + 2 + 4, 1 + 3 + 5], [6 + 8 + 10, 7 + 9 + 11]]
