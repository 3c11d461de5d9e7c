# SPDX-License-Identifier: MIT
"""MoE references of the oracle (CPU). Test infrastructure only."""

from __future__ import annotations

import torch
import torch.nn.functional as F

from oracle.quant import fp8_quant_group128


def route_topk(logits: torch.Tensor, top_k: int, renormalize: bool = True):
    """softmax (fp32) -> top-k -> optional renormalize (vLLM fused_topk, the
    router the reference calls at python/strix_vllm/moe.py:181-184; BASELINE
    configs 3-5). Ids are ordered by logit, larger first, ties to the lower
    expert id (a stable sort of -logit), which is the top-k of the softmax
    since softmax is monotone. Pinned by: tests/test_oracle_moe.py (torch.topk
    on tie-free inputs, hand-made ties, weights summing to 1)."""
    lf = logits.detach().to("cpu", torch.float32)
    probs = torch.softmax(lf, dim=-1)
    order = torch.sort(-lf, dim=-1, stable=True).indices[:, :top_k]
    w = torch.gather(probs, 1, order)
    if renormalize:
        w = w / w.sum(dim=-1, keepdim=True)
    return order.to(torch.int32), w


def align(topk_ids: torch.Tensor, block_m: int, num_experts: int):
    """moe_align_block_size's contract as the reference's tests restate it
    (tests/test_moe_gemm.py:9-31): slot ids grouped by expert in ascending
    expert order, ascending within an expert, each run padded to a multiple
    of block_m with the id T*top_k. Returns (sorted_ids, expert_ids, total)
    as python lists without the reference test's spare tail block. Pinned by:
    tests/test_oracle_moe.py (brute-force invariants: every slot exactly
    once, block experts, padding counts)."""
    flat = topk_ids.detach().to("cpu").flatten()
    pad = flat.numel()
    sorted_ids: list[int] = []
    expert_ids: list[int] = []
    for e in range(num_experts):
        ids = (flat == e).nonzero().flatten().tolist()
        if not ids:
            continue
        ids += [pad] * (-len(ids) % block_m)
        sorted_ids += ids
        expert_ids += [e] * (len(ids) // block_m)
    return sorted_ids, expert_ids, len(sorted_ids)


def moe_expert_gemm(a, b, topk_ids, top_k, weights=None):
    """Per-expert loop (tests/test_moe_gemm.py:34-42): out[slot] =
    a[slot // top_k] @ b[expert(slot)]^T in fp32, times the slot's top-k
    weight when given. `b` is the dequantized expert stack [E, N, K]."""
    flat = topk_ids.detach().to("cpu").flatten().long()
    af = a.detach().to("cpu").float()
    bf = b.detach().to("cpu").float()
    out = torch.zeros(flat.numel(), bf.size(1))
    for e in flat.unique().tolist():
        slots = (flat == e).nonzero().flatten()
        out[slots] = af[slots // top_k] @ bf[e].t()
    if weights is not None:
        out = out * weights.detach().to("cpu").float().flatten()[:, None]
    return out


def moe_sum(y: torch.Tensor, top_k: int) -> torch.Tensor:
    """out[t] = sum_j y[t*k + j] (vLLM moe_sum, python/strix_vllm/moe.py:328-330),
    fp32 in slot order."""
    yf = y.detach().to("cpu").float()
    t = yf.size(0) // top_k
    acc = torch.zeros(t, yf.size(1))
    for j in range(top_k):
        acc = acc + yf[j::top_k]
    return acc


def _act(g: torch.Tensor, activation: str) -> torch.Tensor:
    return F.silu(g) if activation == "silu" else F.gelu(g, approximate="tanh")


def fused_moe(x, topk_ids, topk_w, w13, w2, activation="silu", act_quant=None, tokens=None):
    """Fused MoE reference: per routed (token, slot)
    h = x_t @ w13[e]^T, inter = act(h[:I]) * h[I:], y = inter @ w2[e]^T,
    out_t = sum_j w_tj y_tj. `w13`/`w2` are dequantized fp32 expert stacks.
    act_quant="fp8" applies the kernel path's activation QDQ: x per 1x128
    group to e4m3 before w13, and the bf16 intermediate per 1x128 group
    before w2 (python/strix_vllm/moe.py:963-1014 is the reference's chain;
    the W8A8 QDQ is BASELINE's). The w2 outputs are rounded to bf16 before
    the sum, as the kernel chain stores them. `tokens` restricts the output
    to those token rows (returns [len(tokens), H]). Pinned by:
    tests/test_oracle_moe.py (against moe_expert_gemm + moe_sum composed
    by hand on a small case)."""
    xf = x.detach().to("cpu").float()
    ids = topk_ids.detach().to("cpu").long()
    tw = topk_w.detach().to("cpu").float()
    rows = torch.arange(xf.size(0)) if tokens is None else torch.as_tensor(tokens).long()
    k = ids.size(1)
    if act_quant == "fp8":
        q, s = fp8_quant_group128(x.detach().to("cpu")[rows])
        xa = q.float() * s.repeat_interleave(128, dim=1)
    else:
        xa = xf[rows]
    sub_ids = ids[rows]
    # Expert weights: a stacked tensor [E, N, K] or a callable e -> fp32 [N, K]
    # (which dequantizes one expert at a time for the large configs).
    get13 = w13 if callable(w13) else (lambda e: w13[e])
    get2 = w2 if callable(w2) else (lambda e: w2[e])
    out = None
    pairs_t = torch.arange(rows.numel()).repeat_interleave(k)
    pairs_e = sub_ids.flatten()
    pairs_w = tw[rows].flatten()
    for e in pairs_e.unique().tolist():
        sel = (pairs_e == e).nonzero().flatten()
        t = pairs_t[sel]
        w13e = get13(e).float()
        inter_dim = w13e.size(0) // 2
        h = xa[t] @ w13e.t()
        inter = (_act(h[:, :inter_dim], activation) * h[:, inter_dim:]).to(torch.bfloat16)
        if act_quant == "fp8":
            q, s = fp8_quant_group128(inter)
            ia = q.float() * s.repeat_interleave(128, dim=1)
        else:
            ia = inter.float()
        y = (ia @ get2(e).float().t()) * pairs_w[sel][:, None]
        if out is None:
            out = torch.zeros(rows.numel(), y.size(1))
        out.index_add_(0, t, y.to(torch.bfloat16).float())
    return out
