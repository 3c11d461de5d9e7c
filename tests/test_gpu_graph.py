# SPDX-License-Identifier: MIT
"""HIP graph capture of the hot path: a captured decode step (FP8 dense
linear, fused FP8 MoE with routing and alignment, fused MXFP4 MoE) replayed
several times, with other eager work and synchronizations between replays,
must give the eager result bit for bit on every replay (every kernel here is
deterministic). The reference's microbenchmarks time graph replays
(bench/kernels/w8a8_gemm.py:41-58), and vLLM captures its decode steps."""

import pytest
import torch

import libstrix_amd  # noqa: F401
from libstrix_amd import functional, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
S = torch.ops.strix


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def _replays_match(fn, eager):
    g, out = _capture(fn)
    for r in range(3):
        junk = torch.randn(1 << 20, device=DEV).sum()   # eager work between replays
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r} differs from the eager result"
        del junk


def test_dense_fp8_decode_graph():
    d = workloads.c2_fp8(seed=2, m=4, n=4096, k=5120, device=DEV)
    fn = lambda: S.fp8_w8a8_block_gemm(*S.fp8_quant_group128(d["x"]), d["w"], d["sw"])
    _replays_match(fn, fn().clone())


@pytest.mark.parametrize("t", [1, 64])
def test_fused_moe_fp8_graph(t):
    c3 = workloads.c3_fp8_moe(seed=3, t=t, device=DEV)
    logits = torch.randn(t, 128, generator=torch.Generator().manual_seed(t)).to(DEV)
    x = torch.randn(t, 2048, generator=torch.Generator().manual_seed(t + 1)).to(torch.bfloat16).to(DEV)
    fn = lambda: functional.fused_moe_fp8_w8a8(x, logits, c3["w13"], c3["w13_s"], c3["w2"], c3["w2_s"], 8)
    _replays_match(fn, fn().clone())


def test_fused_moe_mxfp4_graph():
    c4 = workloads.c4_mxfp4_moe(seed=4, t=1, device=DEV)
    logits = torch.randn(2, 32, generator=torch.Generator().manual_seed(5)).to(DEV)
    x = torch.randn(2, 2880, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(DEV)
    fn = lambda: functional.fused_moe_mxfp4(x, logits, c4["w13"], c4["w13_s"], c4["w2"], c4["w2_s"], 4)
    _replays_match(fn, fn().clone())


@pytest.mark.parametrize("t", [1, 64])
def test_plugin_fp8_experts_graph(t):
    # The plugin's FP8 expert chain (quantize, align, both GEMMs, combine)
    # captured as vLLM captures its decode step: every replay equals eager.
    from libstrix_amd.vllm_plugin import moe

    c3 = workloads.c3_fp8_moe(seed=7, t=1, device=DEV)
    g = torch.Generator().manual_seed(t + 9)
    ids = torch.stack([torch.randperm(128, generator=g)[:8] for _ in range(t)]).to(torch.int32).to(DEV)
    tw = torch.rand(t, 8, generator=g).to(DEV)
    x = torch.randn(t, 2048, generator=g).to(torch.bfloat16).to(DEV)
    fn = lambda: moe.fp8_experts(None, x, c3["w13"], c3["w2"], c3["w13_s"], c3["w2_s"], tw, ids, "silu")
    _replays_match(fn, fn().clone())
