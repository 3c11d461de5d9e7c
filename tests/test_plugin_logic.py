# SPDX-License-Identifier: MIT
"""The vLLM plugin's host logic on the CPU, without vLLM: environment gates,
compile-cache key, tile tables, eligibility checks, load-time weight
transforms, and which ops each per-forward dispatcher calls at which M (the
op namespace is swapped for a recorder). The reference's plugin is exercised
the same way, through its module functions (python/strix_vllm/*.py); vLLM's
own kernel-selection hooks need vLLM and are not run here."""

from __future__ import annotations

import importlib

import pytest
import torch

import libstrix_amd.vllm_plugin as plugin
from libstrix_amd.vllm_plugin import fp8, int8, linear, moe, mxfp4


class Recorder:
    """Stands in for torch.ops.strix: records each call, returns CPU tensors of the op's output shape."""

    def __init__(self):
        self.calls: list[str] = []
        self.args: list[tuple] = []

    def _rec(self, name, args):
        self.calls.append(name)
        self.args.append(args)

    def __getattr__(self, name):
        def op(*args):
            self._rec(name, args)
            return _OUT.get(name, lambda *a: None)(*args)

        return op


_OUT = {
    "int8_quant_per_token": lambda x: (torch.zeros(x.shape, dtype=torch.int8), torch.ones(x.size(0))),
    "w8a8_scaled_mm": lambda q, s, w, sw: torch.zeros(q.size(0), w.size(0), dtype=torch.bfloat16),
    "fp8_quant_group128": lambda x: (torch.zeros(x.shape), torch.ones(x.size(0), x.size(1) // 128)),
    "fp8_w8a8_block_gemm": lambda q, s, w, sw: torch.zeros(q.size(0), w.size(0), dtype=torch.bfloat16),
    "fp8_w8a8_block_gemm_kmajor": lambda q, s, w, sw: torch.zeros(q.size(0), w.size(1), dtype=torch.bfloat16),
    "weight8_kmajor": lambda w: w.view(w.size(0), -1, 128).permute(1, 0, 2).contiguous(),
    "fp8_dequant": lambda w, s: torch.zeros(w.shape, dtype=torch.bfloat16),
    "fp8_wmma_gemm": lambda w, x, s: torch.zeros(x.size(0), w.size(0), dtype=torch.bfloat16),
    "mxfp4_gemv": lambda x, w, s: torch.zeros(x.size(0), w.size(0), dtype=torch.bfloat16),
    "mxfp4_dequant": lambda w, s: torch.zeros(w.size(0), 2 * w.size(1), dtype=torch.bfloat16),
    "mxfp4_wmma_gemm": lambda w, x, s, b: torch.zeros(x.size(0), w.size(0), dtype=torch.bfloat16),
    "w8a16_skinny_gemm": lambda w, x, s, b, cu, g: torch.zeros(x.size(0), w.size(0), dtype=x.dtype),
    "w8a8_wmma_gemm": lambda w, x, s: torch.zeros(x.size(0), w.size(0), dtype=x.dtype),
    "w4a16_dequant": lambda w, s, g: torch.zeros(w.size(0), 2 * w.size(1), dtype=torch.bfloat16),
    "w4a16_wmma_gemm": lambda x, w, s, b, g: torch.zeros(x.size(0), w.size(0), dtype=torch.bfloat16),
    "moe_align": lambda ids, e, bm: (torch.zeros(64, dtype=torch.int32), torch.zeros(4, dtype=torch.int32),
                                     torch.zeros(1, dtype=torch.int32)),
    "moe_align_quant": lambda ids, x, e, bm: (torch.zeros(64, dtype=torch.int32), torch.zeros(4, dtype=torch.int32),
                                              torch.zeros(1, dtype=torch.int32), torch.zeros(x.shape),
                                              torch.ones(x.size(0), x.size(1) // 128)),
}


@pytest.fixture
def rec(monkeypatch):
    r = Recorder()
    for mod in (int8, fp8, mxfp4, linear, moe):
        monkeypatch.setattr(mod, "S", r)
    return r


@pytest.fixture
def clean_env(monkeypatch):
    monkeypatch.delenv("STRIX_DISABLE", raising=False)
    monkeypatch.delenv("STRIX_ENABLE", raising=False)
    return monkeypatch


# ------------------------------------------------------------------ environment
def test_disabled_parses_all_and_lists(clean_env):
    assert not plugin.disabled("fp8")
    clean_env.setenv("STRIX_DISABLE", " fp8 , moe_w4a16")
    assert plugin.disabled("fp8") and plugin.disabled("moe_w4a16") and not plugin.disabled("fp8_channel")
    clean_env.setenv("STRIX_DISABLE", "all")
    assert plugin.disabled("anything")


def test_model_gate_needs_enable_or_listed_arch(clean_env):
    assert not plugin.model_gate("moe_w4a8", archs=["SomeModel"])
    clean_env.setenv("STRIX_ENABLE", "moe_w4a8")
    assert plugin.model_gate("moe_w4a8", archs=[]) and plugin.enabled("moe_w4a8")
    clean_env.setenv("STRIX_DISABLE", "moe_w4a8")
    assert not plugin.model_gate("moe_w4a8", archs=[]) and not plugin.enabled("moe_w4a8")
    clean_env.delenv("STRIX_ENABLE")
    clean_env.delenv("STRIX_DISABLE")
    clean_env.setitem(plugin.ARCH_GATED, "moe_w4a8", ("Listed",))
    assert plugin.model_gate("moe_w4a8", archs=["Listed"])


def test_cache_factor_tracks_activity_and_env(clean_env):
    a, b = plugin._cache_factor(True), plugin._cache_factor(False)
    assert len(a) == 16 and a != b and a == plugin._cache_factor(True)
    clean_env.setenv("STRIX_DISABLE", "fp8")
    assert plugin._cache_factor(True) != a


def test_not_on_gfx950_without_a_gpu():
    assert not plugin.on_gfx950()


def test_register_needs_vllm(clean_env, monkeypatch):
    try:
        importlib.import_module("vllm")
        pytest.skip("vLLM is installed: register() is exercised by vLLM itself")
    except ImportError:
        pass
    monkeypatch.setattr(plugin, "_registered", False)
    with pytest.raises(ImportError):
        plugin.register()
    assert plugin._registered  # one attempt per process, as the entry point may run more than once
    plugin.register()           # idempotent: a second call returns at once


# ------------------------------------------------------------------ tile tables and gates
def test_block_m_by_rows_per_expert():
    # config 3 (E=128, top-8): decode rides the 16-row ring, prefill the 256 tile
    assert moe.fp8_blocks(1) == (16, 128)
    assert moe.fp8_blocks(64)[0] == 16
    assert moe.fp8_blocks(4096)[0] == 256
    assert moe.fp8_blocks(1024)[0] == 128
    # config 4 (E=32, top-4): 2048 tokens = 256 rows per expert
    assert moe.strix_blocks(2048, 4, 32) == (256, 64)
    prev = 0
    for t in (1, 2, 8, 64, 128, 512, 700, 1024, 4096, 65536):
        bm = moe.strix_blocks(t, 8, 128)[0]
        assert bm in (16, 32, 64, 128, 256) and bm >= prev
        prev = bm
    assert moe.wna16_blocks(8192, 1536, 2048) == moe.strix_blocks(8192)
    assert moe.fp8_raw_blocks(300) == moe.strix_blocks(300)


def test_block_n_divides_both_gemms():
    assert moe._block_n(1536, 2048) == 128
    assert moe._block_n(5760, 2880) == 64


def test_strix_moe_ok_and_w4a8_gate(clean_env):
    assert moe.strix_moe_ok(1, 1536, 2048)
    clean_env.setitem(moe._MIN_ROWS, (1408, 2816), 3)
    assert not moe.strix_moe_ok(2, 1408, 2816) and moe.strix_moe_ok(3, 1408, 2816)
    assert moe._w4a8_ok(4096, 128, 1536, 2048)
    assert not moe._w4a8_ok(16, 128, 1536, 2048)
    assert not moe._w4a8_ok(4096, 32, 1536, 2048)
    assert not moe._w4a8_ok(4096, 128, 1500, 2048)
    clean_env.setenv("STRIX_DISABLE", "moe_w4a8")
    assert not moe._w4a8_ok(4096, 128, 1536, 2048)


def test_fp8_moe_eligibility_names_each_failure():
    e, n, k = 4, 256, 512
    w1 = torch.empty(e, n, k, dtype=torch.float8_e4m3fn)
    w2 = torch.empty(e, k, n // 2, dtype=torch.float8_e4m3fn)
    s1 = torch.ones(e, n // 128, k // 128)
    s2 = torch.ones(e, k // 128, n // 2 // 128)
    x = torch.empty(3, k, dtype=torch.bfloat16)
    assert moe.fp8_bad(x, w1, w2, s1, s2, [128, 128], "silu", None) == []
    assert moe.fp8_bad(x, w1, w2, s1, s2, [128, 128], "relu", None) == ["activation"]
    assert moe.fp8_bad(x, w1, w2, s1[:, :1], s2, [128, 128], "silu", None) == ["scales"]
    assert moe.fp8_bad(x, w1, w2, s1, s2, [128, 128], "silu", torch.arange(4)) == ["expert_map"]
    assert "w1_fp8" in moe.fp8_bad(x, w1.view(torch.uint8), w2, s1, s2, [128, 128], "silu", None)
    # per-channel scales: one per (expert, row)
    assert moe.fp8_bad(x, w1, w2, torch.ones(e, n), torch.ones(e, k), None, "gelu_tanh", None) == []


def test_wna16_moe_eligibility():
    e, n, k = 4, 256, 512
    w1 = torch.empty(e, n, k // 2, dtype=torch.uint8)
    w2 = torch.empty(e, k, n // 4, dtype=torch.uint8)
    s1 = torch.ones(e, n, k // 128, dtype=torch.bfloat16)
    s2 = torch.ones(e, k, n // 2 // 128, dtype=torch.bfloat16)
    x = torch.empty(3, k, dtype=torch.bfloat16)
    assert moe.wna16_bad(x, w1, w2, s1, s2, 128, "silu", None) == []
    assert moe.wna16_bad(x, w1, w2, s1, s2, 16, "silu", None) == ["group"]
    assert moe.wna16_bad(x, w1, w2, s1, s2, 128, "silu", None, has_zp=True) == ["zero_point"]
    assert moe.wna16_bad(x.half(), w1, w2, s1, s2, 128, "silu", None) == ["act_dtype"]


def test_bf16_moe_gate():
    w1 = torch.empty(4, 256, 512, dtype=torch.bfloat16)
    w2 = torch.empty(4, 512, 128, dtype=torch.bfloat16)
    x = torch.empty(3, 512, dtype=torch.bfloat16)
    assert moe.bf16_ok(x, w1, w2, "silu", None)
    assert not moe.bf16_ok(x, w1, w2, "silu", None, quantized=True)
    assert not moe.bf16_ok(x.half(), w1, w2, "silu", None)


# ------------------------------------------------------------------ load-time transforms
def test_int8_prepare_keeps_rows_and_broadcasts_scale():
    w = torch.randint(-128, 128, (64, 256), dtype=torch.int8)
    w2, s = int8.prepare_weights(w, torch.tensor([0.5]))
    assert w2.data_ptr() == w.data_ptr() and s.shape == (64,) and (s == 0.5).all() and s.dtype == torch.float32
    wt, _ = int8.prepare_weights(w.t().contiguous().t(), torch.ones(64, 1))   # a [N, K] view of [K, N] storage
    assert torch.equal(wt, w) and wt.stride(1) == 1 and wt.shape == (64, 256)
    with pytest.raises(RuntimeError, match="signed int8"):
        int8.prepare_weights(w.view(torch.uint8), torch.ones(64))
    with pytest.raises(RuntimeError, match="per-channel scale"):
        int8.prepare_weights(w, torch.ones(3))
    assert int8.can_implement(False, True)[0]
    assert int8.can_implement(True, True) == (False, "strix W8A8 takes dynamic per-token activations")


def test_fp8_prepare_and_gates():
    w = torch.zeros(300, 256, dtype=torch.float8_e4m3fn)
    w2, bs = fp8.prepare_block(w, torch.ones(3, 2, dtype=torch.bfloat16))
    assert bs.dtype == torch.float32 and bs.shape == (3, 2)
    with pytest.raises(RuntimeError, match="block scales"):
        fp8.prepare_block(w, torch.ones(2, 2))
    wc, s = fp8.prepare_channel(w.t(), torch.ones(300, 1), 300)
    assert wc.shape == (300, 256) and wc.is_contiguous() and s.shape == (300,)
    assert fp8.can_implement_block((128, 128), torch.bfloat16, 5120) == (True, None)
    assert not fp8.can_implement_block((1, 128), torch.bfloat16, 5120)[0]
    assert not fp8.can_implement_block((128, 128), torch.bfloat16, 5000)[0]
    assert fp8.can_implement_channel(torch.float8_e4m3fn, True, None, 704) == (True, None)
    assert not fp8.can_implement_channel(torch.float8_e4m3fn, True, None, 700)[0]


def test_mxfp4_weight_checks():
    mxfp4.check_weights(torch.zeros(8, 64, dtype=torch.uint8), torch.zeros(8, 4, dtype=torch.uint8))
    with pytest.raises(ValueError, match="multiple of 128"):
        mxfp4.check_weights(torch.zeros(8, 48, dtype=torch.uint8), torch.zeros(8, 3, dtype=torch.uint8))
    with pytest.raises(ValueError, match="weight_scale"):
        mxfp4.check_weights(torch.zeros(8, 64, dtype=torch.uint8), torch.zeros(8, 4, dtype=torch.float32))
    assert not mxfp4.can_implement(True, torch.float16)[0]


def test_w8a8_scales_layout_and_cache():
    linear._W8A8_PREP.clear()
    w = torch.zeros(64, 256, dtype=torch.uint8)
    s = torch.rand(64, 2, dtype=torch.bfloat16)
    g = linear.w8a8_scales(w, s, 128)
    assert g.shape == (2, 64) and torch.equal(g, s.float().t())
    assert linear.w8a8_scales(w, s, 128) is g                  # cached per weight
    linear._W8A8_PREP.clear()
    assert linear.w8a8_scales(w, torch.rand(64, 1), 0).shape == (64,)
    assert linear.w8a8_scales(torch.zeros(64, 256, dtype=torch.uint8), torch.rand(64, 8), 32) is None
    assert torch.equal(linear.pack_w8_rows(torch.tensor([[0, 255, 256 + 7]])), torch.tensor([[0, 255, 7]],
                                                                                             dtype=torch.uint8))
    assert linear.can_implement_w8("uint8b128", False, torch.bfloat16, 128, 5120) == (True, None)
    assert not linear.can_implement_w8("uint4b8", False, torch.bfloat16, 128, 5120)[0]
    assert linear.can_implement_w4("uint4b8", False, 64, 5120) == (True, None)
    assert not linear.can_implement_w4("uint4b8", True, 64, 5120)[0]


# ------------------------------------------------------------------ per-forward dispatch
def test_int8_dispatch_quantizes_per_token(rec):
    out = int8._apply_impl(torch.zeros(5, 256, dtype=torch.bfloat16), torch.zeros(64, 256, dtype=torch.int8),
                           torch.ones(64), torch.ones(64, dtype=torch.bfloat16))
    assert rec.calls == ["int8_quant_per_token", "w8a8_scaled_mm"] and out.shape == (5, 64)


@pytest.mark.parametrize("m", [1, 16, 4096])
def test_fp8_block_dispatch_is_w8a8_at_every_m(rec, m):
    fp8._apply_impl(torch.zeros(m, 256, dtype=torch.bfloat16), torch.zeros(128, 256), torch.ones(1, 2), None, True)
    assert rec.calls == ["fp8_quant_group128", "fp8_w8a8_block_gemm"]


def test_fp8_block_kmajor_weights(rec):
    # The W8A8 load transform re-lays the weights K-block-major; the forward
    # then calls the K-major GEMM and the output keeps N columns.
    w = torch.zeros(128, 256)
    wk, _ = fp8.prepare_block(w.to(torch.float8_e4m3fn), torch.ones(1, 2), kmajor=True)
    assert rec.calls == ["weight8_kmajor"] and wk.shape == (2, 128, 128) and fp8.out_features(wk) == 128
    out = fp8._apply_impl(torch.zeros(3, 256, dtype=torch.bfloat16), wk, torch.ones(1, 2), None, True)
    assert rec.calls[1:] == ["fp8_quant_group128", "fp8_w8a8_block_gemm_kmajor"] and out.shape == (3, 128)


@pytest.mark.parametrize("m,expect", [(1, "fp8_wmma_gemm"), (fp8.W8A16_DEQUANT_MIN_M - 1, "fp8_wmma_gemm"),
                                      (fp8.W8A16_DEQUANT_MIN_M, "fp8_dequant")])
def test_fp8_w8a16_dispatch(rec, m, expect):
    out = fp8._apply_impl(torch.zeros(m, 256, dtype=torch.bfloat16), torch.zeros(128, 256), torch.ones(128), None,
                          False)
    assert rec.calls == [expect] and out.shape == (m, 128)


@pytest.mark.parametrize("m,bias,expect", [(1, False, "mxfp4_gemv"), (8, False, "mxfp4_gemv"),
                                           (2, True, "mxfp4_wmma_gemm"), (64, False, "mxfp4_wmma_gemm"),
                                           (mxfp4.DEQUANT_MIN_M, False, "mxfp4_dequant")])
def test_mxfp4_dispatch(rec, m, bias, expect):
    b = torch.zeros(32, dtype=torch.bfloat16) if bias else None
    out = mxfp4._apply_impl(torch.zeros(m, 256, dtype=torch.bfloat16), torch.zeros(32, 128, dtype=torch.uint8),
                            torch.zeros(32, 8, dtype=torch.uint8), b)
    assert rec.calls == [expect] and out.shape == (m, 32)


@pytest.mark.parametrize("m,expect", [(1, "w8a16_skinny_gemm"), (8, "w8a16_skinny_gemm"), (9, "w8a8_wmma_gemm")])
def test_w8a16_dispatch(rec, m, expect):
    linear._W8A8_PREP.clear()
    linear._apply_impl(torch.zeros(m, 256, dtype=torch.bfloat16), torch.zeros(64, 256, dtype=torch.uint8),
                       torch.ones(64, 2, dtype=torch.bfloat16), None, 128)
    assert rec.calls == [expect]


def test_w8a16_group32_prefill_raises(rec):
    with pytest.raises(RuntimeError, match="cannot run"):
        linear._apply_impl(torch.zeros(20, 256, dtype=torch.bfloat16), torch.zeros(64, 256, dtype=torch.uint8),
                           torch.ones(64, 8, dtype=torch.bfloat16), None, 32)


@pytest.mark.parametrize("m,expect", [(1, "w4a16_wmma_gemm"), (mxfp4.DEQUANT_MIN_M - 1, "w4a16_wmma_gemm"),
                                      (mxfp4.DEQUANT_MIN_M, "w4a16_dequant")])
def test_w4a16_dispatch(rec, m, expect):
    linear._w4_apply_impl(torch.zeros(m, 256, dtype=torch.bfloat16), torch.zeros(64, 128, dtype=torch.int8),
                          torch.ones(64, 2, dtype=torch.bfloat16), None, 128)
    assert rec.calls == [expect]
    assert rec.args[0][-1] == 128


def test_w4a16_channel_group_is_whole_k(rec):
    linear._w4_apply_impl(torch.zeros(2, 256, dtype=torch.bfloat16), torch.zeros(64, 128, dtype=torch.int8),
                          torch.ones(64, dtype=torch.bfloat16), None, -1)
    assert rec.args[0][-1] == 256 and rec.args[0][2].shape == (64, 1)


# ------------------------------------------------------------------ expert chains
def _moe_inputs(t=3, top_k=2, e=4, h=256, inter=128, dtype=torch.bfloat16):
    x = torch.zeros(t, h, dtype=dtype)
    ids = torch.zeros(t, top_k, dtype=torch.int64)
    w = torch.rand(t, top_k)
    return x, ids, w, e, h, inter


def test_fp8_chain_order_and_flags(rec):
    x, ids, w, e, h, inter = _moe_inputs()
    w1 = torch.zeros(e, 2 * inter, h, dtype=torch.float8_e4m3fn)
    w2 = torch.zeros(e, h, inter, dtype=torch.float8_e4m3fn)
    s1 = torch.ones(e, 2 * inter // 128, h // 128)
    s2 = torch.ones(e, h // 128, inter // 128)
    out = moe.fp8_experts(None, x, w1, w2, s1, s2, w, ids, "gelu_tanh")
    assert rec.calls == ["moe_align_quant", "moe_gemm_fp8_w8a8", "fp8_quant_group128",
                         "moe_gemm_fp8_w8a8", "moe_sum"]
    assert rec.args[0][0].dtype == torch.int32                     # ids handed to the align as int32
    g13, g2 = rec.args[1], rec.args[3]
    assert g13[8] is None and g13[9] == 2 and g13[-2:] == (True, "gelu_tanh")     # top_k rows, fused act*mul
    assert torch.equal(g2[8], w.reshape(-1)) and g2[9] == 1 and g2[-2] is False   # top-k weight in w2
    assert g13[10] == moe.fp8_blocks(3, 2, 4)[0] and g13[11] == 128
    assert out.shape == (3, h) and g13[0].shape == (6, inter) and g2[0].shape == (6, h)


def test_fp8_chain_channel_scales_take_w8a16(rec):
    x, ids, w, e, h, inter = _moe_inputs()
    w1 = torch.zeros(e, 2 * inter, h, dtype=torch.float8_e4m3fn)
    w2 = torch.zeros(e, h, inter, dtype=torch.float8_e4m3fn)
    moe.fp8_experts(None, x, w1, w2, torch.ones(e, 2 * inter), torch.ones(e, h), w, ids)
    assert rec.calls == ["moe_align", "moe_gemm_fp8", "moe_gemm_fp8", "moe_sum"]


def test_router_weight_on_input_drops_w2_weights(rec):
    x, ids, w, e, h, inter = _moe_inputs(top_k=1)
    w1 = torch.zeros(e, 2 * inter, h, dtype=torch.bfloat16)
    w2 = torch.zeros(e, h, inter, dtype=torch.bfloat16)
    ws13 = torch.zeros(1000, dtype=torch.bfloat16)
    moe.bf16_experts(torch.zeros(3, h, dtype=torch.bfloat16), x, w1, w2, w, ids, "silu", True, ws13, None)
    assert rec.calls == ["moe_align", "moe_gemm_bf16", "moe_gemm_bf16", "moe_sum"]
    assert rec.args[2][6] is None
    assert rec.args[1][0].data_ptr() == ws13.data_ptr()           # the w13 output lives in the caller's workspace


@pytest.mark.parametrize("kind", ["sym", "zp", "w4a8"])
def test_wna16_chain_variants(rec, kind):
    x, ids, w, e, h, inter = _moe_inputs()
    if kind == "zp":
        w1 = torch.zeros(e, 2 * inter, h // 8, dtype=torch.int32)
        w2 = torch.zeros(e, h, inter // 8, dtype=torch.int32)
    else:
        w1 = torch.zeros(e, 2 * inter, h // 2, dtype=torch.uint8)
        w2 = torch.zeros(e, h, inter // 2, dtype=torch.uint8)
    s1, s2 = torch.ones(e, 2 * inter, h // 128), torch.ones(e, h, inter // 128)
    z = torch.zeros(1) if kind == "zp" else None
    moe.wna16_experts(None, x, w1, w2, s1, s2, w, ids, 128, "silu", z1=z, z2=z, w4a8=kind == "w4a8")
    expect = {"sym": ["moe_align"] + ["moe_gemm_w4a16"] * 2, "zp": ["moe_align"] + ["moe_gemm_w4a16_zp"] * 2,
              "w4a8": ["moe_act_quant_i8", "moe_align", "moe_gemm_w4a8", "moe_act_quant_i8", "moe_gemm_w4a8"]}[kind]
    assert rec.calls == expect + ["moe_sum"]


def test_mxfp4_and_int8_chains(rec):
    x, ids, w, e, h, inter = _moe_inputs()
    moe.mxfp4_experts(None, x, torch.zeros(e, 2 * inter, h // 2, dtype=torch.uint8),
                      torch.zeros(e, h, inter // 2, dtype=torch.uint8), None, None, w, ids)
    moe.int8_experts(None, x, torch.zeros(e, 2 * inter, h, dtype=torch.int8), torch.zeros(e, h, inter,
                     dtype=torch.int8), torch.ones(e, 2 * inter), torch.ones(e, h), w, ids)
    assert rec.calls == ["moe_align", "moe_gemm_mxfp4", "moe_gemm_mxfp4", "moe_sum",
                         "moe_align", "moe_gemm_w8a16", "moe_gemm_w8a16", "moe_sum"]
