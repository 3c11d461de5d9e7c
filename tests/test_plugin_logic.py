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

from libstrix_amd import torch_ops

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
    "w8a16_gemm": lambda w, x, s, b, g: torch.zeros(x.size(0), w.size(0), dtype=x.dtype),
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
    d = plugin._cache_factor(True)
    assert d != a
    clean_env.setenv("STRIX_DISABLE", " fp8 ,")                 # the same set of names: the same key
    assert plugin._cache_factor(True) == d
    clean_env.setenv("STRIX_DISABLE", "fp8,mxfp4")
    assert plugin._cache_factor(True) != d


def test_model_architectures_without_vllm():
    assert plugin._model_architectures() == []


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
    z1 = torch.zeros(e, n // 2, k // 128, dtype=torch.uint8)      # vLLM's packed zero points: eligible
    z2 = torch.zeros(e, k // 2, (n // 2) // 128, dtype=torch.uint8)
    assert moe.wna16_bad(x, w1, w2, s1, s2, 128, "silu", None, has_zp=True, z1=z1, z2=z2) == []
    assert moe.wna16_bad(x, w1, w2, s1, s2, 128, "silu", None, has_zp=True, z1=z1, z2=None) == ["zero_point"]
    assert moe.wna16_bad(x, w1, w2, s1.float(), s2, 128, "silu", None, has_zp=True, z1=z1,
                         z2=z2) == ["zero_point"]                 # the zp kernel takes bf16/fp16 scales
    assert moe.wna16_bad(x, w1, w2, s1, s2, 128, "silu", None, has_zp=True,
                         z1=torch.zeros(e, n, k // 128, dtype=torch.uint8), z2=z2) == ["zero_point"]
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


def test_w8_prepare_scale_layouts():
    w = torch.zeros(64, 256, dtype=torch.uint8)
    s = torch.rand(64, 2, dtype=torch.bfloat16)
    p = linear.prepare_w8(w, s, 128)
    assert p.group_size == 128 and p.w8a8_s.shape == (2, 64) and torch.equal(p.w8a8_s, s.float().t())
    assert p.w8a8_s.dtype == torch.float32 and p.w8a8_s.is_contiguous()
    pc = linear.prepare_w8(w, torch.rand(64, 1), -1)           # per channel: [N] for both paths
    assert pc.group_size == 0 and pc.w_s.shape == (64,) and pc.w8a8_s.shape == (64,)
    for g in (32, 64):                                           # no W8A8 layout: W8A16 at every M
        pg = linear.prepare_w8(w, torch.rand(64, 256 // g), g)
        assert pg.w8a8_s is None and pg.w_s.shape == (64, 256 // g)
    assert linear.prepare_w8(torch.zeros(64, 192, dtype=torch.uint8), torch.rand(64, 1), 0).w8a8_s is None
    with pytest.raises(RuntimeError, match="group scales"):
        linear.prepare_w8(w, torch.rand(64, 3), 128)
    with pytest.raises(RuntimeError, match="per-channel"):
        linear.prepare_w8(w, torch.rand(32), 0)
    assert torch.equal(linear.pack_w8_rows(torch.tensor([[0, 255, 256 + 7]])), torch.tensor([[0, 255, 7]],
                                                                                             dtype=torch.uint8))
    assert linear.can_implement_w8("uint8b128", False, torch.bfloat16, 128, 5120) == (True, None)
    assert linear.can_implement_w8("uint8b128", False, torch.bfloat16, 64, 5120) == (True, None)
    assert not linear.can_implement_w8("uint8b128", False, torch.bfloat16, 16, 5120)[0]
    assert not linear.can_implement_w8("uint4b8", False, torch.bfloat16, 128, 5120)[0]
    assert linear.can_implement_w4("uint4b8", False, 64, 5120) == (True, None)
    assert not linear.can_implement_w4("uint4b8", True, 64, 5120)[0]


def test_fp8_channel_prepare_square_weight():
    # A square [K, N] view (vLLM's per-channel layout) must be transposed back
    # to [N, K] rows even though its sizes cannot tell the orientation.
    w = torch.arange(256 * 256, dtype=torch.float32).reshape(256, 256).remainder(97).to(torch.float8_e4m3fn)
    wc, _ = fp8.prepare_channel(w.t(), torch.ones(256), 256)
    assert torch.equal(wc.view(torch.uint8), w.view(torch.uint8)) and wc.is_contiguous()
    wr, _ = fp8.prepare_channel(w, torch.ones(256), 256)       # row-major [N, K] stays as is
    assert torch.equal(wr.view(torch.uint8), w.view(torch.uint8))
    wk, _ = fp8.prepare_channel(w[:, :128].contiguous(), torch.ones(128), 128)   # stored [K, N]: transposed
    assert wk.shape == (128, 256)
    with pytest.raises(RuntimeError, match="no dimension"):
        fp8.prepare_channel(w[:100, :200], torch.ones(64), 64)


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
    p = linear.prepare_w8(torch.zeros(64, 256, dtype=torch.uint8), torch.ones(64, 2, dtype=torch.bfloat16), 128)
    linear._apply_impl(torch.zeros(m, 256, dtype=torch.bfloat16), p.w_q, p.w_s, p.w8a8_s, None, p.group_size)
    assert rec.calls == [expect]
    if expect == "w8a8_wmma_gemm":
        assert rec.args[0][2] is p.w8a8_s                          # the load-time scales, no per-call copy


@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("m,expect", [(8, "w8a16_skinny_gemm"), (20, "w8a16_gemm"), (4096, "w8a16_gemm")])
def test_w8a16_small_group_prefill_stays_w8a16(rec, group, m, expect):
    p = linear.prepare_w8(torch.zeros(64, 256, dtype=torch.uint8), torch.ones(64, 256 // group,
                                                                              dtype=torch.bfloat16), group)
    out = linear._apply_impl(torch.zeros(m, 256, dtype=torch.bfloat16), p.w_q, p.w_s, p.w8a8_s, None, group)
    assert rec.calls == [expect] and out.shape == (m, 64)


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


def test_w4a8_blocks():
    # 128 x 128 once the experts average 128 routed rows.
    assert moe.w4a8_blocks(8192, 8, 128) == (128, 128)
    assert moe.w4a8_blocks(2048, 8, 128) == (128, 128)
    assert moe.w4a8_blocks(1024, 8, 128) == (64, 128)
    for t in (1, 1024, 4096, 8192, 65536):
        bm, bn = moe.w4a8_blocks(t, 8, 128)
        assert (bm, bn) in torch_ops._W4A8_TILES   # tiles the op accepts


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


# ------------------------------------------------------------------ vLLM hook classes (stub vLLM)
class _StubExperts:
    """Stands in for vLLM's TritonExperts / TritonWNA16Experts: `apply` is the
    fallback the Strix classes call when a layer is not eligible."""

    fell: list = []

    def __init__(self, *args, **kwargs):
        self.block_shape = None
        self.w1_scale = self.w2_scale = None
        self.w1_zp = self.w2_zp = None
        self.w1_bias = self.w2_bias = None

    def apply(self, **kwargs):
        self.fell.append(kwargs)   # the class-level list of the stub base, shared by subclasses


class _StubLogger:
    def warning_once(self, *a):
        pass

    info = warning_once


@pytest.fixture
def stub_vllm(monkeypatch):
    import sys
    import types

    names = ["vllm", "vllm.model_executor", "vllm.model_executor.layers", "vllm.model_executor.layers.fused_moe",
             "vllm.model_executor.layers.fused_moe.experts", "vllm.model_executor.layers.fused_moe.experts.triton_moe",
             "vllm.logger"]
    mods = {n: types.ModuleType(n) for n in names}
    tm = mods["vllm.model_executor.layers.fused_moe.experts.triton_moe"]
    tm.TritonExperts = type("TritonExperts", (_StubExperts,), {"fell": []})
    tm.TritonWNA16Experts = type("TritonWNA16Experts", (_StubExperts,), {"fell": []})
    mods["vllm.logger"].init_logger = lambda name: _StubLogger()
    for n, m in mods.items():
        monkeypatch.setitem(sys.modules, n, m)
    return tm


def _apply_kwargs(x, w1, w2, ids, tw):
    return dict(output=None, hidden_states=x, w1=w1, w2=w2, topk_weights=tw, topk_ids=ids, activation="silu",
                global_num_experts=w1.size(0), expert_map=None, a1q_scale=None, a2_scale=None, workspace13=None,
                workspace2=None, expert_tokens_meta=None, apply_router_weight_on_input=False)


def test_wna16_class_runs_zero_points(rec, stub_vllm, clean_env):
    e, n, k, t, top_k = 4, 256, 512, 3, 2
    cls = moe._make_wna16_experts_cls()
    ex = cls()
    ex.block_shape = [0, 128]
    ex.w1_scale = torch.ones(e, n, k // 128, dtype=torch.bfloat16)
    ex.w2_scale = torch.ones(e, k, (n // 2) // 128, dtype=torch.bfloat16)
    ex.w1_zp = torch.zeros(e, n // 2, k // 128, dtype=torch.uint8)
    ex.w2_zp = torch.zeros(e, k // 2, (n // 2) // 128, dtype=torch.uint8)
    x = torch.zeros(t, k, dtype=torch.bfloat16)
    w1 = torch.zeros(e, n, k // 2, dtype=torch.uint8)
    w2 = torch.zeros(e, k, n // 4, dtype=torch.uint8)
    ids, tw = torch.zeros(t, top_k, dtype=torch.int32), torch.rand(t, top_k)
    ex.apply(**_apply_kwargs(x, w1, w2, ids, tw))
    assert rec.calls == ["moe_align", "moe_gemm_w4a16_zp", "moe_gemm_w4a16_zp", "moe_sum"]
    assert rec.args[1][4] is ex.w1_zp and rec.args[2][4] is ex.w2_zp
    assert not stub_vllm.TritonWNA16Experts.fell
    # Zero points in another layout (one byte per n): vLLM's own kernel runs.
    ex.w1_zp = torch.zeros(e, n, k // 128, dtype=torch.uint8)
    ex.apply(**_apply_kwargs(x, w1, w2, ids, tw))
    assert len(stub_vllm.TritonWNA16Experts.fell) == 1 and len(rec.calls) == 4


def test_mxfp4_class_and_gate(rec, stub_vllm, clean_env):
    e, n, k, t, top_k = 4, 256, 512, 5, 2
    ex = moe._make_mxfp4_experts_cls()()
    assert ex.expects_unquantized_inputs
    ex.w1_scale = torch.zeros(e, n, k // 32, dtype=torch.uint8)
    ex.w2_scale = torch.zeros(e, k, (n // 2) // 32, dtype=torch.uint8)
    x = torch.zeros(t, k, dtype=torch.bfloat16)
    w1 = torch.zeros(e, n, k // 2, dtype=torch.uint8)
    w2 = torch.zeros(e, k, n // 4, dtype=torch.uint8)
    ids, tw = torch.zeros(t, top_k, dtype=torch.int32), torch.rand(t, top_k)
    ex.apply(**_apply_kwargs(x, w1, w2, ids, tw))
    assert rec.calls == ["moe_align", "moe_gemm_mxfp4", "moe_gemm_mxfp4", "moe_sum"]
    ex.w1_bias = torch.zeros(e, n)                                  # biases (e.g. gpt-oss): vLLM's own path
    ex.apply(**_apply_kwargs(x, w1, w2, ids, tw))
    assert len(stub_vllm.TritonExperts.fell) == 1 and len(rec.calls) == 4
    assert moe.mxfp4_bad(x, w1, w2, ex.w1_scale, ex.w2_scale, "silu", None) == []
    assert moe.mxfp4_bad(x, w1, w2, ex.w1_scale.float(), ex.w2_scale, "silu", None) == ["scales"]
    assert moe.mxfp4_bad(x, w1, w2, ex.w1_scale, ex.w2_scale, "swigluoai", None) == ["activation"]
    assert moe.mxfp4_bad(x.half(), w1, w2, ex.w1_scale, ex.w2_scale, "silu", None) == ["act_dtype"]


def test_backend_hook_routes_triton_only():
    import enum
    import types

    class Backend(enum.Enum):
        TRITON = 1
        OTHER = 2

    mod = types.SimpleNamespace(Mxfp4MoeBackend=Backend, backend_to_kernel_cls=lambda b: ["vllm-own"])
    assert moe._hook_backend(mod, "Mxfp4MoeBackend", "strix-cls")
    assert mod.backend_to_kernel_cls(Backend.TRITON) == ["strix-cls"]
    assert mod.backend_to_kernel_cls(Backend.OTHER) == ["vllm-own"]
    assert not moe._hook_backend(types.SimpleNamespace(), "Mxfp4MoeBackend", "strix-cls")
