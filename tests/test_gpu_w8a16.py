# SPDX-License-Identifier: MIT
"""The reference's W8A16 and bf16 ops on gfx950: fp8_dequant (byte-exact),
fp8_wmma_gemm(_raw)(_cfg), moe_gemm_fp8(_raw), moe_gemm_w8a16 and
moe_gemm_bf16, against dequantize-then-fp32 references (tests/test_fp8.py,
tests/test_moe_fp8.py, tests/test_moe_w8a16.py, tests/test_moe_gemm.py)."""

import pytest
import torch

import libstrix_amd  # noqa: F401
import oracle
from conftest import peak_rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make(n, k, seed=0):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=g) * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
    bs = torch.rand((n + 127) // 128, k // 128, generator=g) * 0.02 + 0.005
    return w, bs


def make_ch(n, k, seed=0):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=g) * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
    return w, torch.rand(n, generator=g) * 0.02 + 0.005


@pytest.mark.parametrize("n,k", [(16384, 5120), (256, 1024), (300, 1024)])
def test_fp8_dequant_exact(n, k):
    w, bs = make(n, k)
    out = torch.ops.strix.fp8_dequant(w.to(DEV), bs.to(DEV)).cpu()
    assert torch.equal(out, oracle.fp8_block_dequant(w, bs).to(torch.bfloat16))


def test_fp8_dequant_channel_and_all_codes():
    w, s = make_ch(300, 704)
    out = torch.ops.strix.fp8_dequant(w.to(DEV), s.to(DEV)).cpu()
    assert torch.equal(out, (w.float() * s[:, None]).to(torch.bfloat16))
    codes = torch.arange(256, dtype=torch.uint8)
    codes = codes[(codes & 0x7F) != 0x7F]
    wq = torch.nn.functional.pad(codes.reshape(1, -1).repeat(128, 1), (0, 256 - codes.numel())).view(torch.float8_e4m3fn)
    out = torch.ops.strix.fp8_dequant(wq.contiguous().to(DEV), torch.ones(1, 2, device=DEV)).cpu()
    assert torch.equal(out.float(), oracle.e4m3_decode(wq))


@pytest.mark.parametrize("raw", [False, True])
@pytest.mark.parametrize("m", [1, 6, 17, 64, 129, 300])
@pytest.mark.parametrize("n,k", [(512, 1024), (300, 2048)])
def test_fp8_wmma_block(m, n, k, raw):
    w, bs = make(n, k, m)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(torch.float16 if raw else torch.bfloat16)
    op = torch.ops.strix.fp8_wmma_gemm_raw if raw else torch.ops.strix.fp8_wmma_gemm
    out = op(w.to(DEV), x.to(DEV), bs.to(DEV))
    assert out.dtype == torch.bfloat16
    assert peak_rel_err(out, x.float() @ oracle.fp8_block_dequant(w, bs).t()) <= 8e-3


@pytest.mark.parametrize("raw", [False, True])
@pytest.mark.parametrize("n,k", [(2816, 2112), (300, 704)])
def test_fp8_wmma_channel(n, k, raw):
    w, s = make_ch(n, k)
    x = torch.randn(70, k, generator=torch.Generator().manual_seed(1)).to(torch.float16 if raw else torch.bfloat16)
    op = torch.ops.strix.fp8_wmma_gemm_raw if raw else torch.ops.strix.fp8_wmma_gemm
    out = op(w.to(DEV), x.to(DEV), s.to(DEV))
    assert peak_rel_err(out, x.float() @ (w.float() * s[:, None]).t()) <= 8e-3


@pytest.mark.parametrize("cfg", range(8))
def test_fp8_wmma_every_cfg(cfg):
    w, bs = make(640, 1536, cfg)
    x = torch.randn(70, 1536, generator=torch.Generator().manual_seed(cfg)).to(torch.bfloat16)
    out = torch.ops.strix.fp8_wmma_gemm_cfg(w.to(DEV), x.to(DEV), bs.to(DEV), cfg)
    assert peak_rel_err(out, x.float() @ oracle.fp8_block_dequant(w, bs).t()) <= 8e-3


def test_fp8_wmma_padded_rows():
    w, bs = make(512, 1024)
    buf = torch.zeros(512, 1024 + 128, dtype=torch.uint8)
    buf[:, :1024] = w.view(torch.uint8)
    x = torch.randn(40, 1024, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    out = torch.ops.strix.fp8_wmma_gemm(buf.view(torch.float8_e4m3fn).to(DEV)[:, :1024], x.to(DEV), bs.to(DEV))
    assert peak_rel_err(out, x.float() @ oracle.fp8_block_dequant(w, bs).t()) <= 8e-3


# ---------------------------------------------------------------- MoE W8A16 / bf16
E, TOPK = 16, 8


def _routing(tokens, block_m, seed):
    g = torch.Generator().manual_seed(seed)
    ids = torch.stack([torch.randperm(E, generator=g)[:TOPK] for _ in range(tokens)]).to(torch.int32)
    return ids, torch.ops.strix.moe_align(ids.to(DEV), E, block_m), g


def _run(op, gemm, tokens, block_m, activation, b, scales, deq, adtype=torch.bfloat16, out_dtype=torch.bfloat16):
    n, k = b.shape[1], b.shape[2]
    ids, (sorted_ids, expert_ids, num_post), g = _routing(tokens, block_m, tokens * 3 + block_m)
    if gemm == "w13":
        a = torch.randn(tokens, k, generator=g).to(adtype)
        a_topk, weights, cols = TOPK, None, n // 2
    else:
        a = torch.randn(tokens * TOPK, k, generator=g).to(adtype)
        a_topk, weights, cols = 1, torch.rand(tokens, TOPK, generator=g), n
    c = torch.full((tokens * TOPK, cols), float("nan"), dtype=out_dtype, device=DEV)
    args = [c, a.to(DEV), b.to(DEV)] + ([] if scales is None else [scales.to(DEV)])
    op(*args, sorted_ids, expert_ids, num_post, None if weights is None else weights.reshape(-1).to(DEV), a_topk,
       block_m, 64, gemm == "w13", activation)
    ref = oracle.moe_expert_gemm(a, deq, ids, a_topk, weights)
    if gemm == "w13":
        g_, u_ = ref[:, :cols], ref[:, cols:]
        act = torch.nn.functional.silu(g_) if activation == "silu" else torch.nn.functional.gelu(g_, approximate="tanh")
        ref = act * u_
    assert not torch.isnan(c).any()
    return peak_rel_err(c, ref)


GEMMS = [("w13", "silu"), ("w13", "gelu_tanh"), ("w2", "silu")]
SHAPES = {"w13": (1024, 2048), "w2": (2048, 512)}


@pytest.mark.parametrize("tokens", [1, 5, 40])
@pytest.mark.parametrize("block_m", [16, 64, 128])
@pytest.mark.parametrize("gemm,activation", GEMMS)
@pytest.mark.parametrize("scheme", ["block", "channel"])
@pytest.mark.parametrize("raw", [False, True])
def test_moe_gemm_fp8(tokens, block_m, gemm, activation, scheme, raw):
    n, k = SHAPES[gemm]
    g = torch.Generator().manual_seed(7)
    w = (torch.randn(E, n, k, generator=g) * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
    if scheme == "block":
        s = torch.rand(E, n // 128, k // 128, generator=g) * 0.02 + 0.001
        full = s.repeat_interleave(128, 1).repeat_interleave(128, 2)
    else:
        s = torch.rand(E, n, generator=g) * 0.02 + 0.001
        full = s.reshape(E, n, 1)
    deq = w.float() * full
    op = torch.ops.strix.moe_gemm_fp8_raw if raw else torch.ops.strix.moe_gemm_fp8
    out_dtype = torch.float16 if (raw and gemm == "w13") else torch.bfloat16
    err = _run(op, gemm, tokens, block_m, activation, w, s, deq, torch.float16 if raw else torch.bfloat16, out_dtype)
    assert err <= 1e-2


@pytest.mark.parametrize("tokens", [1, 5, 40])
@pytest.mark.parametrize("block_m", [16, 64, 128])
@pytest.mark.parametrize("gemm,activation", GEMMS)
@pytest.mark.parametrize("scale_shape", ["en", "en1"])
def test_moe_gemm_w8a16(tokens, block_m, gemm, activation, scale_shape):
    n, k = SHAPES[gemm]
    g = torch.Generator().manual_seed(8)
    w = torch.randint(-127, 128, (E, n, k), generator=g, dtype=torch.int8)
    s = torch.rand(E, n, generator=g) * 0.02 + 0.001
    deq = w.float() * s.reshape(E, n, 1)
    scales = s if scale_shape == "en" else s.unsqueeze(-1)
    assert _run(torch.ops.strix.moe_gemm_w8a16, gemm, tokens, block_m, activation, w, scales, deq) <= 1e-2


@pytest.mark.parametrize("tokens", [1, 5, 64, 700])
@pytest.mark.parametrize("block_m", [16, 32, 64, 128])
@pytest.mark.parametrize("gemm,activation", GEMMS)
def test_moe_gemm_bf16(tokens, block_m, gemm, activation):
    n, k = SHAPES[gemm]
    g = torch.Generator().manual_seed(9)
    b = (torch.randn(E, n, k, generator=g) / k ** 0.5).to(torch.bfloat16)
    assert _run(torch.ops.strix.moe_gemm_bf16, gemm, tokens, block_m, activation, b, None, b.float()) <= 1e-2
