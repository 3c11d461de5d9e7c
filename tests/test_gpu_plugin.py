# SPDX-License-Identifier: MIT
"""The vLLM plugin's per-forward dispatchers and expert chains on the GPU,
every branch against the oracle (dequantize, then fp32 matmul; the W8A8
branches with the op's own activation QDQ). Bar: max error 1e-2 of the
output's peak. vLLM itself is not needed: these are the functions the
plugin's kernel classes call (python/strix_vllm/{int8,fp8,mxfp4,linear,moe}.py
is the reference's layer)."""

import pytest
import torch

import libstrix_amd  # noqa: F401
import oracle
from conftest import peak_rel_err
from libstrix_amd.vllm_plugin import fp8, int8, linear, moe, mxfp4

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-2


def _g(seed):
    return torch.Generator().manual_seed(seed)


# ------------------------------------------------------------------ dense linears
@pytest.mark.parametrize("m", [1, 32, 300])
def test_int8_linear(m):
    n, k = 512, 1024
    g = _g(m)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    sw = torch.rand(n, generator=g) * 0.01 + 0.001
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    wd, sd = int8.prepare_weights(w.to(DEV), sw.to(DEV))
    out = int8._apply_impl(x.to(DEV), wd, sd, bias.to(DEV)).cpu()
    qa, sa = oracle.int8_quant_per_token(x)
    ref = oracle.w8a8_int8_gemm(qa, sa, w, sw) + bias.float()
    assert out.shape == (m, n) and out.dtype == torch.bfloat16 and peak_rel_err(out, ref) <= TOL


def _fp8_weights(n, k, seed):
    g = _g(seed)
    w = (torch.randn(n, k, generator=g) * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
    bs = torch.rand((n + 127) // 128, k // 128, generator=g) * 0.02 + 0.005
    return w, bs


@pytest.mark.parametrize("m", [1, 16, 100, 600])
def test_fp8_block_linear_w8a8(m):
    n, k = 640, 1024
    w, bs = _fp8_weights(n, k, m)
    x = torch.randn(m, k, generator=_g(m + 1)).to(torch.bfloat16)
    wd, bsd = fp8.prepare_block(w.to(DEV), bs.to(DEV))
    out = fp8._apply_impl(x.to(DEV), wd, bsd, None, True).cpu()
    qa, sa = oracle.fp8_quant_group128(x)
    assert peak_rel_err(out, oracle.fp8_block_gemm(qa, sa, w, bs)) <= TOL
    # The plugin's load transform re-lays the weights K-block-major: same bits.
    wk, bsk = fp8.prepare_block(w.to(DEV), bs.to(DEV), kmajor=True)
    assert wk.shape == (k // 128, n, 128)
    assert torch.equal(fp8._apply_impl(x.to(DEV), wk, bsk, None, True).cpu(), out)


@pytest.mark.parametrize("m", [1, 8, fp8.W8A16_DEQUANT_MIN_M - 1, fp8.W8A16_DEQUANT_MIN_M, 300])
@pytest.mark.parametrize("scales", ["block", "channel"])
def test_fp8_linear_w8a16(m, scales):
    n, k = 640, 1024
    w, bs = _fp8_weights(n, k, 7 * m)
    if scales == "block":
        s, wf = bs, oracle.fp8_block_dequant(w, bs)
    else:
        s = torch.rand(n, generator=_g(m)) * 0.02 + 0.005
        wf = oracle.e4m3_decode(w.view(torch.uint8)) * s[:, None]
    x = torch.randn(m, k, generator=_g(m + 2)).to(torch.bfloat16)
    bias = torch.randn(n, generator=_g(m + 3)).to(torch.bfloat16)
    out = fp8._apply_impl(x.to(DEV), w.to(DEV), s.to(DEV), bias.to(DEV), False).cpu()
    assert peak_rel_err(out, x.float() @ wf.t() + bias.float()) <= TOL


@pytest.mark.parametrize("m", [1, 200])
def test_fp8_channel_square_weight_through_load_transform(m):
    # A square weight handed over as vLLM's [K, N] view: the load transform
    # must restore [N, K] rows from the strides (sizes cannot tell N from K).
    n = k = 1024
    w, _ = _fp8_weights(n, k, 31 + m)
    s = torch.rand(n, generator=_g(m)) * 0.02 + 0.005
    wc, sc = fp8.prepare_channel(w.to(DEV).t(), s.to(DEV), n)
    x = torch.randn(m, k, generator=_g(m + 5)).to(torch.bfloat16)
    out = fp8._apply_impl(x.to(DEV), wc, sc, None, False).cpu()
    wf = oracle.e4m3_decode(w.view(torch.uint8)) * s[:, None]
    assert peak_rel_err(out, x.float() @ wf.t()) <= TOL


@pytest.mark.parametrize("m,bias", [(1, False), (5, False), (3, True), (64, False), (mxfp4.DEQUANT_MIN_M, True),
                                    (300, False)])
def test_mxfp4_linear(m, bias):
    n, k = 512, 1024
    g = _g(m + 100)
    w = torch.randint(0, 256, (n, k // 2), generator=g, dtype=torch.uint8)
    s = torch.randint(118, 134, (n, k // 32), generator=g, dtype=torch.uint8)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    b = torch.randn(n, generator=g).to(torch.bfloat16) if bias else None
    mxfp4.check_weights(w, s)
    out = mxfp4._apply_impl(x.to(DEV), w.to(DEV), s.to(DEV), None if b is None else b.to(DEV)).cpu()
    ref = x.float() @ oracle.mxfp4_decode(w, s).t() + (0 if b is None else b.float())
    assert peak_rel_err(out, ref) <= TOL


@pytest.mark.parametrize("m", [1, 8, 9, 200])
@pytest.mark.parametrize("group", [0, 32, 64, 128])
def test_w8a16_linear(m, group):
    n, k = 512, 1024
    g = _g(m + group)
    w = torch.randint(0, 256, (n, k), generator=g, dtype=torch.uint8)
    s = (torch.rand(n, k // group if group else 1, generator=g) * 0.01 + 0.001).to(torch.bfloat16)
    if group == 0:
        s = s.reshape(n)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    p = linear.prepare_w8(w.to(DEV), s.to(DEV), group)
    out = linear._apply_impl(x.to(DEV), p.w_q, p.w_s, p.w8a8_s, None, group).cpu()
    wf = oracle.u8b128_decode(w, s, group)
    if m <= linear.MAX_SKINNY_BATCH_SIZE or p.w8a8_s is None:   # bf16 activations as given
        ref = x.float() @ wf.t()
    else:   # the W8A8 op quantizes the activations per (row, 128) inside
        qa, sa = oracle.int8_quant_group128(x)
        ref = (qa.float() * sa.repeat_interleave(128, dim=1)) @ wf.t()
    assert peak_rel_err(out, ref) <= TOL


@pytest.mark.parametrize("m", [1, 40, mxfp4.DEQUANT_MIN_M, 260])
@pytest.mark.parametrize("group", [-1, 32, 128])
def test_w4a16_linear(m, group):
    n, k = 512, 1024
    g = _g(m * 3 + group)
    q = torch.randint(0, 16, (n, k), generator=g)
    gs = k if group == -1 else group
    s = (torch.rand(n, k // gs, generator=g) * 0.05 + 0.01).to(torch.bfloat16)
    w = oracle.wna16_ex_pack(q)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    s_arg = s.reshape(n) if group == -1 else s
    out = linear._w4_apply_impl(x.to(DEV), w.to(DEV), s_arg.to(DEV), None, group).cpu()
    assert peak_rel_err(out, x.float() @ oracle.wna16_ex_decode(w, s, gs).t()) <= TOL


# ------------------------------------------------------------------ expert chains
def _route(t, e, top_k, seed):
    g = _g(seed)
    ids = torch.stack([torch.randperm(e, generator=g)[:top_k] for _ in range(t)]).to(torch.int32)
    w = torch.rand(t, top_k, generator=g)
    return ids, w / w.sum(-1, keepdim=True)


@pytest.mark.parametrize("t", [1, 37, 700])
@pytest.mark.parametrize("act", ["silu", "gelu_tanh"])
def test_fp8_experts_w8a8(t, act):
    """Checked per stage: the w13 output (read back from the caller's
    workspace) against the oracle, then the final output against the oracle
    run on that same intermediate, so an e4m3 rounding flip of the
    intermediate's re-quantization cannot make the comparison flaky."""
    e, top_k, h, inter = 16, 4, 512, 256
    g = _g(t)
    w13 = (torch.randn(e, 2 * inter, h, generator=g) * 30).clamp(-448, 448).to(torch.float8_e4m3fn)
    w2 = (torch.randn(e, h, inter, generator=g) * 30).clamp(-448, 448).to(torch.float8_e4m3fn)
    s13 = torch.rand(e, 2 * inter // 128, h // 128, generator=g) * 0.002 + 0.001
    s2 = torch.rand(e, h // 128, inter // 128, generator=g) * 0.002 + 0.001
    x = torch.randn(t, h, generator=g).to(torch.bfloat16)
    ids, tw = _route(t, e, top_k, t + 1)
    ws13 = torch.full((t * top_k * inter,), float("nan"), dtype=torch.bfloat16, device=DEV)
    out = moe.fp8_experts(None, x.to(DEV), w13.to(DEV), w2.to(DEV), s13.to(DEV), s2.to(DEV), tw.to(DEV),
                          ids.to(DEV), act, workspace13=ws13).cpu()
    mid = ws13.cpu().view(t * top_k, inter)
    d13 = torch.stack([oracle.fp8_block_dequant(w13[i], s13[i]) for i in range(e)])
    d2 = torch.stack([oracle.fp8_block_dequant(w2[i], s2[i]) for i in range(e)])
    qx, sx = oracle.fp8_quant_group128(x)
    hh = oracle.moe_expert_gemm(qx.float() * sx.repeat_interleave(128, dim=1), d13, ids, top_k)
    gate = torch.nn.functional.silu(hh[:, :inter]) if act == "silu" else torch.nn.functional.gelu(
        hh[:, :inter], approximate="tanh")
    assert peak_rel_err(mid, gate * hh[:, inter:]) <= TOL
    qi, si = oracle.fp8_quant_group128(mid)
    y = oracle.moe_expert_gemm(qi.float() * si.repeat_interleave(128, dim=1), d2,
                               ids.reshape(-1, 1), 1, tw.reshape(-1))
    ref = oracle.moe_sum(y.to(torch.bfloat16), top_k)
    assert out.shape == (t, h) and peak_rel_err(out, ref) <= TOL


@pytest.mark.parametrize("t", [3, 200])
def test_fp8_experts_channel_w8a16(t):
    e, top_k, h, inter = 8, 2, 512, 256
    g = _g(50 + t)
    w13 = (torch.randn(e, 2 * inter, h, generator=g) * 30).clamp(-448, 448).to(torch.float8_e4m3fn)
    w2 = (torch.randn(e, h, inter, generator=g) * 30).clamp(-448, 448).to(torch.float8_e4m3fn)
    s13 = torch.rand(e, 2 * inter, generator=g) * 0.002 + 0.001
    s2 = torch.rand(e, h, generator=g) * 0.002 + 0.001
    x = torch.randn(t, h, generator=g).to(torch.bfloat16)
    ids, tw = _route(t, e, top_k, t + 2)
    out = moe.fp8_experts(None, x.to(DEV), w13.to(DEV), w2.to(DEV), s13.to(DEV), s2.to(DEV), tw.to(DEV),
                          ids.to(DEV)).cpu()
    dq = lambda w, s: oracle.e4m3_decode(w.view(torch.uint8)) * s[:, None]
    ref = oracle.fused_moe(x, ids, tw, lambda i: dq(w13[i], s13[i]), lambda i: dq(w2[i], s2[i]))
    assert peak_rel_err(out, ref) <= TOL


@pytest.mark.parametrize("t", [1, 300])
def test_bf16_experts_router_weight_on_input(t):
    e, top_k, h, inter = 8, 1, 256, 128
    g = _g(70 + t)
    w13 = (torch.randn(e, 2 * inter, h, generator=g) * 0.05).to(torch.bfloat16)
    w2 = (torch.randn(e, h, inter, generator=g) * 0.05).to(torch.bfloat16)
    x = torch.randn(t, h, generator=g).to(torch.bfloat16)
    ids, tw = _route(t, e, top_k, t + 3)
    # the caller has already scaled the input rows by their router weight
    out = moe.bf16_experts(None, x.to(DEV), w13.to(DEV), w2.to(DEV), tw.to(DEV), ids.to(DEV), "silu", True).cpu()
    ref = oracle.fused_moe(x, ids, torch.ones_like(tw), w13.float(), w2.float())
    assert peak_rel_err(out, ref) <= TOL


@pytest.mark.parametrize("t", [2, 300])
@pytest.mark.parametrize("group", [32, 128])
def test_wna16_experts_symmetric(t, group):
    e, top_k, h, inter = 8, 2, 512, 256
    g = _g(90 + t + group)
    q13 = torch.randint(0, 16, (e, 2 * inter, h), generator=g, dtype=torch.uint8)
    q2 = torch.randint(0, 16, (e, h, inter), generator=g, dtype=torch.uint8)
    pack = lambda q: (q[..., 0::2] | (q[..., 1::2] << 4)).contiguous()
    s13 = (torch.rand(e, 2 * inter, h // group, generator=g) * 0.02 + 0.002).to(torch.bfloat16)
    s2 = (torch.rand(e, h, inter // group, generator=g) * 0.02 + 0.002).to(torch.bfloat16)
    x = torch.randn(t, h, generator=g).to(torch.bfloat16)
    ids, tw = _route(t, e, top_k, t + 4)
    w13, w2 = pack(q13), pack(q2)
    out = moe.wna16_experts(None, x.to(DEV), w13.to(DEV), w2.to(DEV), s13.to(DEV), s2.to(DEV), tw.to(DEV),
                            ids.to(DEV), group).cpu()
    ref = oracle.fused_moe(x, ids, tw, oracle.wna16_sym_decode(w13, s13, group),
                           oracle.wna16_sym_decode(w2, s2, group))
    assert peak_rel_err(out, ref) <= TOL


@pytest.mark.parametrize("t", [2, 300])
@pytest.mark.parametrize("group", [64, 128])
def test_wna16_experts_zero_points(t, group):
    # The vLLM WNA16 class passes w1_zp / w2_zp (uint8 [E, N/2, K/G], even n
    # in the low nibble) with uint8 [E, N, K/2] weights: (q - z) * s.
    e, top_k, h, inter = 8, 2, 512, 256
    g = _g(190 + t + group)
    q13 = torch.randint(0, 16, (e, 2 * inter, h), generator=g, dtype=torch.uint8)
    q2 = torch.randint(0, 16, (e, h, inter), generator=g, dtype=torch.uint8)
    pack = lambda q: (q[..., 0::2] | (q[..., 1::2] << 4)).contiguous()
    zpack = lambda z: (z[..., 0::2, :] | (z[..., 1::2, :] << 4)).contiguous()
    z13 = torch.randint(0, 16, (e, 2 * inter, h // group), generator=g, dtype=torch.uint8)
    z2 = torch.randint(0, 16, (e, h, inter // group), generator=g, dtype=torch.uint8)
    s13 = (torch.rand(e, 2 * inter, h // group, generator=g) * 0.02 + 0.002).to(torch.bfloat16)
    s2 = (torch.rand(e, h, inter // group, generator=g) * 0.02 + 0.002).to(torch.bfloat16)
    x = torch.randn(t, h, generator=g).to(torch.bfloat16)
    ids, tw = _route(t, e, top_k, t + 6)
    w13, w2, zz13, zz2 = pack(q13), pack(q2), zpack(z13), zpack(z2)
    out = moe.wna16_experts(None, x.to(DEV), w13.to(DEV), w2.to(DEV), s13.to(DEV), s2.to(DEV), tw.to(DEV),
                            ids.to(DEV), group, z1=zz13.to(DEV), z2=zz2.to(DEV)).cpu()
    ref13 = (q13.float() - z13.repeat_interleave(group, -1).float()) * s13.float().repeat_interleave(group, -1)
    ref2 = (q2.float() - z2.repeat_interleave(group, -1).float()) * s2.float().repeat_interleave(group, -1)
    # The oracle's decode of the same bytes (uint8 [E, N, K/2] viewed as int32 words) agrees.
    assert torch.equal(oracle.wna16_zp_decode(w13.view(torch.int32), s13, zz13, group), ref13)
    ref = oracle.fused_moe(x, ids, tw, ref13, ref2)
    assert peak_rel_err(out, ref) <= TOL


def test_awq_checkpoint_through_zero_point_experts():
    # AWQ-layout experts ([E, K, N/8] words in AutoAWQ's nibble order), converted
    # on the device at load, then the zero-point expert chain.
    from libstrix_amd import convert
    from test_convert import awq_pack_reference

    e, top_k, h, inter, group, t = 4, 2, 256, 128, 128, 37
    g = _g(777)
    q13 = torch.randint(0, 16, (e, h, 2 * inter), generator=g)     # AWQ is [K, N]
    q2 = torch.randint(0, 16, (e, inter, h), generator=g)
    z13 = torch.randint(0, 16, (e, h // group, 2 * inter), generator=g)
    z2 = torch.randint(0, 16, (e, inter // group, h), generator=g)
    s13 = torch.rand(e, h // group, 2 * inter, generator=g).to(torch.float16) * 0.02 + 0.002
    s2 = torch.rand(e, inter // group, h, generator=g).to(torch.float16) * 0.02 + 0.002
    pk = lambda v: torch.stack([awq_pack_reference(v[i]) for i in range(e)])
    b13, c13, y13 = convert.awq_to_wna16(pk(q13).to(DEV), pk(z13).to(DEV), s13.to(DEV))
    b2, c2, y2 = convert.awq_to_wna16(pk(q2).to(DEV), pk(z2).to(DEV), s2.to(DEV))
    x = torch.randn(t, h, generator=g).to(torch.bfloat16)
    ids, tw = _route(t, e, top_k, 9)
    out = moe.wna16_experts(None, x.to(DEV), b13, b2, c13, c2, tw.to(DEV), ids.to(DEV), group, z1=y13, z2=y2).cpu()
    deq = lambda q, z, sc: ((q.float() - z.float().repeat_interleave(group, 1))
                            * sc.to(torch.bfloat16).float().repeat_interleave(group, 1)).transpose(1, 2)
    ref = oracle.fused_moe(x, ids, tw, deq(q13, z13, s13), deq(q2, z2, s2))
    assert peak_rel_err(out, ref) <= TOL


def test_mxfp4_and_int8_experts():
    e, top_k, h, inter, t = 8, 2, 512, 256, 45
    g = _g(123)
    x = torch.randn(t, h, generator=g).to(torch.bfloat16)
    ids, tw = _route(t, e, top_k, 5)
    w13 = torch.randint(0, 256, (e, 2 * inter, h // 2), generator=g, dtype=torch.uint8)
    w2 = torch.randint(0, 256, (e, h, inter // 2), generator=g, dtype=torch.uint8)
    s13 = torch.randint(118, 126, (e, 2 * inter, h // 32), generator=g, dtype=torch.uint8)
    s2 = torch.randint(118, 126, (e, h, inter // 32), generator=g, dtype=torch.uint8)
    out = moe.mxfp4_experts(None, x.to(DEV), w13.to(DEV), w2.to(DEV), s13.to(DEV), s2.to(DEV), tw.to(DEV),
                            ids.to(DEV)).cpu()
    ref = oracle.fused_moe(x, ids, tw, lambda i: oracle.mxfp4_decode(w13[i], s13[i]),
                           lambda i: oracle.mxfp4_decode(w2[i], s2[i]))
    assert peak_rel_err(out, ref) <= TOL
    i13 = torch.randint(-127, 128, (e, 2 * inter, h), generator=g, dtype=torch.int8)
    i2 = torch.randint(-127, 128, (e, h, inter), generator=g, dtype=torch.int8)
    c13 = torch.rand(e, 2 * inter, generator=g) * 0.002 + 0.0005
    c2 = torch.rand(e, h, generator=g) * 0.002 + 0.0005
    out = moe.int8_experts(None, x.to(DEV), i13.to(DEV), i2.to(DEV), c13.to(DEV), c2.to(DEV), tw.to(DEV),
                           ids.to(DEV)).cpu()
    ref = oracle.fused_moe(x, ids, tw, i13.float() * c13[..., None], i2.float() * c2[..., None])
    assert peak_rel_err(out, ref) <= TOL
