# SPDX-License-Identifier: MIT
"""W4A8 on the int8 MFMA (strix_w4a8_gemm, strix_moe_gemm_w4a8 and the
w4a8_wmma_gemm / moe_gemm_w4a8 ops over them).

The reference's W4A8 arithmetic (csrc/gemm/w8a8_wmma_gemm.hip:15-32,
csrc/moe/moe_gemm_w4a8.hip:1-40): an exact int32 sum per 128-K group of
int8 activations x (q - 8), folded in fp32 with the activation and weight
scales. Two bars:
  * per-group int32 sums bit-exact: through the C-ABI with fp16 output,
    activation scale 1 on one group and 0 on the others, unit weight scales
    and operands small enough that every sum is an fp16 integer, so the output
    is the group's sum itself, compared with the oracle's int64 matmul;
  * full-range values within 1e-2 of the output's peak against the oracle's
    fp32 fold (dequantize, then matmul), the reference tests' bar
    (tests/test_moe_w4a8.py:60-75, tests/test_w8a16.py:90-100).
"""

import numpy as np
import pytest
import torch

import libstrix_amd  # noqa: F401
import oracle
from conftest import peak_rel_err
from libstrix_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-2
S = torch.ops.strix


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def pack_low_first(q: torch.Tensor) -> torch.Tensor:
    """uint4 [.., N, K] -> uint8 [.., N, K/2], even k in the low nibble."""
    return (q[..., 0::2] | (q[..., 1::2] << 4)).to(torch.uint8).contiguous()


def _small_operands(m, n, k, seed):
    g = _g(seed)
    qa = torch.randint(-2, 3, (m, k), generator=g, dtype=torch.int8)
    q = torch.randint(0, 16, (n, k), generator=g, dtype=torch.uint8)
    return qa, q


def _group_sums(qa, q, grp):
    sl = slice(128 * grp, 128 * (grp + 1))
    return oracle.w8a8_int8_acc(qa[:, sl], (q[:, sl].to(torch.int16) - 8).to(torch.int8))


@pytest.mark.parametrize("order", [1, 2])
@pytest.mark.parametrize("m,n,k", [(16, 256, 512), (300, 384, 384)])
def test_dense_group_sums_bit_exact(order, m, n, k):
    qa, q = _small_operands(m, n, k, 5 * m + order)
    w = pack_low_first(q) if order == 1 else oracle.wna16_ex_pack(q).view(torch.uint8)
    sw = torch.ones(n, dtype=torch.float32, device=DEV)
    qa_d, w_d = qa.to(DEV), w.to(DEV)
    out = torch.empty(m, n, dtype=torch.float16, device=DEV)
    for grp in range(k // 128):
        sa = torch.zeros(m, k // 128, dtype=torch.float32)
        sa[:, grp] = 1.0
        sa_d = sa.to(DEV)
        out.fill_(float("nan"))
        _lib.call("strix_w4a8_gemm", _ptr(qa_d), k, _ptr(sa_d), k // 128, _ptr(w_d), k // 2, order, _ptr(sw), 1, 0,
                  _ptr(out), n, _lib.F16, m, n, k, _stream())
        torch.cuda.synchronize()
        want = _group_sums(qa, q, grp)
        assert np.abs(want).max() <= 2048  # every sum is an fp16 integer
        got = out.cpu().float().numpy()
        assert np.array_equal(got, want.astype(np.float32)), f"group {grp}"


@pytest.mark.parametrize("block_m", [64, 128, 256])
def test_moe_group_sums_bit_exact(block_m):
    e, t, top_k, n, k = 4, 150, 2, 512, 384
    g = _g(block_m)
    qa = torch.randint(-2, 3, (t, k), generator=g, dtype=torch.int8)
    q = torch.randint(0, 16, (e, n, k), generator=g, dtype=torch.uint8)
    ids = torch.stack([torch.randperm(e, generator=g)[:top_k] for _ in range(t)]).to(torch.int32)
    w_d = pack_low_first(q).to(DEV)
    sw = torch.ones(e, n, k // 128, dtype=torch.float32, device=DEV)
    sorted_ids, expert_ids, num_post = S.moe_align(ids.to(DEV), e, block_m)
    qa_d = qa.to(DEV)
    c = torch.empty(t * top_k, n, dtype=torch.float16, device=DEV)
    for grp in range(k // 128):
        sa = torch.zeros(t, k // 128, dtype=torch.float32)
        sa[:, grp] = 1.0
        sa_d = sa.to(DEV)
        c.fill_(float("nan"))
        _lib.call("strix_moe_gemm_w4a8", _ptr(c), n, _lib.F16, _ptr(qa_d), k, _ptr(sa_d), k // 128, _ptr(w_d),
                  n * k // 2, k // 2, _ptr(sw), sw.stride(0), sw.stride(1), _ptr(sorted_ids), sorted_ids.numel(),
                  _ptr(expert_ids), expert_ids.numel(), _ptr(num_post), None, t * top_k, top_k, block_m, 0,
                  _lib.ACT_SILU, n, k, _stream())
        torch.cuda.synchronize()
        got = c.cpu().float().reshape(t, top_k, n)
        for ex in range(e):
            rows, slots = (ids == ex).nonzero(as_tuple=True)
            if rows.numel() == 0:
                continue
            want = _group_sums(qa[rows], q[ex], grp)
            assert np.array_equal(got[rows, slots].numpy(), want.astype(np.float32)), f"expert {ex} group {grp}"


# ------------------------------------------------------------------ full range, fp32 fold
def _dense_case(m, n, k, layout, seed):
    g = _g(seed)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    q = torch.randint(0, 16, (n, k), generator=g, dtype=torch.uint8)
    if layout == "channel":
        s = torch.rand(n, 1, generator=g) * 0.05 + 0.01
        sf = s.reshape(n)
    else:
        s = torch.rand(n, k // 128, generator=g) * 0.05 + 0.01
        sf = s.t().contiguous() if layout == "gn" else s
    return x, q, s, sf


@pytest.mark.parametrize("layout", ["channel", "gn", "ng"])
@pytest.mark.parametrize("m,n,k", [(1, 256, 1024), (77, 2048, 2560), (1000, 1536, 2048)])
def test_w4a8_wmma_gemm_int8_mfma(layout, m, n, k):
    x, q, s, sf = _dense_case(m, n, k, layout, m + n)
    w = oracle.wna16_ex_pack(q)
    out = S.w4a8_wmma_gemm(w.to(DEV), x.to(DEV), sf.to(DEV)).cpu()
    qa, sa = oracle.int8_quant_group128(x)
    sw_ng = s if layout != "channel" else s.reshape(n, 1)
    ref = oracle.w8a8_int8_group_gemm(qa, sa, q.to(torch.int16) - 8, sw_ng)
    assert out.dtype == torch.bfloat16 and out.shape == (m, n)
    assert peak_rel_err(out, ref) <= TOL


def _moe_case(e, t, top_k, n, k, seed, scale_dtype=torch.bfloat16):
    g = _g(seed)
    q = torch.randint(0, 16, (e, n, k), generator=g, dtype=torch.uint8)
    scales = (torch.rand(e, n, k // 128, generator=g) * 0.02 + 0.001).to(scale_dtype)
    x = torch.randn(t, k, generator=g).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(e, generator=g)[:top_k] for _ in range(t)]).to(torch.int32)
    weights = torch.rand(t, top_k, generator=g)
    return q, scales, x, ids, weights


def _quant(a):
    qa = torch.empty(a.shape, dtype=torch.int8, device=DEV)
    sa = torch.empty(a.size(0), a.size(1) // 128, dtype=torch.float32, device=DEV)
    S.moe_act_quant_i8(a.to(DEV), qa, sa)
    return qa, sa


@pytest.mark.parametrize("block_m,block_n", [(64, 128), (64, 256), (128, 128), (256, 256)])
@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float16])
def test_moe_gemm_w4a8_w2_weighted(block_m, block_n, scale_dtype):
    """The w2 stage: one input row per routed slot (top_k 1 in the call),
    each output row times its slot's top-k weight."""
    e, top_k, t, n, k = 8, 4, 203, 512, 768
    q, scales, _, ids, weights = _moe_case(e, t, top_k, n, k, block_m + block_n, scale_dtype)
    a = torch.randn(t * top_k, k, generator=_g(block_n)).to(torch.bfloat16)
    qa, sa = _quant(a)
    sorted_ids, expert_ids, num_post = S.moe_align(ids.to(DEV), e, block_m)
    c = torch.full((t * top_k, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    S.moe_gemm_w4a8(c, qa, sa, pack_low_first(q).to(DEV), scales.to(DEV), sorted_ids, expert_ids, num_post,
                    weights.reshape(-1).to(DEV), 1, block_m, block_n, False, "silu")
    a_deq = qa.cpu().float() * sa.cpu().repeat_interleave(128, dim=1)
    b = oracle.wna16_sym_decode(pack_low_first(q), scales, 128)
    ref = oracle.moe_expert_gemm(a_deq, b, ids, 1, weights)
    assert not torch.isnan(c).any()
    assert peak_rel_err(c.cpu(), ref) <= TOL


@pytest.mark.parametrize("activation", ["silu", "gelu_tanh"])
@pytest.mark.parametrize("block_m,block_n", [(64, 128), (128, 128), (256, 256)])
def test_moe_gemm_w4a8_w13_gated(activation, block_m, block_n):
    e, top_k, t, n, k = 8, 2, 150, 512, 640
    q, scales, x, ids, _ = _moe_case(e, t, top_k, n, k, 17 + block_m)
    qa, sa = _quant(x)
    sorted_ids, expert_ids, num_post = S.moe_align(ids.to(DEV), e, block_m)
    c = torch.full((t * top_k, n // 2), float("nan"), dtype=torch.bfloat16, device=DEV)
    S.moe_gemm_w4a8(c, qa, sa, pack_low_first(q).to(DEV), scales.to(DEV), sorted_ids, expert_ids, num_post,
                    None, top_k, block_m, block_n, True, activation)
    a_deq = qa.cpu().float() * sa.cpu().repeat_interleave(128, dim=1)
    b = oracle.wna16_sym_decode(pack_low_first(q), scales, 128)
    y = oracle.moe_expert_gemm(a_deq, b, ids, top_k)  # [t*top_k, n]
    gate, up = y[:, : n // 2], y[:, n // 2:]
    act = torch.nn.functional.silu(gate) if activation == "silu" else torch.nn.functional.gelu(gate, approximate="tanh")
    ref = act * up
    assert not torch.isnan(c).any()
    assert peak_rel_err(c.cpu(), ref) <= TOL


def test_moe_gemm_w4a8_c5_shapes():
    """The C5 expert shapes (E 128, top-8, hidden 2048, intermediate 768),
    w13 gated then w2 weighted, at 256 tokens."""
    e, top_k, t, h, inter = 128, 8, 256, 2048, 768
    g = _g(55)
    q13 = torch.randint(0, 16, (e, 2 * inter, h), generator=g, dtype=torch.uint8)
    s13 = (torch.rand(e, 2 * inter, h // 128, generator=g) * 0.02 + 0.001).to(torch.bfloat16)
    q2 = torch.randint(0, 16, (e, h, inter), generator=g, dtype=torch.uint8)
    s2 = (torch.rand(e, h, inter // 128, generator=g) * 0.02 + 0.001).to(torch.bfloat16)
    x = torch.randn(t, h, generator=g).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(e, generator=g)[:top_k] for _ in range(t)]).to(torch.int32)
    weights = torch.rand(t, top_k, generator=g)
    qx, sx = _quant(x)
    sorted_ids, expert_ids, num_post = S.moe_align(ids.to(DEV), e, 64)
    c13 = torch.empty((t * top_k, inter), dtype=torch.bfloat16, device=DEV)
    S.moe_gemm_w4a8(c13, qx, sx, pack_low_first(q13).to(DEV), s13.to(DEV), sorted_ids, expert_ids, num_post, None,
                    top_k, 64, 128, True, "silu")
    qi, si = _quant(c13)
    c2 = torch.empty((t * top_k, h), dtype=torch.bfloat16, device=DEV)
    S.moe_gemm_w4a8(c2, qi, si, pack_low_first(q2).to(DEV), s2.to(DEV), sorted_ids, expert_ids, num_post,
                    weights.reshape(-1).to(DEV), 1, 64, 128, False, "silu")
    # Oracle per stage, from the kernel's own int8 inputs.
    b13 = oracle.wna16_sym_decode(pack_low_first(q13), s13, 128)
    y = oracle.moe_expert_gemm(qx.cpu().float() * sx.cpu().repeat_interleave(128, 1), b13, ids, top_k)
    ref13 = torch.nn.functional.silu(y[:, :inter]) * y[:, inter:]
    assert peak_rel_err(c13.cpu(), ref13) <= TOL
    b2 = oracle.wna16_sym_decode(pack_low_first(q2), s2, 128)
    ref2 = oracle.moe_expert_gemm(qi.cpu().float() * si.cpu().repeat_interleave(128, 1), b2, ids, 1, weights)
    assert peak_rel_err(c2.cpu(), ref2) <= TOL


def test_moe_gemm_w4a8_rejects_unsupported_tiles():
    e, n, k = 2, 256, 256
    qa = torch.zeros(4, k, dtype=torch.int8, device=DEV)
    sa = torch.ones(4, k // 128, dtype=torch.float32, device=DEV)
    w = torch.zeros(e, n, k // 2, dtype=torch.uint8, device=DEV)
    s = torch.ones(e, n, k // 128, dtype=torch.bfloat16, device=DEV)
    ids = torch.zeros(4, 1, dtype=torch.int32, device=DEV)
    sorted_ids, expert_ids, num_post = S.moe_align(ids, e, 64)
    c = torch.empty(4, n, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="unsupported block_m/block_n"):
        S.moe_gemm_w4a8(c, qa, sa, w, s, sorted_ids, expert_ids, num_post, None, 1, 128, 256, False, "silu")


def test_moe_gemm_w4a8_empty_sorted_ids_writes_nothing():
    """sorted_ids empty (no routed positions): the call returns before any
    kernel and leaves the output as it was."""
    e, top_k, t, n, k = 8, 4, 3, 256, 256
    q, scales, _, ids, weights = _moe_case(e, t, top_k, n, k, 5, torch.bfloat16)
    a = torch.randn(t * top_k, k, generator=_g(5)).to(torch.bfloat16)
    qa, sa = _quant(a)
    c = torch.full((t * top_k, n), 7.0, dtype=torch.bfloat16, device=DEV)
    sorted_ids = torch.empty(0, dtype=torch.int32, device=DEV)
    expert_ids = torch.zeros(1, dtype=torch.int32, device=DEV)
    num_post = torch.zeros(1, dtype=torch.int32, device=DEV)
    for block_m, block_n in ((64, 128), (256, 256)):
        S.moe_gemm_w4a8(c, qa, sa, pack_low_first(q).to(DEV), scales.to(DEV), sorted_ids, expert_ids, num_post,
                        weights.reshape(-1).to(DEV), 1, block_m, block_n, False, "silu")
    torch.cuda.synchronize()
    assert bool((c == 7.0).all())
