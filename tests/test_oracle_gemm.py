# SPDX-License-Identifier: MIT
"""Pins the oracle's dense GEMM references (CPU only)."""

import numpy as np
import torch

import oracle
from libstrix_amd import workloads


def test_int32_accumulator_brute_force():
    g = torch.Generator().manual_seed(0)
    qa = torch.randint(-127, 128, (3, 256), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (5, 256), generator=g, dtype=torch.int8)
    acc = oracle.w8a8_int8_acc(qa, w)
    assert acc.dtype == np.int32
    for m in range(3):
        for n in range(5):
            assert acc[m, n] == sum(int(qa[m, k]) * int(w[n, k]) for k in range(256))


def test_int32_accumulator_extreme_fits():
    # 5120 * 127^2 = 82,580,480: the C1 worst case stays inside int32.
    qa = torch.full((1, 5120), 127, dtype=torch.int8)
    w = torch.full((1, 5120), -127, dtype=torch.int8)
    assert oracle.w8a8_int8_acc(qa, w)[0, 0] == -5120 * 127 * 127


def test_int8_gemm_equals_dequantized_matmul():
    d = workloads.c1_int8(seed=7, m=4, k=256, n=8)
    q, s = oracle.int8_quant_per_token(d["x"])
    out = oracle.w8a8_int8_gemm(q, s, d["w"], d["sw"])
    ref = (q.double() * s.double()[:, None]) @ (d["w"].double() * d["sw"].double()[:, None]).t()
    assert torch.allclose(out.double(), ref, rtol=1e-5, atol=1e-6)


def test_int8_group_gemm_equals_per_group_sum():
    g = torch.Generator().manual_seed(1)
    qa = torch.randint(-127, 128, (2, 256), generator=g, dtype=torch.int8)
    sa = torch.rand(2, 2, generator=g) + 0.1
    w = torch.randint(-127, 128, (3, 256), generator=g, dtype=torch.int8)
    sw = torch.rand(3, 2, generator=g) + 0.1
    out = oracle.w8a8_int8_group_gemm(qa, sa, w, sw)
    for m in range(2):
        for n in range(3):
            want = sum(
                float(sa[m, gi]) * float(sw[n, gi])
                * sum(int(qa[m, k]) * int(w[n, k]) for k in range(128 * gi, 128 * gi + 128))
                for gi in range(2)
            )
            assert abs(out[m, n].item() - want) <= 1e-4 * abs(want) + 1e-3


def test_fp8_block_dequant_elementwise_ragged_n():
    g = torch.Generator().manual_seed(2)
    n, k = 130, 256  # the second block row is partial
    w = (torch.randn(n, k, generator=g) * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
    bs = torch.rand(2, 2, generator=g) + 0.5
    d = oracle.fp8_block_dequant(w, bs)
    for i in (0, 1, 127, 128, 129):
        for j in (0, 127, 128, 255):
            assert d[i, j].item() == (w[i, j].float() * bs[i // 128, j // 128]).item()  # one fp32 rounding


def test_fp8_block_gemm_float64_block_order():
    g = torch.Generator().manual_seed(3)
    qd = workloads.c2_fp8(seed=3, m=5, n=200, k=384)
    qa, sa = oracle.fp8_quant_group128(qd["x"])
    out = oracle.fp8_block_gemm(qa, sa, qd["w"], qd["sw"])
    a = qa.float().double()
    w = qd["w"].float().double()
    ref = torch.zeros(5, 200, dtype=torch.float64)
    for kb in range(3):
        part = a[:, 128 * kb:128 * kb + 128] @ w[:, 128 * kb:128 * kb + 128].t()
        sw = qd["sw"][:, kb].double().repeat_interleave(128)[:200]
        ref += part * sa[:, kb].double()[:, None] * sw[None, :]
    assert torch.allclose(out.double(), ref, rtol=1e-5, atol=1e-5 * ref.abs().max().item())
    del g


def test_fp8_block_gemm_one_hot_reads_back_weights():
    qd = workloads.c2_fp8(seed=4, m=1, n=128, k=128)
    qa = torch.zeros(128, 128).to(torch.float8_e4m3fn)
    qa[range(128), range(128)] = 1.0
    sa = torch.ones(128, 1)
    out = oracle.fp8_block_gemm(qa, sa, qd["w"], qd["sw"])
    assert torch.equal(out.t(), oracle.fp8_block_dequant(qd["w"], qd["sw"]))


def test_fp8_block_weight_quantizer_roundtrip():
    g = torch.Generator().manual_seed(5)
    w = torch.randn(2, 256, 384, generator=g) * 0.02
    q, s = workloads.quantize_fp8_block(w)
    assert tuple(q.shape) == (2, 256, 384) and tuple(s.shape) == (2, 2, 3)
    deq = q.float() * s.repeat_interleave(128, 1).repeat_interleave(128, 2)
    # e4m3 keeps 3 mantissa bits: relative step 2^-3, so |err| <= 2^-4 |w| + subnormal floor
    assert ((deq - w).abs() <= w.abs() / 16 + s.amax() * 2.0**-10).all()
