# SPDX-License-Identifier: MIT
"""Dense GEMM references of the oracle (CPU). Test infrastructure only.

Each follows the reference's test pattern: dequantize the long way, then an
fp32 matmul (tests/test_fp8.py:17-21, 70-78; tests/test_w8a8_int8.py:50-57).
"""

from __future__ import annotations

import numpy as np
import torch

from oracle.quant import e4m3_decode


def w8a8_int8_acc(qa: torch.Tensor, w: torch.Tensor) -> np.ndarray:
    """Exact int32 accumulator sum_k qa[m,k] w[n,k] (int64 numpy matmul; the
    integer dot product is order-independent, so any correct kernel matches
    it bit for bit). Pinned by: tests/test_oracle_gemm.py (python-int brute
    force on tiny shapes)."""
    a = qa.detach().to("cpu").numpy().astype(np.int64)
    b = w.detach().to("cpu").numpy().astype(np.int64)
    acc = a @ b.T
    assert np.abs(acc).max(initial=0) < 2**31, "accumulator leaves int32"
    return acc.astype(np.int32)


def w8a8_int8_gemm(qa, sa, w, sw) -> torch.Tensor:
    """Per-token int8 x per-channel int8 -> fp32 (acc * sa[m]) * sw[n]
    (epilogue order matches the kernel so the fp32 values
    agree exactly). Pinned by: tests/test_oracle_gemm.py (against the fp32
    matmul of the dequantized operands)."""
    acc = torch.from_numpy(w8a8_int8_acc(qa, w)).float()
    return (acc * sa.detach().cpu().float()[:, None]) * sw.detach().cpu().float()[None, :]


def w8a8_int8_group_gemm(qa, sa, w_signed, sw_ng) -> torch.Tensor:
    """Per-(row,128-group) int8 activations x int8 weights with [N, G] (or
    [N, 1]) scales: sum_g (sum_{k in g} qa w) sa[m,g] sw[n,g]
    (csrc/gemm/w8a8_wmma_gemm.hip:15-32; tests/test_w8a8_int8.py:50-57
    dequantizes the same way). Pinned by: tests/test_oracle_gemm.py."""
    a = qa.detach().cpu().float()
    m, k = a.shape
    g = k // 128
    sa_f = sa.detach().cpu().float().reshape(m, g)
    sw_f = sw_ng.detach().cpu().float()
    sw_f = sw_f.reshape(sw_f.shape[0], -1).expand(-1, g) if sw_f.numel() == sw_f.shape[0] else sw_f
    a_deq = a * sa_f.repeat_interleave(128, dim=1)
    w_deq = w_signed.detach().cpu().float() * sw_f.repeat_interleave(128, dim=1)
    return a_deq @ w_deq.t()


def fp8_block_dequant(w_q: torch.Tensor, bs: torch.Tensor) -> torch.Tensor:
    """e4m3 [N, K] x fp32 128x128 block scales [ceil(N/128), K/128] -> fp32
    (tests/test_fp8.py:17-21 `ref_weight`). Pinned by:
    tests/test_oracle_gemm.py (per-element loop on a tiny ragged shape)."""
    n, k = w_q.shape
    s = bs.detach().cpu().float().repeat_interleave(128, 0)[:n].repeat_interleave(128, 1)[:, :k]
    return e4m3_decode(w_q) * s


def fp8_block_gemm(qa, sa, w_q, bs) -> torch.Tensor:
    """FP8-block W8A8: dequantize both operands, fp32 matmul (BASELINE config
    2; the activation half follows tests/test_fp8.py's dequant-then-matmul with
    the same 1x128 QDQ applied). Pinned by: tests/test_oracle_gemm.py
    (float64 sum over blocks in a different order; one-hot activations)."""
    m, k = qa.shape
    a = e4m3_decode(qa) * sa.detach().cpu().float().repeat_interleave(128, dim=1)[:, :k]
    return a @ fp8_block_dequant(w_q, bs).t()
